"""Pin the CPU oracle's codec against the reference's own known-answer tests,
library routines (torch casts / topk / complex multiply) and closed forms.

Each test names what it pins; a plausible slip in the oracle (dropped term,
wrong sign or index, transposed operand, wrong tie or rounding rule) fails one.
"""

import math

import numpy as np
import pytest
import torch

import oracle

ONES = np.ones(512, np.float32)


def all_bf16_magnitudes(limit=None):
    bits = np.arange(0, 0x7F80, dtype=np.uint32) << 16  # every finite positive bf16
    vals = bits.view(np.float32)
    return vals if limit is None else vals[vals <= limit]


# ---- scalar pieces -----------------------------------------------------------

def test_e4m3_encode_matches_torch_cast_exhaustively_over_bf16():
    """E4M3 RNE == torch float8_e4m3fn cast for every bf16 value |q| <= 448
    (every value the packer quantises is a bf16 value times 2^-e)."""
    mags = all_bf16_magnitudes(448.0)
    vals = np.concatenate([mags, -mags])
    expect = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.e4m3_encode(v) for v in vals], np.uint8)
    bad = np.nonzero(got != expect)[0]
    assert bad.size == 0, (vals[bad[:5]], got[bad[:5]], expect[bad[:5]])


def test_e4m3_encode_matches_torch_on_random_fp32_ties():
    rng = np.random.default_rng(1)
    # midpoints between adjacent e4m3 values hit the ties-to-even branch
    codes = np.arange(0, 0x7E, dtype=np.uint8)
    lo = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    hi = torch.from_numpy(codes + 1).view(torch.float8_e4m3fn).float().numpy()
    vals = np.concatenate([(lo + hi) / 2, rng.uniform(0, 448, 5000).astype(np.float32),
                           rng.uniform(0, 2**-6, 2000).astype(np.float32)]).astype(np.float32)
    expect = torch.from_numpy(vals).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([oracle.e4m3_encode(v) for v in vals], np.uint8)
    assert np.array_equal(got, expect)


def test_e4m3_decode_matches_torch_for_every_code():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    expect = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([oracle.e4m3_decode(c) for c in codes], np.float32)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32))


def test_ue8m0_exponent_is_ceil_log2_exhaustively():
    """Integer UE8M0 rule == ceil(log2(max(a, 1e-4) / 448)) in float64 for every
    finite bf16 magnitude (test_integration.py:1603 formula)."""
    for a in all_bf16_magnitudes():
        expect = math.ceil(math.log2(max(float(a), 1e-4) / 448))
        assert oracle.ue8m0_exponent(a) == expect, a


def test_ue8m0_zero_group_is_byte_105():
    assert oracle.ue8m0_exponent(0.0) + 127 == 105


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(2)
    base = rng.standard_normal(20000).astype(np.float32) * 10
    u = base.view(np.uint32)
    ties = ((u & 0xFFFF0000) | 0x8000).view(np.float32)  # exact halfway cases
    vals = np.concatenate([base, ties, np.array([0.0, -0.0, 1e-40, -3e38], np.float32)])
    expect = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.f32_to_bf16_np(vals), expect)
    assert np.array_equal(oracle.bf16_bits(vals[:500]), expect[:500])


# ---- selection ------------------------------------------------------------------

def torch_rule(x: np.ndarray) -> np.ndarray:
    """evaluate.py:65-91: prune topk(|x|, 256, largest=False)."""
    t = torch.from_numpy(x)
    mask = torch.ones_like(t, dtype=torch.bool)
    mask.scatter_(-1, t.abs().topk(256, dim=-1, largest=False).indices, False)
    return mask.numpy()


def test_selection_matches_reference_tie_rows():
    """The three rows the reference asserts against topmag_keep_mask
    (test_integration.py:1527-1548): arange, -arange, zeros."""
    raw = np.stack([np.arange(512, dtype=np.float32), -np.arange(512, dtype=np.float32),
                    np.zeros(512, np.float32)])
    assert np.array_equal(oracle.select_keep(raw), torch_rule(raw))
    assert np.array_equal(oracle.select_keep(raw)[2], np.arange(512) < 256)


def test_selection_matches_torch_topk_on_untied_rows():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((220, 512)).astype(np.float32)
    x = x[[len(np.unique(np.abs(r))) == 512 for r in x]]
    assert len(x) > 150
    assert np.array_equal(oracle.select_keep(x), torch_rule(x))


def test_selection_is_rank_rule_by_brute_force():
    """keep[c] iff #{|x_j| > |x_c|} + #{j < c : |x_j| == |x_c|} < 256, on rows
    with heavy ties (small integer magnitudes, signed zeros)."""
    rng = np.random.default_rng(4)
    x = rng.integers(-6, 7, (40, 512)).astype(np.float32)
    x[x == 0] = np.where(rng.random((x == 0).sum()) < 0.5, 0.0, -0.0)
    keep = oracle.select_keep(x)
    a = np.abs(x)
    for r in range(x.shape[0]):
        gt = (a[r][None, :] > a[r][:, None]).sum(1)
        eq_before = np.array([(a[r][:c] == a[r][c]).sum() for c in range(512)])
        assert np.array_equal(keep[r], gt + eq_before < 256)
    assert (keep.sum(1) == 256).all()


# ---- RMSNorm ----------------------------------------------------------------

def test_masked_rmsnorm_agrees_with_torch_formula():
    """losses.py:84-89 computed by torch: the oracle's fixed reduction order may
    move a result by one bf16 ulp at a rounding boundary, nothing more."""
    x = oracle.synthetic_latents(512, seed=5)
    keep = oracle.select_keep(x)
    w = np.linspace(0.5, 1.5, 512).astype(np.float32)
    got = oracle.normalize(x, keep, w, 1e-6)
    m = torch.from_numpy(x).masked_fill(~torch.from_numpy(keep), 0)
    ref = (m * torch.rsqrt(m.square().mean(-1, keepdim=True) + 1e-6) * torch.from_numpy(w))
    ref = ref.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1
    assert (diff == 0).mean() > 0.999


def test_rmsnorm_constant_rows_closed_form():
    """Constant survivors: r = 1/sqrt(kept/512 + eps) exactly as Python floats."""
    for kept in (64, 192, 256, 448):
        x = np.zeros(512, np.float32)
        x[:kept] = 1.0
        keep = x != 0
        n = oracle.bf16_to_f32(oracle.normalize(x[None], keep[None], ONES, 1e-6))[0]
        expect = float(torch.tensor(1.0 / math.sqrt(kept / 512 + 1e-6)).bfloat16())
        assert np.all(n[:kept] == np.float32(expect)) and np.all(n[kept:] == 0)


# ---- closed-form codec KATs ----------------------------------------------------

def rotate_torch(rows_bf16_bits: np.ndarray, freqs_c: torch.Tensor) -> np.ndarray:
    """Independent tail rotation: torch complex multiply on the bf16 tail
    (candidate-sglang.patch:850-859), result rounded to bf16."""
    rows = torch.from_numpy(oracle.bf16_to_f32(rows_bf16_bits).copy())
    tail = torch.view_as_complex(rows[:, 448:].reshape(-1, 32, 2).contiguous()) * freqs_c
    rows[:, 448:] = torch.view_as_real(tail).reshape(-1, 64)
    return rows.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def test_reference_closed_form_tile_kat_192_survivors():
    """test_integration.py:1588-1619: raw ones, weight 2^tile per 64-group,
    survivors arange % 8 >= 5, expected built from Python scalars."""
    eps = 1e-6
    raw = np.ones((512, 512), np.float32)
    weight = np.repeat(np.array([2.0**t for t in range(8)], np.float32), 64)
    mask = np.broadcast_to(np.arange(512) % 8 >= 5, (512, 512))
    expected = np.zeros((512, 512), np.float32)
    for tile in range(8):
        normalized = float(torch.tensor((2.0**tile) / math.sqrt(192 / 512 + eps)).bfloat16())
        scale = 2.0 ** math.ceil(math.log2(max(abs(normalized), 1e-4) / 448))
        code = torch.tensor(normalized / scale).to(torch.float8_e4m3fn).float()
        expected[:, tile * 64:(tile + 1) * 64] = float((code * scale).bfloat16())
    expected[~mask] = 0
    got = oracle.bf16_to_f32(oracle.simulate_rows(raw, mask, weight, eps))
    assert np.array_equal(got, expected)
    g = torch.Generator().manual_seed(42)
    freqs = torch.polar(torch.ones(512, 32), torch.randn(512, 32, generator=g))
    f = torch.view_as_real(freqs).numpy()
    exp_bits = oracle.f32_to_bf16_np(expected)
    rot = oracle.rope_tail(exp_bits, f)
    ref = rotate_torch(exp_bits, freqs)
    assert np.abs(rot.astype(np.int32) - ref.astype(np.int32)).max() <= 1


def test_packed_record_closed_form_256_survivors():
    """256-survivor restatement of the tile KAT through the real packer:
    odd coordinates hold 1.0, weight 2^tile. Every byte follows from the math."""
    eps = 1e-6
    x = (np.arange(512) % 2).astype(np.float32)
    weight = np.repeat(np.array([2.0**t for t in range(8)], np.float32), 64)
    data, scales, normed, keep = oracle.pack_rows(x[None], weight, eps)
    assert np.array_equal(keep[0], np.arange(512) % 2 == 1)
    bitmap = data[0, 256:].view("<u8")
    assert np.all(bitmap == 0x5555555555555555)  # MSB-first: coord 1 -> bit 62
    for tile in range(8):
        n = float(torch.tensor((2.0**tile) / math.sqrt(256 / 512 + eps)).bfloat16())
        e = math.ceil(math.log2(n / 448))
        assert scales[0, tile] == e + 127
        code = int(torch.tensor(n / 2.0**e).to(torch.float8_e4m3fn).view(torch.uint8))
        assert np.all(data[0, tile * 32:(tile + 1) * 32] == code)
    dec = oracle.bf16_to_f32(oracle.unpack_row(data[0], scales[0]))
    assert np.all(dec[::2] == 0)


def test_pack_unpack_roundtrip_is_exact_dequantisation():
    """a4: unpack(pack(x)) == the dense simulation of the same mask, and every
    survivor is within E4M3 precision of the normalised value."""
    x = oracle.synthetic_latents(256, seed=6)
    data, scales, normed, keep = oracle.pack_rows(x, ONES, 1e-6)
    dec = oracle.unpack_rows(data, scales)
    assert np.array_equal(dec, oracle.simulate_rows(x, keep, ONES, 1e-6))
    d, n = oracle.bf16_to_f32(dec), oracle.bf16_to_f32(normed)
    sb = np.repeat(scales.astype(np.int32) - 127, 64, axis=1)
    tol = np.maximum(np.abs(n) * 2.0**-4, 2.0 ** (sb - 10).astype(np.float64))
    assert np.all(np.abs(d - n)[keep] <= tol[keep])
    assert np.all(d[~keep] == 0)
    assert all(bin(int(w)).count("1") for w in data[:, 256:].view("<u8").ravel())
    pop = np.unpackbits(data[:, 256:], axis=1).sum(1)
    assert np.all(pop == 256)


def test_native_record_layout_fixture():
    """test_integration.py:361-367: codes e4m3(1), tail bf16(1), scales 127 decode to ones."""
    data = np.zeros(576, np.uint8)
    data[:448] = torch.ones(448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    data[448:] = torch.ones(64).to(torch.bfloat16).view(torch.uint8).numpy()
    scales = np.full(8, 127, np.uint8)
    assert np.all(oracle.bf16_to_f32(oracle.native_unpack_row(data, scales)) == 1.0)


def test_native_pack_constant_row():
    x = np.full(512, 3.0, np.float32)
    data, scales = oracle.native_pack_row(x, ONES, 1e-6)
    one = float(torch.tensor(1.0 / math.sqrt(1.0 + 1e-6)).bfloat16())
    e = math.ceil(math.log2(one / 448))
    assert np.all(scales[:7] == e + 127) and scales[7] == 0
    code = int(torch.tensor(one / 2.0**e).to(torch.float8_e4m3fn).view(torch.uint8))
    assert np.all(data[:448] == code)
    assert np.all(data[448:].view(np.uint16) == oracle.f32_to_bf16_np(np.float32(one)))


# ---- RoPE ---------------------------------------------------------------------

def test_rope_tail_matches_torch_complex_multiply():
    rng = np.random.default_rng(7)
    rows = oracle.f32_to_bf16_np(rng.standard_normal((300, 512)).astype(np.float32))
    ang = torch.from_numpy(rng.uniform(-50, 50, (300, 32)).astype(np.float32))
    freqs = torch.polar(torch.ones_like(ang), ang)
    got = oracle.rope_tail(rows, torch.view_as_real(freqs).numpy())
    ref = rotate_torch(rows, freqs)
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99
    assert np.array_equal(got[:, :448], rows[:, :448])


def test_rotation_reaches_pruned_partner_lanes():
    """candidate-sglang.patch:708-736: a retained lane feeds its pruned partner."""
    latent = np.zeros((2, 512), np.float32)
    latent[:, :254] = 2
    latent[:, 448] = 3
    latent[:, 451] = -3
    keep = oracle.select_keep(latent)
    assert np.array_equal(keep, latent != 0)
    pool = np.zeros((1, oracle.PAGE_BYTES), np.uint8)
    oracle.pack_rows_paged(latent, ONES, 1e-6, np.array([0, 1], np.int32), pool)
    angles = torch.linspace(0.2, 1.1, 16 * 32).reshape(16, 32)
    freqs = torch.polar(torch.ones_like(angles), angles)
    out = oracle.unpack_gather(pool, np.array([[1, 1]]), np.array([[0, 2]]),
                               np.array([2]), torch.view_as_real(freqs).numpy())
    dec = oracle.unpack_gather(pool, np.array([[1, 1]]), None, np.array([2]))
    expected = rotate_torch(dec, freqs[[0, 8]])
    assert np.all(oracle.bf16_to_f32(expected[:, [449, 450]]) != 0)
    assert np.abs(out.astype(np.int32) - expected.astype(np.int32)).max() <= 1


def test_unpack_gather_validity_rules():
    """Zero rows for k >= length, negative/out-of-pool physical, raw*4 beyond the
    table; rows follow the changing-input fixture's index pattern
    (candidate-sglang.patch:775-865)."""
    src = oracle.synthetic_latents(4, seed=8)
    pool = np.zeros((2, oracle.PAGE_BYTES), np.uint8)
    oracle.pack_rows_paged(src, ONES, 1e-6, np.array([0, 2, 3, 64], np.int32), pool)
    physical = np.array([[0, 2, -1, 3], [3, 128, 64, 0]], np.int32)
    raw = np.array([[0, 2, 1, 3], [2, 0, 1, 8]], np.int32)
    lengths = np.array([4, 3], np.int32)
    angles = torch.arange(32 * 32).float().reshape(32, 32) * 0.0037
    freqs = torch.view_as_real(torch.polar(torch.ones_like(angles), angles)).numpy()
    out = oracle.unpack_gather(pool, physical, raw, lengths, freqs)
    plain = oracle.unpack_gather(pool, physical, None, lengths)
    for row in range(8):
        q, k = divmod(row, 4)
        p, r = physical[q, k], raw[q, k]
        valid = k < lengths[q] and 0 <= p < 128 and 0 <= r * 4 < 32
        if not valid:
            assert np.all(out[row] == 0)
        else:
            assert np.array_equal(out[row, :448], plain[row, :448])
            ref = oracle.rope_tail(plain[row], freqs[r * 4])
            assert np.array_equal(out[row], ref[0])
    zero_rows = [row for row in range(8) if not out[row].any()]
    assert zero_rows == [2, 5, 7]


# ---- survivor profiles 64..448 (count + 72 byte records) -----------------------

def ranking_rule(x: np.ndarray, retained: int) -> np.ndarray:
    """evaluate.py:65-91 with one 512-group: prune topk(|x|, 512 - retained,
    largest=False); budgets RETENTION_COUNTS = 64..448 (losses.py:17)."""
    t = torch.from_numpy(x).abs()
    mask = torch.ones_like(t, dtype=torch.bool)
    mask.scatter_(-1, t.topk(512 - retained, dim=-1, largest=False).indices, False)
    return mask.numpy()


@pytest.mark.parametrize("keep_count", oracle.KEEP_COUNTS)
def test_selection_any_survivor_count(keep_count):
    """Untied rows agree with the reference's ranking rule; tied rows follow the
    rank rule (#{greater} + #{equal, lower coordinate} < K) by brute force."""
    rng = np.random.default_rng(30 + keep_count)
    x = rng.standard_normal((48, 512)).astype(np.float32)
    x = x[[len(np.unique(np.abs(r))) == 512 for r in x]]
    assert len(x) > 20
    assert np.array_equal(oracle.select_keep(x, keep_count), ranking_rule(x, keep_count))
    t = rng.integers(-6, 7, (6, 512)).astype(np.float32)
    keep = oracle.select_keep(t, keep_count)
    a = np.abs(t)
    bigger = (a[:, None, :] > a[:, :, None]).sum(2)          # [row, c]: #{j : |x_j| > |x_c|}
    lower = np.arange(512)[None, :] < np.arange(512)[:, None]  # [c, j]: j < c
    tied_before = ((a[:, None, :] == a[:, :, None]) & lower).sum(2)
    assert np.array_equal(keep, bigger + tied_before < keep_count)
    assert (keep.sum(1) == keep_count).all()


@pytest.mark.parametrize("keep_count", oracle.KEEP_COUNTS)
def test_packed_record_closed_form_any_survivor_count(keep_count):
    """K survivors at coordinates c % 8 < K / 64, weight 2^tile: every byte of
    the (K + 72)-byte record follows from the math (codes K/8 per group, bitmap
    bytes with their top K/64 bits set, scale ceil(log2(n / 448)) + 127)."""
    eps, per = 1e-6, keep_count // 64
    x = (np.arange(512) % 8 < per).astype(np.float32)
    weight = np.repeat(np.array([2.0**t for t in range(8)], np.float32), 64)
    data, scales, normed, keep = oracle.pack_rows(x[None], weight, eps, keep_count)
    assert data.shape == (1, keep_count + 64)
    assert np.array_equal(keep[0], x != 0)
    assert np.all(data[0, keep_count:] == (0xFF << (8 - per)) & 0xFF)
    for tile in range(8):
        n = float(torch.tensor((2.0**tile) / math.sqrt(keep_count / 512 + eps)).bfloat16())
        e = math.ceil(math.log2(n / 448))
        assert scales[0, tile] == e + 127
        code = int(torch.tensor(n / 2.0**e).to(torch.float8_e4m3fn).view(torch.uint8))
        assert np.all(data[0, tile * 8 * per:(tile + 1) * 8 * per] == code)
    dec = oracle.bf16_to_f32(oracle.unpack_row(data[0], scales[0], keep_count))
    assert np.all(dec[x == 0] == 0) and np.all(dec[x != 0] > 0)


@pytest.mark.parametrize("keep_count", [64, 192, 448])
def test_pack_unpack_roundtrip_any_survivor_count(keep_count):
    """unpack(pack(x)) equals the dense simulation of the same mask; the paged
    pool of (K + 72)-byte records holds the same bytes as the row packer."""
    x = oracle.synthetic_latents(96, seed=7 + keep_count)
    data, scales, normed, keep = oracle.pack_rows(x, ONES, 1e-6, keep_count)
    dec = oracle.unpack_rows(data, scales, keep_count)
    assert np.array_equal(dec, oracle.simulate_rows(x, keep, ONES, 1e-6))
    assert np.all(np.unpackbits(data[:, keep_count:], axis=1).sum(1) == keep_count)
    slots = np.random.default_rng(9).permutation(128)[:96].astype(np.int32)
    pool = np.zeros((2, oracle.page_bytes(keep_count)), np.uint8)
    oracle.pack_rows_paged(x, ONES, 1e-6, slots, pool, keep_count)
    recs = pool.reshape(128, oracle.record_bytes(keep_count))
    assert np.array_equal(recs[slots], np.concatenate([data, scales], axis=1))
    lengths = np.array([96], np.int32)
    got = oracle.unpack_gather(pool, slots[None], None, lengths, keep_count=keep_count)
    assert np.array_equal(got, dec)


@pytest.mark.parametrize("keep_count", [192, 448])
def test_rotation_reaches_pruned_partner_lanes_any_survivor_count(keep_count):
    """candidate-sglang.patch:707-736 (parametrized over 192 and 256 there):
    survivors 0..K-3 plus 448 and 451; the rotation fills pruned 449 and 450."""
    latent = np.zeros((2, 512), np.float32)
    latent[:, : keep_count - 2] = 2
    latent[:, 448] = 3
    latent[:, 451] = -3
    keep = oracle.select_keep(latent, keep_count)
    assert np.array_equal(keep, latent != 0)
    pool = np.zeros((1, oracle.page_bytes(keep_count)), np.uint8)
    oracle.pack_rows_paged(latent, ONES, 1e-6, np.array([0, 1], np.int32), pool, keep_count)
    angles = torch.linspace(0.2, 1.1, 16 * 32).reshape(16, 32)
    freqs = torch.polar(torch.ones_like(angles), angles)
    out = oracle.unpack_gather(pool, np.array([[1, 1]]), np.array([[0, 2]]), np.array([2]),
                               torch.view_as_real(freqs).numpy(), keep_count=keep_count)
    dec = oracle.unpack_gather(pool, np.array([[1, 1]]), None, np.array([2]),
                               keep_count=keep_count)
    expected = rotate_torch(dec, freqs[[0, 8]])
    assert np.all(oracle.bf16_to_f32(expected[:, [449, 450]]) != 0)
    assert np.abs(out.astype(np.int32) - expected.astype(np.int32)).max() <= 1


def test_survivor_count_outside_profiles_is_rejected():
    """512 survivors (and non-multiples of 64) are not profiles
    (docs/agents/numerical-and-validation.md:11-13)."""
    for bad in (0, 32, 200, 512):
        with pytest.raises(ValueError):
            oracle.select_keep(np.zeros((1, 512), np.float32), bad)


# ---- Adapter: Packed -> Native workspace ------------------------------------------

def test_adapter_is_lossless_and_encodes_invalid_rows_as_zero_rows():
    """Re-encoding a dequantized Packed row as a Native record loses nothing:
    each group's values are E4M3 codes times 2^e, so the Native scale is 2^e or
    2^(e-1) and every code re-encodes exactly. Decoding the Adapter's records
    gives back unpack_gather_bf16's rows bit for bit (tail included); invalid
    selections are the Native encoding of a zero row (codes 0, scale bytes 105)."""
    src = oracle.synthetic_latents(128, seed=14)
    src[5] = 0.0
    src[6, :8] = 1e-3  # tiny group maxima: the 1e-4 floor and subnormal codes
    src[6, 8:] = 0.0
    pool = np.zeros((2, oracle.PAGE_BYTES), np.uint8)
    oracle.pack_rows_paged(src, np.linspace(0.5, 1.5, 512).astype(np.float32), 1e-6,
                           np.arange(128, dtype=np.int32), pool)
    rng = np.random.default_rng(15)
    physical = rng.integers(-3, 131, (3, 50)).astype(np.int32)
    physical[0, :3] = [5, 6, 7]
    raw = rng.integers(0, 40, (3, 50)).astype(np.int32)
    lengths = np.array([50, 20, 0], np.int32)
    freqs = oracle.rope_table(4 * 32)  # raw >= 32 is beyond the table
    rows = oracle.unpack_gather(pool, physical, raw, lengths, freqs)
    native = oracle.packed_to_native(pool, physical, raw, lengths, freqs)
    assert native.shape == (3, oracle.NATIVE_PAGE_BYTES)
    for i in range(150):
        page, slot = divmod(i, 64)
        data = native[page, slot * 576:(slot + 1) * 576]
        scales = native[page, 64 * 576 + slot * 8:64 * 576 + slot * 8 + 8]
        assert np.array_equal(oracle.native_unpack_row(data, scales), rows[i]), i
        if not rows[i].any():
            assert not data.any() and list(scales) == [105] * 7 + [0]
    assert sum(not r.any() for r in rows) > 20


def test_array_helpers_match_torch_and_ieee_float32():
    """The oracle's array forms, used to check the GPU's hardware rounding,
    agree with library routines: E4M3 encode with torch's float8_e4m3fn cast
    on every BF16 magnitude <= 448 and both signs; dequantisation with torch's
    float8 -> float32 cast times 2^(s - 127) rounded by torch's bfloat16 cast
    for every finite code and scale byte 105..247; the RMS reciprocal with
    numpy's correctly rounded float32 sqrt and division."""
    mags = all_bf16_magnitudes(448.0)
    q = np.concatenate([mags, -mags]).astype(np.float32)
    want = torch.from_numpy(q).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(oracle.e4m3_encode_array(q), want)
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    for s in (105, 110, 120, 127, 128, 140, 200, 247):
        vals = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float() * 2.0 ** (s - 127)
        want = vals.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        got = oracle.e4m3_dequant_array(codes, np.full(codes.shape, s, np.uint8))
        assert np.array_equal(got, want), s
    rng = np.random.default_rng(9)
    sumsq = rng.integers(0, 0x7F800000, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    for eps in (0.0, 1e-6):
        x = sumsq * np.float32(1.0 / 512.0) + np.float32(eps)
        want = (np.float32(1.0) / np.sqrt(x.astype(np.float32))).astype(np.float32)
        got = oracle.rms_scale_array(sumsq, np.full(sumsq.shape, eps, np.float32))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
