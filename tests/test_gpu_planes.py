"""GPU parity of the plane-form buffers: the reference's Packed pool planes
(values u8 [rows, K], bitmaps u64 [rows, 8], scales u8 [rows, 8];
candidate-sglang.patch:782-789, 839, 900-911) written by pack_rows_fused,
read in place by unpack_gather_bf16, the Adapter and the Direct decode
(through remnant_buffers). Bars: planes byte-identical to the contiguous
records the oracle checks, reconstruct and Adapter bit-exact vs the oracle,
decode identical to the contiguous-pool decode and within tolerance of the
oracle."""

import numpy as np
import pytest
import torch

import oracle
import remnant
from remnant import synthetic as syn
from test_gpu_parity import (DEV, KEEPS, OUT_TOL, COS_MIN, assert_pool_equal, build_decode_case,
                             gpu_pack, oracle_decode, oracle_pack)

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"[gpu-planes] {msg}", flush=True)


def planes_of(pool, keep=256):
    """Plane copies of a contiguous pool's records: values, bitmaps (u64), scales."""
    rec = pool.layer().reshape(-1, keep + 72)
    return (rec[:, :keep].contiguous(), rec[:, keep:keep + 64].contiguous().view(torch.uint64),
            rec[:, keep + 64:].contiguous())


def empty_planes(rows, keep, fill):
    return (torch.full((rows, keep), fill, dtype=torch.uint8, device=DEV),
            torch.full((rows, 64), fill, dtype=torch.uint8, device=DEV).view(torch.uint64),
            torch.full((rows, 8), fill, dtype=torch.uint8, device=DEV))


@pytest.mark.parametrize("keep_count", KEEPS)
def test_pack_into_planes_equals_contiguous_records(keep_count):
    """Every profile, both input dtypes: shuffled slots with skipped ones and
    canaries; the planes equal the (oracle-checked) contiguous records."""
    banner(f"pack planes keep {keep_count}")
    rng = np.random.default_rng(300 + keep_count)
    pages = 6
    x = torch.cat([syn.latents(320, seed=300 + keep_count).float(),
                   torch.from_numpy(rng.integers(-6, 7, (64, 512)).astype(np.float32))])
    slots = rng.permutation(pages * 64)[:384].astype(np.int32)
    slots[::41] = -1
    slots[7] = pages * 64 + 2  # past the planes
    for dtype in (torch.float32, torch.bfloat16):
        contiguous = gpu_pack(x.to(dtype), slots, pages, fill=0x5A, keep_count=keep_count)
        assert_pool_equal(contiguous, oracle_pack(x.to(dtype), slots, pages, fill=0x5A,
                                                  keep_count=keep_count))
        planes = empty_planes(pages * 64, keep_count, 0x5A)
        remnant.pack_rows_fused(x.to(dtype).to(DEV), torch.ones(512, device=DEV), 1e-6,
                                torch.from_numpy(slots).to(DEV), planes)
        torch.cuda.synchronize()
        for got, want in zip(planes, planes_of(contiguous, keep_count)):
            assert torch.equal(got.view(torch.uint8), want.view(torch.uint8))


@pytest.mark.parametrize("keep_count", KEEPS)
def test_unpack_gather_reads_planes_in_place(keep_count):
    """Reconstruct from the plane tuple (with RoPE, strided indices, invalid
    entries; and pre-RoPE) equals the oracle byte for byte."""
    banner(f"unpack planes keep {keep_count}")
    pages = 5
    rng = np.random.default_rng(320 + keep_count)
    x = syn.latents(pages * 64, seed=320 + keep_count)
    slots = rng.permutation(pages * 64).astype(np.int32)
    pool = gpu_pack(x, slots, pages, keep_count=keep_count)
    ref_pool = pool.layer().cpu().numpy()
    planes = planes_of(pool, keep_count)
    nq, nk = 4, 90
    physical = rng.integers(-3, pages * 64 + 3, (nq, nk)).astype(np.int32)
    raw = rng.integers(-1, 90, (nq, nk)).astype(np.int32)
    lengths = np.array([90, 0, 33, 89], np.int32)
    freqs = syn.rope_freqs(4 * 80)  # raw >= 80 is beyond the table
    wide = torch.zeros((nq, 2 * nk), dtype=torch.int32)
    wide[:, ::2] = torch.from_numpy(physical)
    ph, rw, ln = wide.to(DEV)[:, ::2], torch.from_numpy(raw).to(DEV), torch.from_numpy(lengths).to(DEV)
    out = torch.full((nq * nk + 2, 512), -91.0, dtype=torch.bfloat16, device=DEV)
    remnant.unpack_gather_bf16(planes, ph, rw, ln, freqs.to(DEV), out, fused_rope=True)
    plain = torch.empty((nq * nk, 512), dtype=torch.bfloat16, device=DEV)
    remnant.unpack_gather_bf16(remnant.remnant_buffers(*planes), ph, None, ln, None, plain)
    torch.cuda.synchronize()
    want = oracle.unpack_gather(ref_pool, physical, raw, lengths,
                                torch.view_as_real(freqs).numpy(), keep_count=keep_count)
    assert np.array_equal(syn.bf16_bits(out)[:nq * nk], want)
    assert np.all(out[nq * nk:].float().cpu().numpy() == -91)
    want_plain = oracle.unpack_gather(ref_pool, physical, None, lengths, keep_count=keep_count)
    assert np.array_equal(syn.bf16_bits(plain), want_plain)


def test_adapter_reads_planes_in_place():
    banner("adapter planes")
    pages = 4
    x = syn.latents(pages * 64, seed=341)
    slots = np.random.default_rng(341).permutation(pages * 64).astype(np.int32)
    pool = gpu_pack(x, slots, pages)
    rng = np.random.default_rng(342)
    nq, nk = 2, 100
    physical = rng.integers(-2, pages * 64 + 2, (nq, nk)).astype(np.int32)
    raw = rng.integers(-1, 70, (nq, nk)).astype(np.int32)
    lengths = np.array([100, 57], np.int32)
    freqs = syn.rope_freqs(4 * 64)
    native = remnant.LatentPool((nq * nk + 63) // 64, fmt="native", device=DEV)
    remnant.packed_to_native(planes_of(pool), torch.from_numpy(physical).to(DEV),
                             torch.from_numpy(raw).to(DEV), torch.from_numpy(lengths).to(DEV),
                             freqs.to(DEV), native)
    torch.cuda.synchronize()
    want = oracle.packed_to_native(pool.layer().cpu().numpy(), physical, raw, lengths,
                                   torch.view_as_real(freqs).numpy())
    got = native.layer().cpu().numpy()
    for i in range(nq * nk):
        pg, r = divmod(i, 64)
        assert np.array_equal(got[pg, r * 576:(r + 1) * 576], want[pg, r * 576:(r + 1) * 576])
        so = 64 * 576 + r * 8
        assert np.array_equal(got[pg, so:so + 8], want[pg, so:so + 8])


@pytest.mark.parametrize("swa", [False, True], ids=["c4", "c4+window"])
def test_direct_decode_reads_planes_through_remnant_buffers(swa):
    """The Direct decode over remnant_buffers(values, bitmaps, scales) gives
    the same bits as over the contiguous pool, and matches the oracle."""
    banner(f"decode planes swa={swa}")
    c = build_decode_case([900, 300, 2000, 1300], q_len=2, heads=32, topk=512, seed=343)
    c["lens"][1] = 77
    kw = dict(seqlens=torch.tensor(c["contexts"], dtype=torch.int32, device=DEV),
              topk_length=torch.from_numpy(c["lens"]).to(DEV), sink=c["sink"].to(DEV),
              freqs_cis=c["freqs"].to(DEV))
    if swa:
        from test_gpu_parity import add_swa
        add_swa(c, 64, seed=344)
        kw.update(swa_pool=c["swa_pool"], swa_indices=torch.from_numpy(c["swa_idx"]).to(DEV))
    q = c["q"].to(DEV)
    bt = torch.from_numpy(c["table"]).to(DEV)
    idx = torch.from_numpy(c["idx"]).to(DEV)
    out_c, lse_c = remnant.remnant_sparse_decode_fwd(q, c["pool"], bt, idx, **kw)
    buffers = remnant.remnant_buffers(*planes_of(c["pool"]))
    out_p, lse_p = remnant.remnant_sparse_decode_fwd(q, buffers, bt, idx, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out_p.view(torch.int16), out_c.view(torch.int16))
    assert torch.equal(lse_p, lse_c)
    ref, ref_lse = oracle_decode(c)
    got = out_p.float().cpu().numpy()
    assert np.abs(got - ref).max() <= OUT_TOL
    assert syn.cosine(got, ref) >= COS_MIN
    assert np.abs(lse_p.cpu().numpy() - ref_lse).max() <= OUT_TOL
