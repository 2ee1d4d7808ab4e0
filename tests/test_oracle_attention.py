"""Pin the oracle's sparse sink attention (training/losses.py:393-398,
test_integration.py:1620-1635) against torch's scaled-dot-product attention
(a library routine) and the invariants the reference's decode tests rely on."""

import numpy as np
import torch

import oracle


def bf16(x):
    return oracle.f32_to_bf16_np(np.asarray(x, np.float32))


def sdpa_reference(q_bits, rows_bits, valid, sink, scale):
    """Sink as an extra zero key/value row whose logit is the sink value
    (test_integration.py:1620-1627), through torch SDPA in float64. The scale
    is the float32 value the kernels receive."""
    scale = float(np.float32(scale))
    q = torch.from_numpy(oracle.bf16_to_f32(q_bits).astype(np.float64))
    k = torch.from_numpy(oracle.bf16_to_f32(rows_bits).astype(np.float64))[valid]
    k = torch.cat([k, torch.zeros(1, 512, dtype=torch.float64)])
    bias = torch.zeros(q.shape[0], k.shape[0], dtype=torch.float64)
    bias[:, -1] = torch.from_numpy(sink.astype(np.float64))
    out = torch.nn.functional.scaled_dot_product_attention(
        q[None], k[None], k[None], attn_mask=bias[None], scale=scale)[0]
    logits = torch.cat([q @ k[:-1].T * scale, bias[:, -1:]], 1)
    return out.numpy(), torch.logsumexp(logits, 1).numpy()


def make(seed, heads=16, nk=300):
    rng = np.random.default_rng(seed)
    q = bf16(rng.standard_normal((heads, 512)) * 0.5)
    rows = bf16(rng.standard_normal((nk, 512)))
    valid = rng.random(nk) < 0.9
    sink = rng.standard_normal(heads).astype(np.float32)
    return q, rows, valid, sink


def test_attention_matches_torch_sdpa_with_sink_row():
    q, rows, valid, sink = make(0)
    scale = 1 / np.sqrt(512)
    out, lse = oracle.sink_attention(q, rows, valid.astype(np.uint8), sink, scale)
    ref_out, ref_lse = sdpa_reference(q, rows, valid, sink, scale)
    np.testing.assert_allclose(out, ref_out, rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(lse, ref_lse, rtol=1e-12, atol=1e-12)


def test_attention_probabilities_sum_to_one_with_sink():
    """Identical rows: out = row * (1 - sink weight) exactly (closed form)."""
    q, rows, _, sink = make(1, nk=50)
    rows[:] = rows[0]
    valid = np.ones(50, np.uint8)
    out, lse = oracle.sink_attention(q, rows, valid, sink, 0.1)
    row = oracle.bf16_to_f32(rows[0]).astype(np.float64)
    logit = (oracle.bf16_to_f32(q).astype(np.float64) @ row) * np.float64(np.float32(0.1))
    z = 50 * np.exp(logit) + np.exp(sink.astype(np.float64))
    np.testing.assert_allclose(out, (50 * np.exp(logit) / z)[:, None] * row[None], rtol=1e-12)
    np.testing.assert_allclose(lse, np.log(z), rtol=1e-12)


def test_attention_invariants_permutation_duplicates_invalid():
    q, rows, valid, sink = make(2, nk=64)
    v = valid.astype(np.uint8)
    base, base_lse = oracle.sink_attention(q, rows, v, sink, 0.05)
    perm = np.random.default_rng(3).permutation(64)
    p_out, p_lse = oracle.sink_attention(q, rows[perm], v[perm], sink, 0.05)
    np.testing.assert_allclose(p_out, base, rtol=1e-12, atol=1e-14)
    # invalid rows contribute nothing, whatever they hold
    garbage = rows.copy()
    garbage[~valid] = bf16(np.full(512, 1e4))
    g_out, _ = oracle.sink_attention(q, garbage, v, sink, 0.05)
    np.testing.assert_array_equal(g_out, base)
    # a duplicated index counts twice: same as adding log(2) to its logit
    dup_rows = np.concatenate([rows, rows[:1]])
    dup_valid = np.concatenate([v, [1]]).astype(np.uint8)
    d_out, d_lse = oracle.sink_attention(q, dup_rows, dup_valid, sink, 0.05)
    ref_out, ref_lse = sdpa_reference(q, dup_rows, dup_valid.astype(bool), sink, 0.05)
    np.testing.assert_allclose(d_out, ref_out, rtol=1e-9, atol=1e-12)
    assert not np.allclose(d_out, base)


def test_attention_empty_selection():
    q, rows, _, sink = make(4, nk=8)
    none = np.zeros(8, np.uint8)
    out, lse = oracle.sink_attention(q, rows, none, None, 0.1)
    assert np.all(out == 0) and np.all(np.isneginf(lse))
    out, lse = oracle.sink_attention(q, rows, none, sink, 0.1)
    assert np.all(out == 0) and np.allclose(lse, sink)


def test_decode_gather_through_block_table_matches_unpack_gather():
    """Decode reads record r of request b at page block_table[b, r // 64], slot
    r % 64, with RoPE row r * 4: the same rows unpack_gather_bf16 returns."""
    rng = np.random.default_rng(5)
    pages = 6
    x = oracle.synthetic_latents(pages * 64, seed=9)
    pool = np.zeros((pages, oracle.PAGE_BYTES), np.uint8)
    oracle.pack_rows_paged(x, np.ones(512, np.float32), 1e-6,
                           np.arange(pages * 64, dtype=np.int32), pool)
    block_table = rng.permutation(pages).astype(np.int32)[None, :4]
    freqs = oracle.rope_table(4 * 256)
    idx = rng.choice(256, 40, replace=False).astype(np.int32)
    q = bf16(rng.standard_normal((1, 1, 16, 512)))
    out, lse = oracle.sparse_decode(q, pool, True, block_table, np.array([256]),
                                    idx[None, None], None, None, freqs, 1 / np.sqrt(512))
    physical = block_table[0, idx // 64] * 64 + idx % 64
    rows = oracle.unpack_gather(pool, physical[None], idx[None], np.array([40]), freqs)
    ref, ref_lse = oracle.sink_attention(q[0, 0], rows, np.ones(40, np.uint8), None,
                                         1 / np.sqrt(512))
    np.testing.assert_array_equal(out[0, 0], ref)
    np.testing.assert_array_equal(lse[0, 0], ref_lse)
