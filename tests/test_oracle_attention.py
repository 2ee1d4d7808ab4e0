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


def test_joint_swa_decode_matches_reference_formula():
    """training/losses.py:393-398: rows = cat(swa, C4 rows); probabilities =
    softmax(cat(q rows^T * scale, sink))[..., :-1]; out = probabilities @ rows,
    evaluated with torch in float64. SWA rows come from a Native pool by
    physical slot; slots past swa_length or outside the pool are skipped."""
    rng = np.random.default_rng(11)
    pages, swa_pages = 4, 2
    x = oracle.synthetic_latents(pages * 64, seed=12)
    pool = np.zeros((pages, oracle.PAGE_BYTES), np.uint8)
    oracle.pack_rows_paged(x, np.ones(512, np.float32), 1e-6,
                           np.arange(pages * 64, dtype=np.int32), pool)
    sx = oracle.synthetic_latents(swa_pages * 64, seed=13)
    spool = np.zeros((swa_pages, oracle.NATIVE_PAGE_BYTES), np.uint8)
    freqs = oracle.rope_table(4 * 256)
    oracle.native_pack_rows_paged(sx, np.ones(512, np.float32), 1e-6,
                                  np.arange(swa_pages * 64, dtype=np.int32),
                                  np.arange(swa_pages * 64, dtype=np.int32), freqs, spool)
    block_table = np.arange(pages, dtype=np.int32)[None]
    idx = rng.choice(256, 48, replace=False).astype(np.int32)
    swa = rng.choice(128, 20, replace=False).astype(np.int32)
    swa[3] = 128 * 5  # outside the SWA pool
    swa[7] = -1
    q = bf16(rng.standard_normal((1, 1, 16, 512)) * 0.3)
    sink = rng.standard_normal(16).astype(np.float32)
    scale = float(np.float32(1 / np.sqrt(512)))
    out, lse = oracle.sparse_decode_swa(q, pool, True, block_table, None, idx[None, None], None,
                                        spool, swa[None, None], np.array([18], np.int32), sink,
                                        freqs, scale)
    # independent assembly of the rows: Native records by slot, C4 rows by unpack_gather
    swa_rows = []
    for k, sl in enumerate(swa[:18]):
        if 0 <= sl < 128:
            pg, inn = divmod(int(sl), 64)
            page = spool[pg]
            swa_rows.append(oracle.native_unpack_row(page[inn * 576:(inn + 1) * 576],
                                                     page[64 * 576 + inn * 8:64 * 576 + inn * 8 + 8]))
    c4 = oracle.unpack_gather(pool, idx[None], idx[None], np.array([48]), freqs)
    rows = torch.from_numpy(oracle.bf16_to_f32(np.concatenate([np.stack(swa_rows), c4]))
                            .astype(np.float64))
    qf = torch.from_numpy(oracle.bf16_to_f32(q[0, 0]).astype(np.float64))
    logits = qf @ rows.T * scale
    s = torch.from_numpy(sink.astype(np.float64))[:, None]
    prob = torch.softmax(torch.cat([logits, s], 1), 1)[:, :-1]
    np.testing.assert_allclose(out[0, 0], (prob @ rows).numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(lse[0, 0], torch.logsumexp(torch.cat([logits, s], 1), 1).numpy(),
                               rtol=1e-12)
    assert len(swa_rows) == 16
    # no SWA rows: identical to the plain decode
    none, none_lse = oracle.sparse_decode_swa(q, pool, True, block_table, None, idx[None, None],
                                              None, spool, swa[None, None], np.array([0], np.int32),
                                              sink, freqs, scale)
    plain, plain_lse = oracle.sparse_decode(q, pool, True, block_table, None, idx[None, None],
                                            None, sink, freqs, scale)
    np.testing.assert_array_equal(none, plain)
    np.testing.assert_array_equal(none_lse, plain_lse)


def test_threaded_batch_loops_give_identical_results():
    """The CPU baseline runs the oracle's pack, reconstruct and decode loops on
    every host core; each record, row and token is computed the same way on
    any thread count. Three tokens on 2 threads take the per-token schedule,
    on 4 threads the one for fewer tokens than threads (records gathered in
    chunks, heads in parallel)."""
    from remnant import synthetic as syn
    x = syn.latents(640, seed=90).float().numpy()
    slots = np.random.default_rng(90).permutation(640).astype(np.int32)
    q = syn.bf16_bits(syn.latents(3 * 16, seed=91)).reshape(3, 1, 16, 512)
    table = np.arange(10, dtype=np.int32).reshape(1, 10).repeat(3, 0)
    idx = np.random.default_rng(92).integers(-1, 640, (3, 1, 300)).astype(np.int32)
    lens = np.array([300, 17, 0], np.int32)
    freqs = torch.view_as_real(syn.rope_freqs(4 * 640)).numpy()
    results = []
    try:
        for threads in (1, 2, 4):
            oracle.set_threads(threads)
            assert oracle.get_threads() == threads
            pool = np.zeros((10, oracle.PAGE_BYTES), np.uint8)
            oracle.pack_rows_paged(x, np.ones(512, np.float32), 1e-6, slots, pool)
            rows = oracle.unpack_gather(pool, slots.reshape(4, 160), slots.reshape(4, 160),
                                        np.array([160, 3, 160, 0], np.int32), freqs)
            out, lse = oracle.sparse_decode(q, pool, True, table, np.full(3, 640, np.int32), idx,
                                            lens, np.zeros(16, np.float32), freqs,
                                            1 / np.sqrt(512))
            results.append((pool, rows, out, lse))
    finally:
        oracle.set_threads(1)
    for other in results[1:]:
        for a, b in zip(results[0], other):
            assert np.array_equal(a, b)


def test_single_precision_decode_baseline_matches_double():
    """The CPU baseline's single-precision decode (oracle.set_decode_f32) agrees
    with the checker's double-precision decode within the decode bar, and the
    checker's arithmetic is restored afterwards."""
    from remnant import synthetic as syn
    x = syn.latents(640, seed=95).float().numpy()
    slots = np.random.default_rng(95).permutation(640).astype(np.int32)
    pool = np.zeros((10, oracle.PAGE_BYTES), np.uint8)
    oracle.pack_rows_paged(x, np.ones(512, np.float32), 1e-6, slots, pool)
    q = syn.bf16_bits(syn.latents(2 * 16, seed=96) * 4).reshape(2, 1, 16, 512)
    table = np.arange(10, dtype=np.int32).reshape(1, 10).repeat(2, 0)
    idx = np.random.default_rng(97).integers(0, 640, (2, 1, 400)).astype(np.int32)
    lens = np.array([400, 250], np.int32)
    freqs = torch.view_as_real(syn.rope_freqs(4 * 640)).numpy()
    sink = np.linspace(-1, 1, 16).astype(np.float32)
    args = (q, pool, True, table, np.full(2, 640, np.int32), idx, lens, sink, freqs,
            1 / np.sqrt(512))
    ref, ref_lse = oracle.sparse_decode(*args)
    try:
        oracle.set_decode_f32(True)
        out, lse = oracle.sparse_decode(*args)
    finally:
        oracle.set_decode_f32(False)
    assert not np.array_equal(out, ref)  # a different evaluation
    assert np.abs(out - ref).max() <= 1e-4 and np.abs(lse - ref_lse).max() <= 1e-4
    again, _ = oracle.sparse_decode(*args)
    assert np.array_equal(again, ref)
