"""The Direct decode's position mode: the tail rotation computed from the
record positions and the table's inverse frequencies instead of read from
256-byte table rows.

The reference's reader rotates the BF16 tail of logical record r by row r * 4
of ``freqs_cis`` (candidate-sglang.patch:640-661, 692), a table the caller
builds as polar(1, pos * theta_j) with the angle in FP32. In position mode the
kernel forms the same FP32 angle RN(RN(4 r) * theta_j) and evaluates its cos
and sin itself (remnant_device.h rope_sincos: a two-term reduction to
revolutions, then v_sin_f32 / v_cos_f32). Checked here:

* the hardware sin/cos over every FP32 fraction of a revolution in [-1/2, 1/2]
  against sin(2 pi f) in double precision;
* the kernel's (cos, sin) for positions 0 .. 2^22 (step 4) against float64
  cos/sin of the same FP32 angles, and against torch.polar's table rows;
* the decode in position mode against the oracle (which rotates with the
  table) at every kernel variant the mode adds: one and two 16-head groups,
  contiguous pools and plane buffers, short and long (table-refilling) splits,
  with and without window rows, second passes, the batched shape at
  4k-128k-token contexts (angles up to 131,068 rad), per-row at a realistic
  logit spread, and under HIP-graph replay with changed inputs.

Parity bar: the decode's, |out - ref| <= 0.02 + 0.02 |ref| and cosine >=
0.9999 per (token, head) row where stated, else max-abs <= 0.02 and cosine >=
0.9999 overall (the stated decode tolerance; the reference checks attention at
atol = rtol = 0.02, docs/report.md:20).
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import remnant
from remnant import synthetic as syn
from test_gpu_decode_edges import per_row_check
from test_gpu_parity import (COS_MIN, DEV, OUT_TOL, add_swa, build_decode_case, check_decode,
                             oracle_decode, run_decode)
from test_gpu_planes import planes_of

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "..", "flash-optimizations_amd", "remnant", "_lib",
                   "libremnant_selftest.so")
# cos/sin of a RoPE angle within this absolute error of float64 (and of the
# FP32 table): a few FP32 ulps of 1
SINCOS_TOL = 2.0 ** -20


def banner(msg):
    print(f"[gpu-rope-positions] {msg}", flush=True)


@pytest.fixture(scope="module")
def st():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (make -C flash-optimizations_amd/csrc)")
    lib = ctypes.CDLL(LIB)
    vp, i64, i32, u32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint32
    lib.rmt_rope_cos_sin.argtypes = [vp, i64, i32, vp, vp]
    lib.rmt_sincos_error.argtypes = [u32, u32, vp, vp]
    return lib


def test_hardware_sincos_error_over_every_fraction(st):
    """v_sin_f32 / v_cos_f32 at every FP32 f in [-1/2, 1/2] (about 2.1e9
    inputs) against sin(2 pi f), cos(2 pi f) evaluated in double."""
    banner("v_sin / v_cos over every fraction of a revolution")
    worst = []
    for first, end in ((0x00000000, 0x3F000001), (0x80000000, 0xBF000001)):
        err = torch.zeros(2, dtype=torch.int32, device=DEV)
        assert st.rmt_sincos_error(first, end, err.data_ptr(),
                                   torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        worst.append(err.cpu().numpy().view(np.float32))
    worst = np.max(np.stack(worst), axis=0)
    banner(f"max |error|: sin {worst[0]:.3e}, cos {worst[1]:.3e}")
    assert worst.max() <= SINCOS_TOL, worst


def test_position_rotation_against_float64_and_the_table(st):
    """cos and sin of RN(pos * theta_j) for pos = 0, 4, ..., 4 (2^20 - 1):
    within SINCOS_TOL of float64 at every position, and of the rows torch.polar
    builds for the decode's table (positions below 4 * 32768)."""
    banner("position rotation vs float64 and torch.polar")
    theta = syn.rope_inv_freq()
    n_pos = 1 << 20
    out = torch.empty(n_pos * 64, dtype=torch.float32, device=DEV)
    assert st.rmt_rope_cos_sin(theta.to(DEV).data_ptr(), n_pos, 4, out.data_ptr(),
                               torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(n_pos, 32, 2)
    pos = (np.arange(n_pos, dtype=np.int64) * 4).astype(np.float32)
    ang = (pos[:, None] * theta.numpy()[None, :]).astype(np.float32)  # one FP32 rounding
    a64 = ang.astype(np.float64)
    err_c = np.abs(got[..., 0] - np.cos(a64)).max()
    err_s = np.abs(got[..., 1] - np.sin(a64)).max()
    banner(f"vs float64: cos {err_c:.3e}, sin {err_s:.3e} (angles up to {ang.max():.0f} rad)")
    assert max(err_c, err_s) <= SINCOS_TOL
    rows = 32768
    table = torch.polar(torch.ones(rows, 32), torch.from_numpy(ang[:rows]))
    ref = torch.view_as_real(table).numpy()
    diff = np.abs(got[:rows] - ref)
    banner(f"vs table: max {diff.max():.3e}, identical {np.mean(diff == 0):.4f}")
    assert diff.max() <= SINCOS_TOL
    # the synthetic table's rows 4 r are the same rows
    full = syn.rope_freqs(4 * 1024)
    np.testing.assert_array_equal(torch.view_as_real(full[::4]).numpy(), ref[:1024])


POSITION_CASES = {
    # name: (contexts, q_len, heads, topk, seed, extra)
    "padding_duplicates_sink": ([300, 70, 1000], 1, 16, 256, 611, "dup"),
    "b1_topk2048_ctx8192": ([8192], 1, 16, 2048, 612, None),
    "next_n2_h32": ([700, 2000], 2, 32, 512, 613, None),
    "h128_two_head_groups": ([900, 1500, 600, 2000, 700, 1100, 1300, 800], 2, 128, 512, 614,
                             None),
    "second_pass_wide_scores": ([3000, 900], 1, 16, 1024, 615, "wide"),
    "partial_stage_short_lengths": ([500, 300, 800, 64], 1, 16, 100, 616, "short"),
    "maximum_topk": ([33000], 1, 16, 32768, 617, None),
    "window_lengths": ([300, 70, 1000], 1, 16, 256, 618, "swa"),
    "window_h128_b16": (None, 1, 128, 512, 619, "swa16"),
}


@pytest.mark.parametrize("name", list(POSITION_CASES))
def test_decode_position_mode_matches_oracle(name):
    contexts, q_len, heads, topk, seed, extra = POSITION_CASES[name]
    banner(f"decode positions {name}")
    if contexts is None:
        contexts = syn.log_uniform_contexts(16, 2048, 16384, seed)
    c = build_decode_case(contexts, q_len=q_len, heads=heads, topk=topk, seed=seed)
    c["rope"] = "positions"
    if extra == "dup":
        c["idx"][1, 0, 3] = 5000  # beyond the request's records
        c["idx"][2, 0, 7] = c["idx"][2, 0, 8]
    elif extra == "wide":
        c["q"] = (c["q"].float() * 300).to(torch.bfloat16)
    elif extra == "short":
        c["lens"][:] = np.array([100, 37, 0, 1], np.int32).reshape(c["lens"].shape)
    elif extra == "swa":
        add_swa(c, 64, seed=seed + 100, lengths=[64, 10, 0])
    elif extra == "swa16":
        add_swa(c, 64, seed=seed + 100)
    check_decode(c)


@pytest.mark.parametrize("shape", ["b1", "b64_128k"])
def test_decode_position_mode_per_row_at_realistic_logit_spread(shape):
    """Logits with std ~4 and every (token, head) row on its own bar; the
    batched shape spans 4k-128k-token contexts (positions up to 131,068)."""
    banner(f"decode positions per row {shape}")
    if shape == "b1":
        c = build_decode_case([8192], q_len=1, heads=16, topk=2048, seed=621)
    else:
        ctx = syn.log_uniform_contexts(64, 4096, 131072, 622)
        c = build_decode_case(ctx, q_len=1, heads=16, topk=2048, seed=622)
    c["q"] = (c["q"].float() * 8.0).to(torch.bfloat16)
    c["rope"] = "positions"
    out, lse = run_decode(c)
    ref, ref_lse = oracle_decode(c)
    per_row_check(out, ref, lse, ref_lse)
    # and close to the table-row decode of the same inputs
    c["rope"] = "table"
    out_t, _ = run_decode(c)
    banner(f"positions vs table rows: max |diff| {np.abs(out - out_t).max():.3e}")
    assert np.abs(out - out_t).max() <= OUT_TOL


@pytest.mark.parametrize("rope", ["table", "positions"])
@pytest.mark.parametrize("swa", [False, True], ids=["c4", "c4+window"])
def test_decode_long_splits_on_plane_buffers(rope, swa):
    """Long splits (256 tokens x 16 heads, top-k 1504: one split per token
    streaming 47 stages, its record table refilled ring-wise) read from plane
    buffers, with and without window rows: the same bits as the contiguous
    pool, and every row within the bar of the oracle."""
    banner(f"decode long splits planes rope={rope} swa={swa}")
    ctx = syn.log_uniform_contexts(128, 6400, 12000, 631)
    topk = 1504
    c = build_decode_case(ctx, q_len=2, heads=16, topk=topk, seed=631)
    assert remnant.get_decode_metadata(256, 16, topk)[0] == 1
    lens = c["lens"].reshape(-1)
    lens[1:6] = [1000, 513, 512, 31, 0]
    c["rope"] = rope
    if swa:
        add_swa(c, 64, seed=632)
    out_c, lse_c = run_decode(c)
    contiguous = c["pool"]
    c["pool"] = remnant.remnant_buffers(*planes_of(contiguous))
    out_p, lse_p = run_decode(c)
    assert np.array_equal(out_p.view(np.uint32), out_c.view(np.uint32))
    assert np.array_equal(lse_p.view(np.uint32), lse_c.view(np.uint32))
    c["pool"] = contiguous
    ref, ref_lse = oracle_decode(c)
    per_row_check(out_p, ref, lse_p, ref_lse)


@pytest.mark.parametrize("swa", [False, True], ids=["c4", "c4+window"])
def test_decode_position_mode_short_splits_on_plane_buffers(swa):
    banner(f"decode planes positions swa={swa}")
    c = build_decode_case([900, 300, 2000, 1300], q_len=2, heads=32, topk=512, seed=641)
    c["lens"][1] = 77
    c["rope"] = "positions"
    if swa:
        add_swa(c, 64, seed=642)
    out_c, lse_c = run_decode(c)
    contiguous = c["pool"]
    c["pool"] = remnant.remnant_buffers(*planes_of(contiguous))
    out_p, lse_p = run_decode(c)
    assert np.array_equal(out_p.view(np.uint32), out_c.view(np.uint32))
    assert np.array_equal(lse_p.view(np.uint32), lse_c.view(np.uint32))
    c["pool"] = contiguous
    ref, ref_lse = oracle_decode(c)
    assert np.abs(out_p - ref).max() <= OUT_TOL
    assert syn.cosine(out_p, ref) >= COS_MIN


def test_decode_position_mode_bounded_by_a_given_table():
    """With both inverse frequencies and a table, the table's rows still bound
    the valid records (records with 4 r >= rows contribute nothing), as in
    table mode; the rotation comes from the positions."""
    banner("decode positions + table bound")
    c = build_decode_case([2000, 700], q_len=1, heads=16, topk=512, seed=651)
    c["freqs"] = syn.rope_freqs(4 * 1000)  # records >= 1000 are beyond the table
    ref, ref_lse = oracle_decode(c)
    q = c["q"].to(DEV)
    out, lse = remnant.remnant_sparse_decode_fwd(
        q, c["pool"], torch.from_numpy(c["table"]).to(DEV), torch.from_numpy(c["idx"]).to(DEV),
        seqlens=torch.tensor(c["contexts"], dtype=torch.int32, device=DEV),
        topk_length=torch.from_numpy(c["lens"]).to(DEV), sink=c["sink"].to(DEV),
        freqs_cis=c["freqs"].to(DEV), rope_inv_freq=syn.rope_inv_freq().to(DEV))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert (c["idx"][0, 0] >= 1000).sum() > 100  # the bound removes many records
    assert np.abs(got - ref).max() <= OUT_TOL and syn.cosine(got, ref) >= COS_MIN
    assert np.abs(lse.cpu().numpy() - ref_lse).max() <= OUT_TOL
