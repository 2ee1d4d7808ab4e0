"""The hardware-rounded primitives the kernels use, checked over their whole
input domains on the GPU (through libremnant_selftest.so, which calls the same
functions of remnant_device.h as the pack, reconstruct and decode kernels):

  * v_cvt_pk_bf16_f32 (BF16 rounding of the normalised values): every one of
    the 2^32 FP32 inputs, NaNs aside, equals round-to-nearest-even; a sample of
    16M inputs (plus every halfway case of a sample of exponents) equals the
    oracle's BF16 rounding byte for byte;
  * v_cvt_scalef32_pk_fp8_bf16 (the store's E4M3 encode): every finite BF16
    input at every scale exponent a store writes (-22..120), where
    |n / 2^e| <= 448, equals the oracle's E4M3 encode of n / 2^e;
  * v_cvt_scalef32_pk_bf16_fp8 (the readers' dequantisation): every finite
    code at every scale byte a store writes (105..247) equals the oracle's
    BF16(code * 2^(s - 127));
  * the store's RMS reciprocal r = RN(1 / RN(sqrt(x))): for every positive
    finite x, the root is the correctly rounded square root and r the
    correctly rounded reciprocal of it (proved per input by exact midpoint
    brackets in double precision), and r equals the oracle's on 4M sampled
    sums of squares and epsilons (denormals, zero, infinity included). The
    hardware v_sqrt_f32 alone fails this (x = 1e-6 gives the lower
    neighbour), which this test caught.

Each kernel counts mismatches with one global atomic per wave.
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"
HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "..", "flash-optimizations_amd", "remnant", "_lib",
                   "libremnant_selftest.so")


def banner(msg):
    print(f"[gpu-rounding] {msg}", flush=True)


@pytest.fixture(scope="module")
def st():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is not built (make -C flash-optimizations_amd/csrc)")
    lib = ctypes.CDLL(LIB)
    vp, u64, i64, i32, u32 = (ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int64, ctypes.c_int,
                              ctypes.c_uint32)
    lib.rmt_bf16_pair_mismatches.argtypes = [u64, u64, vp, vp]
    lib.rmt_fp8_encode_table.argtypes = [i32, i32, vp, vp, vp]
    lib.rmt_fp8_decode_table.argtypes = [vp, vp]
    lib.rmt_inv_root_mismatches.argtypes = [u32, u32, vp, vp]
    lib.rmt_inv_rms.argtypes = [vp, vp, vp, i64, vp]
    lib.rmt_bf16_array.argtypes = [vp, vp, i64, vp]
    return lib


def stream():
    return torch.cuda.current_stream().cuda_stream


def result_buffer():
    r = torch.zeros(2, dtype=torch.int64, device=DEV)
    r[1] = -1  # ~0: no mismatch seen
    return r


def read_result(r):
    torch.cuda.synchronize()
    count, first = r.cpu().numpy().view(np.uint64)
    return int(count), int(first)


def test_bf16_conversion_every_fp32_input(st):
    banner("bf16 conversion: all 2^32 inputs")
    r = result_buffer()
    for base in range(0, 1 << 32, 1 << 30):  # four launches of 2^30 inputs
        assert st.rmt_bf16_pair_mismatches(base, 1 << 30, r.data_ptr(), stream()) == 0
    count, first = read_result(r)
    assert count == 0, f"{count} mismatches, first input 0x{first:08x}"
    # the hardware results on a sample equal the oracle's rounding
    rng = np.random.default_rng(71)
    bits = rng.integers(0, 1 << 32, 1 << 24, dtype=np.uint64).astype(np.uint32)
    exps = np.arange(0, 255, dtype=np.uint32) << 23
    halfway = (exps[:, None] | (rng.integers(0, 1 << 7, (255, 64), dtype=np.uint32) << 16)
               | 0x8000).ravel()  # exact ties, both mantissa parities
    bits = np.concatenate([bits, halfway, halfway | 0x80000000, [0x7f7fffff, 0x7f7f8000]])
    bits = bits[(bits & 0x7fffffff) <= 0x7f800000]  # NaNs aside
    bits = bits[: bits.size // 2 * 2].astype(np.uint32)
    x = torch.from_numpy(bits.view(np.float32)).to(DEV)
    out = torch.empty(bits.size, dtype=torch.int16, device=DEV)
    assert st.rmt_bf16_array(x.data_ptr(), out.data_ptr(), bits.size, stream()) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16)
    assert np.array_equal(got, oracle.f32_to_bf16_np(bits.view(np.float32)))


def test_fp8_encode_every_bf16_input_and_scale(st):
    banner("scaled fp8 encode: all bf16 x scales -22..120")
    e_lo, e_hi = -22, 120
    n_e = e_hi - e_lo + 1
    out = torch.empty(n_e * 65536, dtype=torch.uint8, device=DEV)
    r = result_buffer()
    assert st.rmt_fp8_encode_table(e_lo, e_hi, out.data_ptr(), r.data_ptr(), stream()) == 0
    count, _ = read_result(r)
    assert count == 0, "the two halves of a pair conversion differ"
    table = out.cpu().numpy().reshape(n_e, 65536)
    n_bits = np.arange(65536, dtype=np.uint32)
    with np.errstate(invalid="ignore"):  # NaN patterns, excluded below
        n_val = (n_bits << 16).view(np.float32).astype(np.float64)
    finite = np.isfinite(n_val)
    checked = 0
    for i, e in enumerate(range(e_lo, e_hi + 1)):
        q = n_val * 2.0 ** -e
        ok = finite & (np.abs(q) <= 448.0)
        want = oracle.e4m3_encode_array(q[ok].astype(np.float32))
        got = table[i][ok]
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (e, hex(int(n_bits[ok][bad[0]])), got[bad[0]], want[bad[0]])
        checked += int(ok.sum())
    assert checked > 5_000_000


def test_fp8_dequant_every_code_and_scale(st):
    banner("scaled fp8 decode: all codes x scale bytes 105..247")
    out = torch.empty(256 * 256, dtype=torch.int16, device=DEV)
    assert st.rmt_fp8_decode_table(out.data_ptr(), stream()) == 0
    torch.cuda.synchronize()
    table = out.cpu().numpy().view(np.uint16).reshape(256, 256)
    codes = np.array([c for c in range(256) if (c & 0x7f) != 0x7f], np.uint8)  # NaN codes aside
    for s in range(105, 248):
        want = oracle.e4m3_dequant_array(codes, np.full(codes.shape, s, np.uint8))
        got = table[s][codes]
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (s, int(codes[bad[0]]), hex(got[bad[0]]), hex(want[bad[0]]))


def test_rms_reciprocal_correctly_rounded_every_input_and_oracle_sample(st):
    banner("rms reciprocal: every positive finite x, oracle sample")
    r = result_buffer()
    lo, hi = 0x00000001, 0x7F800000
    step = 1 << 28
    for base in range(lo, hi, step):
        assert st.rmt_inv_root_mismatches(base, min(base + step, hi), r.data_ptr(),
                                          stream()) == 0
    count, first = read_result(r)
    assert count == 0, f"{count} mismatches, first x 0x{first:08x}"
    rng = np.random.default_rng(72)
    n = 1 << 22
    sumsq = rng.integers(0, 0x7F800001, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    sumsq[:8] = np.array([0.0, 1e-45, 1e-40, 2.0 ** -150 * 3, 1.0, 512.0, 3e38, np.inf],
                         np.float32)
    eps = np.choose(rng.integers(0, 3, n), [np.float32(0.0), np.float32(1e-6),
                                            np.float32(1e-5)]).astype(np.float32)
    s_d = torch.from_numpy(sumsq).to(DEV)
    e_d = torch.from_numpy(eps).to(DEV)
    out = torch.empty(n, dtype=torch.float32, device=DEV)
    assert st.rmt_inv_rms(s_d.data_ptr(), e_d.data_ptr(), out.data_ptr(), n, stream()) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32)
    want = oracle.rms_scale_array(sumsq, eps).view(np.uint32)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (float(sumsq[bad[0]]), float(eps[bad[0]]), hex(got[bad[0]]),
                           hex(want[bad[0]]))
