"""CPU oracle for the Remnant packed-KV path -- test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import this package, and only as the checker. The product
path (``remnant`` under ``flash-optimizations_amd/``) never calls it.

The arithmetic lives in ``remnant_oracle.c`` (built to ``liboracle.so`` by the
Makefile beside it); this module wraps it with numpy arrays. Reference
formulas it restates are cited in the C file's header; every function here is
pinned by tests in ``tests/test_oracle_*.py`` against the reference's own
known-answer tests, library routines (torch's float8/bfloat16 casts, topk,
scaled-dot-product attention) and closed forms.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HEAD_DIM = 512
NOPE_DIM = 448
ROPE_PAIRS = 32
KEEP = 256
PAGE_RECORDS = 64
DATA_BYTES = 320
SCALE_BYTES = 8
RECORD_BYTES = DATA_BYTES + SCALE_BYTES
PAGE_BYTES = PAGE_RECORDS * RECORD_BYTES
NATIVE_DATA_BYTES = 576
NATIVE_RECORD_BYTES = NATIVE_DATA_BYTES + SCALE_BYTES
NATIVE_PAGE_BYTES = PAGE_RECORDS * NATIVE_RECORD_BYTES
KEEP_COUNTS = tuple(range(64, 512, 64))  # survivor profiles 64..448


def record_bytes(keep_count: int = KEEP) -> int:
    """Bytes of one Packed record with ``keep_count`` survivors (count + 72)."""
    return keep_count + 64 + SCALE_BYTES


def page_bytes(keep_count: int = KEEP) -> int:
    return PAGE_RECORDS * record_bytes(keep_count)

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        i64, f32, vp = ctypes.c_int64, ctypes.c_float, ctypes.c_void_p
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_f32_to_bf16.argtypes = [f32]
        _lib.orc_e4m3_encode.restype = ctypes.c_uint8
        _lib.orc_e4m3_encode.argtypes = [f32]
        _lib.orc_e4m3_decode.restype = f32
        _lib.orc_e4m3_decode.argtypes = [ctypes.c_uint8]
        _lib.orc_ue8m0_exponent.restype = ctypes.c_int
        _lib.orc_ue8m0_exponent.argtypes = [f32]
        _lib.orc_sumsq.restype = f32
        _lib.orc_sumsq.argtypes = [vp]
        _lib.orc_rms_scale.restype = f32
        _lib.orc_rms_scale.argtypes = [f32, f32]
        _lib.orc_select_keep.argtypes = [vp, vp]
        _lib.orc_select_keep_k.argtypes = [vp, vp, ctypes.c_int]
        _lib.orc_pack_row_k.argtypes = [vp, vp, f32, ctypes.c_int, vp, vp, vp, vp]
        _lib.orc_pack_rows_paged_k.argtypes = [vp, vp, f32, ctypes.c_int, vp, i64, vp, i64]
        _lib.orc_unpack_row_k.argtypes = [vp, vp, ctypes.c_int, vp]
        _lib.orc_unpack_gather_k.argtypes = [vp, i64, ctypes.c_int, vp, i64, i64, vp, i64,
                                             i64, vp, i64, i64, i64, vp, i64, vp]
        _lib.orc_normalize.argtypes = [vp, vp, vp, f32, vp]
        _lib.orc_set_threads.argtypes = [ctypes.c_int]
        _lib.orc_set_decode_f32.argtypes = [ctypes.c_int]
        _lib.orc_get_threads.restype = ctypes.c_int
        _lib.orc_e4m3_encode_n.argtypes = [vp, i64, vp]
        _lib.orc_e4m3_dequant_n.argtypes = [vp, vp, i64, vp]
        _lib.orc_rms_scale_n.argtypes = [vp, vp, i64, vp]
        _lib.orc_simulate_rows.argtypes = [vp, vp, vp, f32, i64, vp]
        _lib.orc_pack_row.argtypes = [vp, vp, f32, vp, vp, vp, vp]
        _lib.orc_pack_rows_paged.argtypes = [vp, vp, f32, vp, i64, vp, i64]
        _lib.orc_unpack_row.argtypes = [vp, vp, vp]
        _lib.orc_rope_tail.argtypes = [vp, vp]
        _lib.orc_unpack_gather.argtypes = [vp, i64, vp, i64, i64, vp, i64, i64, vp, i64,
                                           i64, i64, vp, i64, vp]
        _lib.orc_native_pack_row.argtypes = [vp, vp, f32, vp, vp, vp]
        _lib.orc_native_pack_rows_paged.argtypes = [vp, vp, f32, vp, vp, vp, i64, i64, vp, i64]
        _lib.orc_native_unpack_row.argtypes = [vp, vp, vp]
        _lib.orc_sink_attention.argtypes = [vp, i64, vp, vp, i64, vp, f32, vp, vp]
        _lib.orc_sparse_decode.argtypes = [vp, i64, i64, i64, vp, i64, ctypes.c_int, vp, i64,
                                           i64, vp, vp, i64, vp, vp, vp, i64, f32, vp, vp]
        _lib.orc_native_encode_row.argtypes = [vp, vp, vp]
        _lib.orc_packed_to_native.argtypes = [vp, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64,
                                              i64, vp, i64, vp]
        _lib.orc_swa_gather.argtypes = [vp, i64, vp, i64, i64, vp, vp]
        _lib.orc_sparse_decode_swa.argtypes = [vp, i64, i64, i64, vp, i64, ctypes.c_int, vp,
                                               i64, i64, vp, vp, i64, vp, vp, i64, vp, i64, vp,
                                               vp, vp, i64, f32, vp, vp]
    return _lib


def set_threads(n: int) -> None:
    """Threads of the batch loops (pack, reconstruct, decode); results do not
    depend on it. With more than one thread pack slots must be distinct."""
    lib().orc_set_threads(int(n))


def get_threads() -> int:
    return int(lib().orc_get_threads())


def set_decode_f32(on: bool) -> None:
    """Decode arithmetic in single precision (a CPU baseline at the kernels'
    accumulation width) instead of the checker's double precision."""
    lib().orc_set_decode_f32(int(bool(on)))


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---- scalar codec pieces -------------------------------------------------

def bf16_bits(x) -> np.ndarray:
    """float32 values -> bf16 bit patterns (uint16), round to nearest even."""
    x = _c(x, np.float32)
    f = np.vectorize(lambda v: lib().orc_f32_to_bf16(float(v)), otypes=[np.uint16])
    return f(x) if x.size else x.astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (_c(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_np(x) -> np.ndarray:
    """Vectorised float32 -> bf16 bits (RNE), same rule as orc_f32_to_bf16."""
    u = _c(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def e4m3_encode(q: float) -> int:
    return int(lib().orc_e4m3_encode(float(q)))


def e4m3_decode(code: int) -> float:
    return float(lib().orc_e4m3_decode(int(code)))


def ue8m0_exponent(amax: float) -> int:
    return int(lib().orc_ue8m0_exponent(float(amax)))


def e4m3_encode_array(q) -> np.ndarray:
    """E4M3 codes (RNE) of float32 values with |q| <= 448."""
    q = _c(q, np.float32).ravel()
    out = np.zeros(q.shape, np.uint8)
    lib().orc_e4m3_encode_n(_p(q), q.size, _p(out))
    return out


def e4m3_dequant_array(codes, scale_bytes) -> np.ndarray:
    """BF16 bits of code * 2^(scale_byte - 127) (the unpack's dequantisation)."""
    codes, sb = np.broadcast_arrays(_c(codes, np.uint8), _c(scale_bytes, np.uint8))
    codes, sb = _c(codes, np.uint8).ravel(), _c(sb, np.uint8).ravel()
    out = np.zeros(codes.shape, np.uint16)
    lib().orc_e4m3_dequant_n(_p(codes), _p(sb), codes.size, _p(out))
    return out


def rms_scale_array(sumsq, eps) -> np.ndarray:
    """r = RN(1 / RN(sqrt(sumsq / 512 + eps))) elementwise."""
    sumsq, eps = np.broadcast_arrays(_c(sumsq, np.float32), _c(eps, np.float32))
    sumsq, eps = _c(sumsq, np.float32).ravel(), _c(eps, np.float32).ravel()
    out = np.zeros(sumsq.shape, np.float32)
    lib().orc_rms_scale_n(_p(sumsq), _p(eps), sumsq.size, _p(out))
    return out


# ---- rows ------------------------------------------------------------------

def _check_keep(keep_count: int) -> int:
    if keep_count not in KEEP_COUNTS:
        raise ValueError(f"keep_count must be one of {KEEP_COUNTS}")
    return keep_count


def select_keep(x, keep_count: int = KEEP) -> np.ndarray:
    """[rows, 512] float32 -> bool keep mask, keep_count per row."""
    _check_keep(keep_count)
    x = _c(x, np.float32).reshape(-1, HEAD_DIM)
    out = np.zeros(x.shape, dtype=np.uint8)
    for r in range(x.shape[0]):
        lib().orc_select_keep_k(_p(x[r]), _p(out[r]), keep_count)
    return out.astype(bool)


def normalize(x, keep, weight, eps: float) -> np.ndarray:
    """Masked RMSNorm -> bf16 bits [rows, 512] (keep=None: unmasked)."""
    x = _c(x, np.float32).reshape(-1, HEAD_DIM)
    w = _c(weight, np.float32)
    km = None if keep is None else _c(keep, np.uint8).reshape(-1, HEAD_DIM)
    out = np.zeros(x.shape, dtype=np.uint16)
    for r in range(x.shape[0]):
        lib().orc_normalize(_p(x[r]), None if km is None else _p(km[r]), _p(w), eps,
                            _p(out[r]))
    return out


def simulate_rows(x, keep, weight, eps: float) -> np.ndarray:
    """Dense codec simulation (any mask): decoded pre-RoPE bf16 bits [rows, 512]."""
    x = _c(x, np.float32).reshape(-1, HEAD_DIM)
    km = _c(keep, np.uint8).reshape(-1, HEAD_DIM)
    w = np.broadcast_to(_c(weight, np.float32), x.shape).copy()
    out = np.zeros(x.shape, dtype=np.uint16)
    lib().orc_simulate_rows(_p(x), _p(km), _p(w), eps, x.shape[0], _p(out))
    return out


def pack_rows(x, weight, eps: float, keep_count: int = KEEP):
    """Records in row order: data [rows, keep_count + 64] u8 (codes, bitmap),
    scales [rows, 8] u8, normalized bf16 bits [rows, 512], keep mask [rows, 512]."""
    _check_keep(keep_count)
    x = _c(x, np.float32).reshape(-1, HEAD_DIM)
    w = _c(weight, np.float32)
    n = x.shape[0]
    data = np.zeros((n, keep_count + 64), np.uint8)
    scales = np.zeros((n, SCALE_BYTES), np.uint8)
    normed = np.zeros((n, HEAD_DIM), np.uint16)
    keep = np.zeros((n, HEAD_DIM), np.uint8)
    for r in range(n):
        lib().orc_pack_row_k(_p(x[r]), _p(w), eps, keep_count, _p(data[r]), _p(scales[r]),
                             _p(normed[r]), _p(keep[r]))
    return data, scales, normed, keep.astype(bool)


def pack_rows_paged(x, weight, eps: float, slots, pool: np.ndarray,
                    keep_count: int = KEEP) -> np.ndarray:
    """Pack rows into a paged pool (uint8 [pages, 64 * (keep_count + 72)]) in place."""
    _check_keep(keep_count)
    x = _c(x, np.float32).reshape(-1, HEAD_DIM)
    s = _c(slots, np.int32)
    assert pool.dtype == np.uint8 and pool.flags.c_contiguous
    pages = pool.size // page_bytes(keep_count)
    lib().orc_pack_rows_paged_k(_p(x), _p(_c(weight, np.float32)), eps, keep_count, _p(s),
                                x.shape[0], _p(pool), pages)
    return pool


def unpack_row(data, scales, keep_count: int = KEEP) -> np.ndarray:
    _check_keep(keep_count)
    out = np.zeros(HEAD_DIM, np.uint16)
    lib().orc_unpack_row_k(_p(_c(data, np.uint8)), _p(_c(scales, np.uint8)), keep_count,
                           _p(out))
    return out


def unpack_rows(data, scales, keep_count: int = KEEP) -> np.ndarray:
    data = _c(data, np.uint8).reshape(-1, keep_count + 64)
    scales = _c(scales, np.uint8).reshape(-1, SCALE_BYTES)
    return np.stack([unpack_row(d, s, keep_count) for d, s in zip(data, scales)]) \
        if len(data) else np.zeros((0, HEAD_DIM), np.uint16)


def rope_tail(row_bits, freq_row) -> np.ndarray:
    """Rotate the tail of bf16 rows with freq rows ([32, 2] float32 each)."""
    rows = _c(row_bits, np.uint16).reshape(-1, HEAD_DIM).copy()
    f = _c(freq_row, np.float32).reshape(-1, ROPE_PAIRS * 2)
    for r in range(rows.shape[0]):
        lib().orc_rope_tail(_p(rows[r]), _p(f[r if f.shape[0] > 1 else 0]))
    return rows


def unpack_gather(pool, physical, raw, lengths, freqs=None, keep_count: int = KEEP) -> np.ndarray:
    """unpack_gather_bf16 on a paged pool of ``keep_count``-survivor records:
    returns bf16 bits [Q*K, 512]."""
    _check_keep(keep_count)
    pool = _c(pool, np.uint8)
    phys = np.asarray(physical, np.int32)
    raw_a = None if raw is None else np.asarray(raw, np.int32)
    lens = _c(lengths, np.int32)
    nq, nk = phys.shape
    out = np.zeros((nq * nk, HEAD_DIM), np.uint16)
    f = None if freqs is None else _c(freqs, np.float32)
    phys_c, raw_c = _c(phys, np.int32), None if raw_a is None else _c(raw_a, np.int32)
    lib().orc_unpack_gather_k(_p(pool), pool.size // page_bytes(keep_count), keep_count,
                              _p(phys_c), nk, 1, _p(raw_c), nk, 1, _p(lens), 1, nq, nk, _p(f),
                              0 if f is None else f.size // (ROPE_PAIRS * 2), _p(out))
    return out


def native_pack_row(x, weight, eps: float, freq_row=None):
    data = np.zeros(NATIVE_DATA_BYTES, np.uint8)
    scales = np.zeros(SCALE_BYTES, np.uint8)
    f = None if freq_row is None else _c(freq_row, np.float32)
    lib().orc_native_pack_row(_p(_c(x, np.float32)), _p(_c(weight, np.float32)), eps, _p(f),
                              _p(data), _p(scales))
    return data, scales


def native_pack_rows_paged(x, weight, eps, slots, positions, freqs, pool):
    x = _c(x, np.float32).reshape(-1, HEAD_DIM)
    f = None if freqs is None else _c(freqs, np.float32)
    lib().orc_native_pack_rows_paged(
        _p(x), _p(_c(weight, np.float32)), eps, _p(_c(slots, np.int32)),
        _p(_c(positions, np.int32)), _p(f), 0 if f is None else f.size // (ROPE_PAIRS * 2),
        x.shape[0], _p(pool), pool.size // NATIVE_PAGE_BYTES)
    return pool


def native_unpack_row(data, scales) -> np.ndarray:
    out = np.zeros(HEAD_DIM, np.uint16)
    lib().orc_native_unpack_row(_p(_c(data, np.uint8)), _p(_c(scales, np.uint8)), _p(out))
    return out


def sink_attention(q_bits, rows_bits, valid, sink, scale: float):
    """One token: q bf16 bits [H, 512], rows bf16 bits [K, 512] -> (out [H,512] f64, lse [H])."""
    q = _c(q_bits, np.uint16)
    rows = _c(rows_bits, np.uint16).reshape(-1, HEAD_DIM)
    heads = q.size // HEAD_DIM
    out = np.zeros((heads, HEAD_DIM), np.float64)
    lse = np.zeros(heads, np.float64)
    s = None if sink is None else _c(sink, np.float32)
    lib().orc_sink_attention(_p(q), heads, _p(rows), _p(_c(valid, np.uint8)), rows.shape[0],
                             _p(s), scale, _p(out), _p(lse))
    return out, lse


def sparse_decode(q_bits, pool, packed: bool, block_table, seqlens, indices, topk_length,
                  sink, freqs, scale: float):
    """Full decode step. q [B, Sq, H, 512] bf16 bits; indices [B, Sq, K] logical
    records; block_table [B, max_blocks]; returns (out f64 [B,Sq,H,512], lse [B,Sq,H])."""
    q = _c(q_bits, np.uint16)
    batch, q_len, heads, _ = q.shape
    idx = _c(indices, np.int32)
    topk = idx.shape[-1]
    bt = _c(block_table, np.int32)
    pool = _c(pool, np.uint8)
    page_bytes = PAGE_BYTES if packed else NATIVE_PAGE_BYTES
    out = np.zeros((batch, q_len, heads, HEAD_DIM), np.float64)
    lse = np.zeros((batch, q_len, heads), np.float64)
    f = None if freqs is None else _c(freqs, np.float32)
    lib().orc_sparse_decode(
        _p(q), batch, q_len, heads, _p(pool), pool.size // page_bytes, int(packed), _p(bt),
        bt.shape[1], bt.shape[1], _p(None if seqlens is None else _c(seqlens, np.int32)),
        _p(idx), topk, _p(None if topk_length is None else _c(topk_length, np.int32)),
        _p(None if sink is None else _c(sink, np.float32)), _p(f),
        0 if f is None else f.size // (ROPE_PAIRS * 2), scale, _p(out), _p(lse))
    return out, lse


def native_encode_row(row_bits):
    """Native record (data [576], scales [8]) of a BF16 row."""
    data = np.zeros(NATIVE_DATA_BYTES, np.uint8)
    scales = np.zeros(SCALE_BYTES, np.uint8)
    lib().orc_native_encode_row(_p(_c(row_bits, np.uint16)), _p(data), _p(scales))
    return data, scales


def packed_to_native(pool, physical, raw, lengths, freqs=None) -> np.ndarray:
    """Adapter: Native pages [ceil(Q*K/64), 37376] holding row (q, k) of the
    gather at workspace row q * K + k."""
    pool = _c(pool, np.uint8)
    phys = _c(np.asarray(physical, np.int32), np.int32)
    raw_c = None if raw is None else _c(np.asarray(raw, np.int32), np.int32)
    lens = _c(lengths, np.int32)
    nq, nk = phys.shape
    out = np.zeros(((nq * nk + 63) // 64, NATIVE_PAGE_BYTES), np.uint8)
    f = None if freqs is None else _c(freqs, np.float32)
    lib().orc_packed_to_native(_p(pool), pool.size // PAGE_BYTES, _p(phys), nk, 1, _p(raw_c), nk,
                               1, _p(lens), 1, nq, nk, _p(f),
                               0 if f is None else f.size // (ROPE_PAIRS * 2), _p(out))
    return out


def swa_gather(swa_pool, slots, length=None):
    """SWA rows of one token from a Native pool: (bf16 bits [K, 512], valid [K])."""
    pool = _c(swa_pool, np.uint8)
    sl = _c(slots, np.int32)
    rows = np.zeros((sl.size, HEAD_DIM), np.uint16)
    valid = np.zeros(sl.size, np.uint8)
    lib().orc_swa_gather(_p(pool), pool.size // NATIVE_PAGE_BYTES, _p(sl), sl.size,
                         sl.size if length is None else int(length), _p(rows), _p(valid))
    return rows, valid.astype(bool)


def sparse_decode_swa(q_bits, pool, packed: bool, block_table, seqlens, indices, topk_length,
                      swa_pool, swa_indices, swa_length, sink, freqs, scale: float):
    """Decode step attending the SWA rows (Native pool slots swa_indices
    [B, Sq, W], swa_length [B*Sq] or None) jointly with the C4 top-k."""
    q = _c(q_bits, np.uint16)
    batch, q_len, heads, _ = q.shape
    idx = _c(indices, np.int32)
    topk = idx.shape[-1]
    sidx = _c(swa_indices, np.int32)
    swa_topk = sidx.shape[-1]
    bt = _c(block_table, np.int32)
    pool = _c(pool, np.uint8)
    spool = _c(swa_pool, np.uint8)
    page_bytes = PAGE_BYTES if packed else NATIVE_PAGE_BYTES
    out = np.zeros((batch, q_len, heads, HEAD_DIM), np.float64)
    lse = np.zeros((batch, q_len, heads), np.float64)
    f = None if freqs is None else _c(freqs, np.float32)
    lib().orc_sparse_decode_swa(
        _p(q), batch, q_len, heads, _p(pool), pool.size // page_bytes, int(packed), _p(bt),
        bt.shape[1], bt.shape[1], _p(None if seqlens is None else _c(seqlens, np.int32)),
        _p(idx), topk, _p(None if topk_length is None else _c(topk_length, np.int32)),
        _p(spool), spool.size // NATIVE_PAGE_BYTES, _p(sidx), swa_topk,
        _p(None if swa_length is None else _c(swa_length, np.int32)),
        _p(None if sink is None else _c(sink, np.float32)), _p(f),
        0 if f is None else f.size // (ROPE_PAIRS * 2), scale, _p(out), _p(lse))
    return out, lse


# ---- synthetic inputs of the benchmark shapes ---------------------------------

SEED = 20260919


def synthetic_latents(rows: int, seed: int = SEED) -> np.ndarray:
    """BF16-valued float32 [rows, 512]: N(0,1) * sigma_c with per-coordinate sigma
    log-uniform on [0.1, 10] (shared across rows), seeded."""
    rng = np.random.default_rng(seed)
    sigma = np.exp(rng.uniform(np.log(0.1), np.log(10.0), HEAD_DIM)).astype(np.float32)
    x = rng.standard_normal((rows, HEAD_DIM), dtype=np.float32) * sigma
    return bf16_to_f32(f32_to_bf16_np(x))


def rope_table(positions: int, base: float = 10000.0) -> np.ndarray:
    """complex64-as-float32 [positions, 32, 2]: (cos, sin) of pos * base^(-j/32)
    with the angle rounded to float32, as torch.polar(ones, outer(t, inv_freq))."""
    inv = (1.0 / (base ** (np.arange(0, 64, 2, dtype=np.float32) / 64))).astype(np.float32)
    ang = (np.arange(positions, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    return np.stack([np.cos(ang.astype(np.float64)), np.sin(ang.astype(np.float64))],
                    -1).astype(np.float32)
