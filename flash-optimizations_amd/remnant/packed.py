"""Packed store and reconstruct operators (torch tensors in, HIP kernels out).

Host-side mirror of the reference's fork ``srt/remnant/packed.py``:
``pack_rows_fused`` (fused Triton store, third_party/README.md:257) and
``unpack_gather_bf16`` (candidate-sglang.patch:427-480): same names, argument
meaning, ``ValueError``/``TypeError`` behaviour and empty-input rule (return
``output`` untouched, launch nothing). Work runs on the current HIP stream,
asynchronously, through the C ABI in include/remnant_mi355x.h.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib, config
from .pool import LatentPool


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class RemnantBuffers(NamedTuple):
    """A Packed record source resolved for the kernels: contiguous pages
    (``pages`` u8 [pages, 64 * (K + 72)]) or the reference's three planes
    (``values`` u8 [rows, K], ``bitmaps`` u64 [rows, 8], ``scales`` u8 [rows, 8];
    candidate-sglang.patch:900-904), with the survivor count and record rows."""
    pages: torch.Tensor | None
    values: torch.Tensor | None
    bitmaps: torch.Tensor | None
    scales: torch.Tensor | None
    keep_count: int
    rows: int

    @property
    def planes(self) -> bool:
        return self.pages is None

    def tensors(self) -> tuple:
        return (self.pages,) if self.pages is not None else (self.values, self.bitmaps,
                                                             self.scales)


def _plane_buffers(values, bitmaps, scales) -> RemnantBuffers:
    """Validate the reference's plane tuple (values, bitmaps, scales)."""
    for t in (values, bitmaps, scales):
        if not isinstance(t, torch.Tensor):
            raise ValueError("packed buffers must be (values, bitmaps, scales) tensors")
    if values.dtype != torch.uint8 or values.dim() != 2 or not values.is_contiguous():
        raise ValueError("values must be a contiguous uint8 [rows, keep_count] tensor")
    rows, keep = values.shape
    if keep not in config.KEEP_COUNTS:
        raise ValueError(f"values width {keep} is not a survivor profile {config.KEEP_COUNTS}")
    if bitmaps.dtype in (torch.uint64, torch.int64):
        bshape = (rows, config.BITMAP_WORDS)
    elif bitmaps.dtype == torch.uint8:
        bshape = (rows, 8 * config.BITMAP_WORDS)
    else:
        raise ValueError("bitmaps must be uint64 [rows, 8] (or its uint8 [rows, 64] view)")
    if tuple(bitmaps.shape) != bshape or not bitmaps.is_contiguous():
        raise ValueError(f"bitmaps must be a contiguous [rows, 8] uint64 tensor of {rows} rows")
    if scales.dtype != torch.uint8 or tuple(scales.shape) != (rows, 8) or not scales.is_contiguous():
        raise ValueError(f"scales must be a contiguous uint8 [rows, 8] tensor of {rows} rows")
    if not (values.device == bitmaps.device == scales.device):
        raise ValueError("values, bitmaps and scales must share a device")
    return RemnantBuffers(None, values, bitmaps, scales, keep, rows)


def _as_source(buffers, layer_id) -> tuple[RemnantBuffers | torch.Tensor, bool, int]:
    """Resolve the packed_buffers argument: a LatentPool (+ layer), a raw uint8
    page tensor [pages, page_bytes] (its page size names its format), the
    reference's plane tuple (values, bitmaps, scales) or RemnantBuffers.
    Returns (source, packed, survivor count); a Native source is its page tensor."""
    if isinstance(buffers, RemnantBuffers):
        return buffers, True, buffers.keep_count
    if isinstance(buffers, (tuple, list)) and not isinstance(buffers, torch.Tensor):
        if len(buffers) != 3:
            raise ValueError("plane buffers are (values, bitmaps, scales)")
        b = _plane_buffers(*buffers)
        return b, True, b.keep_count
    if isinstance(buffers, LatentPool):
        pages = buffers.layer(layer_id)
        if not buffers.packed:
            return pages, False, config.KEEP_COUNT
        return (RemnantBuffers(pages, None, None, None, buffers.keep_count,
                               pages.shape[0] * config.PAGE_RECORDS), True, buffers.keep_count)
    if isinstance(buffers, torch.Tensor):
        if buffers.dtype != torch.uint8 or buffers.dim() != 2 or not buffers.is_contiguous():
            raise ValueError("pool must be a contiguous uint8 [pages, page_bytes] tensor")
        if buffers.shape[1] == config.NATIVE_PAGE_BYTES:
            return buffers, False, config.KEEP_COUNT
        keep = config.keep_count_of_page_bytes(buffers.shape[1])
        if keep is not None:
            return (RemnantBuffers(buffers, None, None, None, keep,
                                   buffers.shape[0] * config.PAGE_RECORDS), True, keep)
        raise ValueError(f"unknown page size {buffers.shape[1]}")
    raise ValueError("packed_buffers must be a LatentPool, a uint8 page tensor or the "
                     "(values, bitmaps, scales) planes")


def _as_pool(buffers, layer_id) -> tuple[torch.Tensor, bool, int]:
    """Page-tensor form of a pool (contiguous layouts only): (pages, packed, keep)."""
    src, packed, keep = _as_source(buffers, layer_id)
    if packed:
        if src.planes:
            raise ValueError("this operator reads contiguous pages, not plane buffers")
        return src.pages, True, keep
    return src, False, keep


def _check_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("tensors must live on the GPU")


def pack_rows_fused(x: torch.Tensor, weight: torch.Tensor, eps: float, loc: torch.Tensor,
                    pool, *, layer_id: int | None = None) -> None:
    """Pack raw C4 rows ``x`` [n, 512] (float32 compressor output or bfloat16)
    into Packed records at pool slots ``loc`` [n] int32 (slots outside the
    pool are skipped). The pool's survivor count (256 by default) sets how many
    coordinates each record keeps. ``pool`` may also be the reference's plane
    buffers (values, bitmaps, scales): slot s is then row s of each plane."""
    src, packed, keep = _as_source(pool, layer_id)
    if not packed:
        raise ValueError("pack_rows_fused writes the Packed (remnant) format")
    if x.dim() != 2 or x.shape[-1] != config.HEAD_DIM or x.stride(-1) != 1:
        raise ValueError("x must be [rows, 512] with unit inner stride")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("x must be float32 or bfloat16")
    if loc.dtype != torch.int32 or loc.shape != (x.shape[0],) or not loc.is_contiguous():
        raise ValueError("loc must be a contiguous int32 [rows] tensor")
    if weight.dtype != torch.float32 or weight.shape != (config.HEAD_DIM,) or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous float32 [512] tensor")
    if x.shape[0] == 0:
        return
    _check_cuda(x, weight, loc, *src.tensors())
    dtype = 1 if x.dtype == torch.bfloat16 else 0
    lib = _lib.load()
    if src.planes:
        _lib.check(lib.rm_pack_rows_planes(
            x.data_ptr(), dtype, x.stride(0), weight.data_ptr(), float(eps), loc.data_ptr(),
            x.shape[0], src.values.data_ptr(), src.bitmaps.data_ptr(), src.scales.data_ptr(),
            src.rows, keep, _stream()), "rm_pack_rows_planes")
    else:
        _lib.check(lib.rm_pack_rows_k(
            x.data_ptr(), dtype, x.stride(0), weight.data_ptr(), float(eps), loc.data_ptr(),
            x.shape[0], src.pages.data_ptr(), src.pages.shape[0], keep, _stream()),
            "rm_pack_rows_k")


def native_store_rows(x: torch.Tensor, weight: torch.Tensor, eps: float, loc: torch.Tensor,
                      positions: torch.Tensor | None, freqs_cis: torch.Tensor | None, pool,
                      *, layer_id: int | None = None) -> None:
    """Native 584-byte control store (unpruned RMSNorm, tail rotated with
    frequency row positions * 4)."""
    buf, packed, _ = _as_pool(pool, layer_id)
    if packed:
        raise ValueError("native_store_rows writes the Native format")
    if x.dim() != 2 or x.shape[-1] != config.HEAD_DIM or x.stride(-1) != 1:
        raise ValueError("x must be [rows, 512] with unit inner stride")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("x must be float32 or bfloat16")
    if loc.dtype != torch.int32 or loc.shape != (x.shape[0],) or not loc.is_contiguous():
        raise ValueError("loc must be a contiguous int32 [rows] tensor")
    if weight.dtype != torch.float32 or weight.shape != (config.HEAD_DIM,) or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous float32 [512] tensor")
    freq_ptr, freq_rows, pos_ptr = None, 0, None
    if freqs_cis is not None:
        if freqs_cis.dtype != torch.complex64 or not freqs_cis.is_contiguous():
            raise ValueError("freqs_cis must be a contiguous complex64 tensor")
        if positions is None or positions.dtype != torch.int32 or positions.shape != loc.shape \
                or not positions.is_contiguous():
            raise ValueError("positions must be a contiguous int32 [rows] tensor when freqs_cis "
                             "is given")
        freq_ptr = freqs_cis.data_ptr()
        freq_rows = freqs_cis.numel() // (config.ROPE_DIM // 2)
        pos_ptr = positions.data_ptr()
    if x.shape[0] == 0:
        return
    _check_cuda(x, weight, loc, buf, freqs_cis, positions if freqs_cis is not None else None)
    dtype = 1 if x.dtype == torch.bfloat16 else 0
    _lib.check(_lib.load().rm_native_store_rows(
        x.data_ptr(), dtype, x.stride(0), weight.data_ptr(), float(eps),
        loc.data_ptr(), pos_ptr, freq_ptr, freq_rows, x.shape[0], buf.data_ptr(),
        buf.shape[0], _stream()), "rm_native_store_rows")


def unpack_gather_bf16(packed_buffers, physical_indices: torch.Tensor,
                       raw_indices: torch.Tensor | None, topk_lengths: torch.Tensor,
                       freqs_cis: torch.Tensor | None, output: torch.Tensor, *,
                       layer_id: int | None = None, fused_rope: bool = False) -> torch.Tensor:
    """Gather selected records, dequantize, zero-fill and apply tail RoPE.

    ``packed_buffers`` is a ``LatentPool``, a uint8 page tensor or the
    reference's plane buffers (values, bitmaps, scales) as its Packed pool
    allocates them (candidate-sglang.patch:900-904); the planes are read in
    place. physical/raw indices are int32 [queries, k] (any strides); physical
    entries address pool slots (plane rows), raw entries logical C4 rows
    (frequency row raw * 4).
    Lengths are int32 [queries]. ``output`` is caller-owned contiguous BF16 with
    at least queries * k rows of 512. Invalid/padded selections produce zero
    rows. ``freqs_cis=None`` returns pre-RoPE rows. The MI355X kernel always
    reads in one pass and rounds dequantized values to BF16 before rotating, so
    ``fused_rope`` True and False give the same bytes (the reference requires
    its fused and split readers to agree bitwise, candidate-sglang.patch:682-686).
    """
    if type(fused_rope) is not bool:
        raise TypeError("fused_rope must be a bool")
    src, packed, keep = _as_source(packed_buffers, layer_id)
    if not packed:
        raise ValueError("unpack_gather_bf16 reads the Packed (remnant) format")
    if raw_indices is not None and physical_indices.shape != raw_indices.shape:
        raise ValueError("physical_indices and raw_indices must have equal shape")
    if physical_indices.dim() != 2:
        raise ValueError("indices must be [queries, k]")
    for name, t in (("physical_indices", physical_indices), ("raw_indices", raw_indices),
                    ("topk_lengths", topk_lengths)):
        if t is not None and t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    n_queries, selected_k = physical_indices.shape
    if topk_lengths.dim() != 1 or topk_lengths.shape[0] != n_queries:
        raise ValueError("topk_lengths must be [queries]")
    if output.dtype != torch.bfloat16 or not output.is_contiguous() or output.dim() != 2 \
            or output.shape[-1] != config.HEAD_DIM:
        raise ValueError("output must be a contiguous bfloat16 [rows, 512] tensor")
    if output.shape[0] < n_queries * selected_k:
        raise ValueError("output has fewer rows than queries * k")
    freq_ptr, freq_rows = None, 0
    if freqs_cis is not None:
        if not freqs_cis.is_complex() or not freqs_cis.is_contiguous():
            raise ValueError("freqs_cis must be a contiguous complex tensor")
        if freqs_cis.dtype != torch.complex64:
            raise ValueError("freqs_cis must be complex64")
        if raw_indices is None:
            raise ValueError("raw_indices are required with freqs_cis")
        freq_ptr = freqs_cis.data_ptr()
        freq_rows = freqs_cis.numel() // (config.ROPE_DIM // 2)
    if n_queries * selected_k == 0:
        return output
    _check_cuda(*src.tensors(), physical_indices, raw_indices, topk_lengths, output, freqs_cis)
    index_args = (physical_indices.data_ptr(), physical_indices.stride(0),
                  physical_indices.stride(1),
                  None if raw_indices is None else raw_indices.data_ptr(),
                  0 if raw_indices is None else raw_indices.stride(0),
                  0 if raw_indices is None else raw_indices.stride(1), topk_lengths.data_ptr(),
                  topk_lengths.stride(0), n_queries, selected_k, freq_ptr, freq_rows,
                  output.data_ptr(), _stream())
    lib = _lib.load()
    if src.planes:
        _lib.check(lib.rm_unpack_gather_bf16_planes(
            src.values.data_ptr(), src.bitmaps.data_ptr(), src.scales.data_ptr(), src.rows, keep,
            *index_args), "rm_unpack_gather_bf16_planes")
    else:
        _lib.check(lib.rm_unpack_gather_bf16_k(src.pages.data_ptr(), src.pages.shape[0], keep,
                                               *index_args), "rm_unpack_gather_bf16_k")
    return output


def packed_to_native(packed_buffers, physical_indices: torch.Tensor,
                     raw_indices: torch.Tensor | None, topk_lengths: torch.Tensor,
                     freqs_cis: torch.Tensor | None, native_output, *,
                     layer_id: int | None = None):
    """Adapter (the reference's CUDA Adapter, third_party/README.md:259): the
    rows ``unpack_gather_bf16`` would return, each written as a Native 584-byte
    record at workspace row q * k_sel + k of ``native_output`` (a Native
    ``LatentPool`` or uint8 [pages, 37376] tensor with >= ceil(rows / 64)
    pages), for a stock Native decode to read. Invalid selections become the
    Native encoding of a zero row. 256-survivor pools only, as in the reference."""
    src, packed, keep = _as_source(packed_buffers, layer_id)
    if not packed:
        raise ValueError("packed_to_native reads the Packed (remnant) format")
    if keep != config.KEEP_COUNT:
        raise ValueError("the Adapter reads 256-survivor records only")
    nbuf, npacked, _ = _as_pool(native_output, None)
    if npacked:
        raise ValueError("native_output must be a Native pool")
    if raw_indices is not None and physical_indices.shape != raw_indices.shape:
        raise ValueError("physical_indices and raw_indices must have equal shape")
    if physical_indices.dim() != 2:
        raise ValueError("indices must be [queries, k]")
    for name, t in (("physical_indices", physical_indices), ("raw_indices", raw_indices),
                    ("topk_lengths", topk_lengths)):
        if t is not None and t.dtype != torch.int32:
            raise ValueError(f"{name} must be int32")
    n_queries, selected_k = physical_indices.shape
    if topk_lengths.dim() != 1 or topk_lengths.shape[0] != n_queries:
        raise ValueError("topk_lengths must be [queries]")
    if n_queries * selected_k > nbuf.shape[0] * config.PAGE_RECORDS:
        raise ValueError("native_output has fewer records than queries * k")
    freq_ptr, freq_rows = None, 0
    if freqs_cis is not None:
        if freqs_cis.dtype != torch.complex64 or not freqs_cis.is_contiguous():
            raise ValueError("freqs_cis must be a contiguous complex64 tensor")
        if raw_indices is None:
            raise ValueError("raw_indices are required with freqs_cis")
        freq_ptr = freqs_cis.data_ptr()
        freq_rows = freqs_cis.numel() // (config.ROPE_DIM // 2)
    if n_queries * selected_k == 0:
        return native_output
    _check_cuda(*src.tensors(), physical_indices, raw_indices, topk_lengths, nbuf, freqs_cis)
    index_args = (physical_indices.data_ptr(), physical_indices.stride(0),
                  physical_indices.stride(1),
                  None if raw_indices is None else raw_indices.data_ptr(),
                  0 if raw_indices is None else raw_indices.stride(0),
                  0 if raw_indices is None else raw_indices.stride(1), topk_lengths.data_ptr(),
                  topk_lengths.stride(0), n_queries, selected_k, freq_ptr, freq_rows,
                  nbuf.data_ptr(), nbuf.shape[0], _stream())
    lib = _lib.load()
    if src.planes:
        _lib.check(lib.rm_packed_to_native_planes(
            src.values.data_ptr(), src.bitmaps.data_ptr(), src.scales.data_ptr(), src.rows,
            *index_args), "rm_packed_to_native_planes")
    else:
        _lib.check(lib.rm_packed_to_native(src.pages.data_ptr(), src.pages.shape[0],
                                           *index_args), "rm_packed_to_native")
    return native_output


def unpack_rows(pool, slots: torch.Tensor, *, layer_id: int | None = None) -> torch.Tensor:
    """Pre-RoPE BF16 rows [n, 512] of pool slots (exact dequantization)."""
    slots = slots.to(torch.int32).reshape(1, -1).contiguous()
    out = torch.empty((slots.shape[1], config.HEAD_DIM), dtype=torch.bfloat16,
                      device=slots.device)
    lengths = torch.full((1,), slots.shape[1], dtype=torch.int32, device=slots.device)
    return unpack_gather_bf16(pool, slots, None, lengths, None, out, layer_id=layer_id)
