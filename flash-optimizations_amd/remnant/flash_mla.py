"""Sparse-MLA decode operators: Direct (Packed records) and Native control.

Host-side mirror of the reference binding ``sgl_kernel/flash_mla.py::
remnant_sparse_decode_fwd`` over FlashMLA's sparse decode + combine
(third_party/README.md:260, 351-361; Dockerfile.v0.5.18:56-57) and the
metadata step that plans split-KV partitions. Output and LSE follow the
reference's decode contract (output/LSE checked at atol=rtol=0.02,
docs/report.md:20): out = softmax([logits, sink]) over the top-k rows with the
sink column dropped, V = K, lse = natural log of the full normaliser.

The sliding-window (SWA) rows a DeepSeek-V4 decode also attends (decode-store
timing.json ``swa_length: 64``; joint softmax over cat(swa, C4 rows) plus the
sink, training/losses.py:393-398) are passed as ``swa_pool`` (a Native pool:
584-byte records, tail stored rotated) with per-token pool slots
``swa_indices`` [B, Sq, W] (W <= 512, -1 = padding) and optional valid counts
``swa_lengths`` [B * Sq]. They are read in the same launch as the C4 list.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib, config
from .packed import RemnantBuffers, _as_pool, _as_source, _check_cuda, _plane_buffers, _stream


def get_decode_metadata(tokens: int, heads: int, topk: int, swa_topk: int = 0) -> tuple[int, int]:
    """(num_splits, workspace_bytes) for a decode of ``tokens`` query tokens
    (``swa_topk`` window rows per token add one partial slot)."""
    splits = ctypes.c_int32(0)
    nbytes = ctypes.c_size_t(0)
    _lib.check(_lib.load().rm_sparse_decode_workspace_swa(tokens, heads, topk, swa_topk,
                                                           ctypes.byref(splits),
                                                           ctypes.byref(nbytes)),
               "rm_sparse_decode_workspace_swa")
    return splits.value, nbytes.value


def _swa_args(swa_pool, swa_indices, swa_lengths, batch, q_len):
    """Validate the window inputs: (pool pages, indices, lengths, W)."""
    if swa_pool is None and swa_indices is None:
        return None, None, None, 0
    if swa_pool is None or swa_indices is None:
        raise ValueError("swa_pool and swa_indices are given together")
    sbuf, spacked, _ = _as_pool(swa_pool, None)
    if spacked:
        raise ValueError("the window rows are read from a Native pool")
    if swa_indices.dtype != torch.int32 or swa_indices.dim() != 3 \
            or swa_indices.shape[:2] != (batch, q_len) or not swa_indices.is_contiguous():
        raise ValueError("swa_indices must be a contiguous int32 [batch, q_len, W] tensor")
    width = swa_indices.shape[-1]
    if width > 512:
        raise ValueError("at most 512 window rows per token")
    if swa_lengths is not None and (swa_lengths.dtype != torch.int32
                                    or swa_lengths.numel() != batch * q_len
                                    or not swa_lengths.is_contiguous()):
        raise ValueError(f"swa_lengths must be a contiguous int32 tensor of {batch * q_len} entries")
    return sbuf, swa_indices, swa_lengths, width


def remnant_buffers(values, bitmaps=None, scales=None, *, layer_id=None) -> RemnantBuffers:
    """The Packed record source a Direct decode reads (the binding's
    ``remnant_buffers``, Dockerfile.v0.5.18:56): the reference's pool planes
    ``remnant_buffers(values, bitmaps, scales)`` (values u8 [rows, 256],
    bitmaps u64 [rows, 8], scales u8 [rows, 8]), a ``(values, bitmaps,
    scales)`` tuple, a ``LatentPool`` (with ``layer_id``) or a uint8 page
    tensor. The result is accepted wherever a pool is: by
    ``remnant_sparse_decode_fwd``, ``unpack_gather_bf16``, ``pack_rows_fused``
    and ``packed_to_native``."""
    if bitmaps is not None or scales is not None:
        if bitmaps is None or scales is None:
            raise ValueError("remnant_buffers takes values, bitmaps and scales together")
        return _plane_buffers(values, bitmaps, scales)
    src, packed, _ = _as_source(values, layer_id)
    if not packed:
        raise ValueError("remnant_buffers describes a Packed pool")
    return src


def _decode(packed: bool, q, pool, block_table, indices, *, seqlens, topk_length, sink,
            freqs_cis, softmax_scale, out, lse, workspace, layer_id, swa_pool=None,
            swa_indices=None, swa_lengths=None, rope_inv_freq=None):
    src, is_packed, keep = _as_source(pool, layer_id)
    buf = src if not is_packed else None
    if is_packed != packed:
        raise ValueError("pool format does not match the decode reader")
    if packed and keep != config.KEEP_COUNT:
        raise ValueError("the Direct decode reader reads 256-survivor records only; use "
                         "unpack_gather_bf16 for other survivor counts")
    if q.dim() != 4 or q.shape[-1] != config.HEAD_DIM or q.dtype != torch.bfloat16 \
            or not q.is_contiguous():
        raise ValueError("q must be a contiguous bfloat16 [batch, q_len, heads, 512] tensor")
    batch, q_len, heads, _ = q.shape
    if heads % 16:
        raise ValueError("heads must be a multiple of 16")
    if indices.dtype != torch.int32 or indices.dim() != 3 or indices.shape[:2] != (batch, q_len) \
            or not indices.is_contiguous():
        raise ValueError("indices must be a contiguous int32 [batch, q_len, topk] tensor")
    topk = indices.shape[-1]
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != batch \
            or block_table.stride(1) != 1:
        raise ValueError("block_table must be int32 [batch, max_blocks] with unit inner stride")
    for name, t, shape in (("seqlens", seqlens, (batch,)),
                           ("topk_length", topk_length, (batch * q_len,))):
        if t is not None and (t.dtype != torch.int32 or t.numel() != shape[0]
                              or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous int32 tensor of {shape[0]} entries")
    if sink is not None and (sink.dtype != torch.float32 or sink.shape != (heads,)
                             or not sink.is_contiguous()):
        raise ValueError("sink must be a contiguous float32 [heads] tensor")
    freq_ptr, freq_rows = None, 0
    if freqs_cis is not None:
        if not packed:
            raise ValueError("Native records store a rotated tail; freqs_cis is not used")
        if freqs_cis.dtype != torch.complex64 or not freqs_cis.is_contiguous():
            raise ValueError("freqs_cis must be a contiguous complex64 tensor")
        freq_ptr, freq_rows = freqs_cis.data_ptr(), freqs_cis.numel() // (config.ROPE_DIM // 2)
        if freq_rows == 0:
            raise ValueError("freqs_cis must hold at least one row of 32 frequencies")
    inv_ptr = None
    if rope_inv_freq is not None:
        if not packed:
            raise ValueError("Native records store a rotated tail; rope_inv_freq is not used")
        if rope_inv_freq.dtype != torch.float32 or rope_inv_freq.numel() != config.ROPE_DIM // 2 \
                or not rope_inv_freq.is_contiguous():
            raise ValueError("rope_inv_freq must be a contiguous float32 tensor of 32 inverse "
                             "frequencies")
        inv_ptr = rope_inv_freq.data_ptr()
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(config.HEAD_DIM)
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty((batch, q_len, heads), dtype=torch.float32, device=q.device)
    if out.shape != q.shape or out.dtype != torch.bfloat16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous bfloat16 tensor shaped like q")
    if lse.shape != (batch, q_len, heads) or lse.dtype != torch.float32 or not lse.is_contiguous():
        raise ValueError("lse must be a contiguous float32 [batch, q_len, heads] tensor")
    sbuf, sidx, slen, width = _swa_args(swa_pool, swa_indices, swa_lengths, batch, q_len)
    # a single request's table may be a broadcast view (stride 0 in dim 0)
    bt_stride = block_table.stride(0) if batch > 1 else max(block_table.stride(0),
                                                            block_table.shape[1])
    _, need = get_decode_metadata(batch * q_len, heads, topk, width)
    if workspace is not None and (workspace.dtype != torch.uint8 or not workspace.is_cuda
                                  or not workspace.is_contiguous()):
        raise ValueError("workspace must be a contiguous uint8 tensor on the GPU")
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    if packed and src.planes and src.rows % 2:
        raise ValueError("plane buffers need an even number of rows")
    pool_tensors = src.tensors() if packed else (buf,)
    _check_cuda(q, *pool_tensors, block_table, indices, seqlens, topk_length, sink, freqs_cis,
                rope_inv_freq, out, lse, sbuf, sidx, slen, workspace)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    ws_ptr = ptr(workspace) if need else None
    ws_bytes = workspace.numel() * workspace.element_size() if need else 0
    lib = _lib.load()
    if packed and src.planes:
        _lib.check(lib.rm_remnant_sparse_decode_planes_fwd(
            q.data_ptr(), batch, q_len, heads, src.values.data_ptr(), src.bitmaps.data_ptr(),
            src.scales.data_ptr(), src.rows, block_table.data_ptr(), bt_stride,
            block_table.shape[1], ptr(seqlens), indices.data_ptr(), topk, ptr(topk_length),
            ptr(sbuf), 0 if sbuf is None else sbuf.shape[0], ptr(sidx), width, ptr(slen),
            ptr(sink), freq_ptr, freq_rows, inv_ptr, float(softmax_scale), out.data_ptr(),
            lse.data_ptr(), ws_ptr, ws_bytes, _stream()), "rm_remnant_sparse_decode_planes_fwd")
        return out, lse
    if packed:
        buf = src.pages
    if width > 0:
        common = (q.data_ptr(), batch, q_len, heads, buf.data_ptr(), buf.shape[0],
                  block_table.data_ptr(), bt_stride, block_table.shape[1], ptr(seqlens),
                  indices.data_ptr(), topk, ptr(topk_length), sbuf.data_ptr(), sbuf.shape[0],
                  sidx.data_ptr(), width, ptr(slen), ptr(sink))
        tail = (float(softmax_scale), out.data_ptr(), lse.data_ptr(), ws_ptr, ws_bytes, _stream())
        if packed:
            _lib.check(lib.rm_remnant_sparse_decode_swa_fwd(*common, freq_ptr, freq_rows, inv_ptr,
                                                            *tail),
                       "rm_remnant_sparse_decode_swa_fwd")
        else:
            _lib.check(lib.rm_native_sparse_decode_swa_fwd(*common, *tail),
                       "rm_native_sparse_decode_swa_fwd")
    elif packed:
        status = lib.rm_remnant_sparse_decode_fwd(
            q.data_ptr(), batch, q_len, heads, buf.data_ptr(), buf.shape[0],
            block_table.data_ptr(), bt_stride, block_table.shape[1], ptr(seqlens),
            indices.data_ptr(), topk, ptr(topk_length), ptr(sink), freq_ptr, freq_rows, inv_ptr,
            float(softmax_scale), out.data_ptr(), lse.data_ptr(), ws_ptr, ws_bytes, _stream())
        _lib.check(status, "rm_remnant_sparse_decode_fwd")
    else:
        status = lib.rm_native_sparse_decode_fwd(
            q.data_ptr(), batch, q_len, heads, buf.data_ptr(), buf.shape[0],
            block_table.data_ptr(), bt_stride, block_table.shape[1], ptr(seqlens),
            indices.data_ptr(), topk, ptr(topk_length), ptr(sink), float(softmax_scale),
            out.data_ptr(), lse.data_ptr(), ws_ptr, ws_bytes, _stream())
        _lib.check(status, "rm_native_sparse_decode_fwd")
    return out, lse


def remnant_sparse_decode_fwd(q, pool, block_table, indices, *, seqlens=None, topk_length=None,
                              sink=None, freqs_cis=None, softmax_scale=None, out=None, lse=None,
                              workspace=None, layer_id=None, swa_pool=None, swa_indices=None,
                              swa_lengths=None, rope_inv_freq=None):
    """Direct packed sparse-MLA decode (with the window rows when ``swa_pool``
    is given). Returns (out [B, Sq, H, 512] bf16, lse [B, Sq, H]).

    The stored pre-RoPE tail of logical record r is rotated by row 4 r of
    ``freqs_cis`` (complex64 [P, 32]; a record with 4 r >= P contributes
    nothing). With ``rope_inv_freq`` (float32 [32], the theta_j the table is
    built from as ``polar(1, outer(positions, theta))``) the kernel computes
    those rotations from the positions instead of reading 256-byte table rows
    (within a few FP32 ulps of the table); ``freqs_cis`` may then be omitted."""
    return _decode(True, q, pool, block_table, indices, seqlens=seqlens,
                   topk_length=topk_length, sink=sink, freqs_cis=freqs_cis,
                   softmax_scale=softmax_scale, out=out, lse=lse, workspace=workspace,
                   layer_id=layer_id, swa_pool=swa_pool, swa_indices=swa_indices,
                   swa_lengths=swa_lengths, rope_inv_freq=rope_inv_freq)


def native_sparse_decode_fwd(q, pool, block_table, indices, *, seqlens=None, topk_length=None,
                             sink=None, softmax_scale=None, out=None, lse=None, workspace=None,
                             layer_id=None, swa_pool=None, swa_indices=None, swa_lengths=None):
    """Native 584-byte control decode on the same harness."""
    return _decode(False, q, pool, block_table, indices, seqlens=seqlens,
                   topk_length=topk_length, sink=sink, freqs_cis=None,
                   softmax_scale=softmax_scale, out=out, lse=lse, workspace=workspace,
                   layer_id=layer_id, swa_pool=swa_pool, swa_indices=swa_indices,
                   swa_lengths=swa_lengths)


def sparse_decode_fwd(q, pool, block_table, indices, **kwargs):
    """Dispatch on the configured ``--kv-cache-format`` (native | direct)."""
    if config.current().packed:
        return remnant_sparse_decode_fwd(q, pool, block_table, indices, **kwargs)
    kwargs.pop("freqs_cis", None)
    kwargs.pop("rope_inv_freq", None)
    return native_sparse_decode_fwd(q, pool, block_table, indices, **kwargs)
