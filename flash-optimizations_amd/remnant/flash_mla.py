"""Sparse-MLA decode operators: Direct (Packed records) and Native control.

Host-side mirror of the reference binding ``sgl_kernel/flash_mla.py::
remnant_sparse_decode_fwd`` over FlashMLA's sparse decode + combine
(third_party/README.md:260, 351-361; Dockerfile.v0.5.18:56-57) and the
metadata step that plans split-KV partitions. Output and LSE follow the
reference's decode contract (output/LSE checked at atol=rtol=0.02,
docs/report.md:20): out = softmax([logits, sink]) over the top-k rows with the
sink column dropped, V = K, lse = natural log of the full normaliser.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _lib, config
from .packed import _as_pool, _check_cuda, _stream


def get_decode_metadata(tokens: int, heads: int, topk: int) -> tuple[int, int]:
    """(num_splits, workspace_bytes) for a decode of ``tokens`` query tokens."""
    splits = ctypes.c_int32(0)
    nbytes = ctypes.c_size_t(0)
    _lib.check(_lib.load().rm_sparse_decode_workspace(tokens, heads, topk, ctypes.byref(splits),
                                                       ctypes.byref(nbytes)),
               "rm_sparse_decode_workspace")
    return splits.value, nbytes.value


def _decode(packed: bool, q, pool, block_table, indices, *, seqlens, topk_length, sink,
            freqs_cis, softmax_scale, out, lse, workspace, layer_id):
    buf, is_packed, keep = _as_pool(pool, layer_id)
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
    # a single request's table may be a broadcast view (stride 0 in dim 0)
    bt_stride = block_table.stride(0) if batch > 1 else max(block_table.stride(0),
                                                            block_table.shape[1])
    _, need = get_decode_metadata(batch * q_len, heads, topk)
    if need and (workspace is None or workspace.numel() * workspace.element_size() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _check_cuda(q, buf, block_table, indices, seqlens, topk_length, sink, freqs_cis, out, lse)
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    ws_ptr = ptr(workspace) if need else None
    ws_bytes = workspace.numel() * workspace.element_size() if need else 0
    lib = _lib.load()
    if packed:
        status = lib.rm_remnant_sparse_decode_fwd(
            q.data_ptr(), batch, q_len, heads, buf.data_ptr(), buf.shape[0],
            block_table.data_ptr(), bt_stride, block_table.shape[1], ptr(seqlens),
            indices.data_ptr(), topk, ptr(topk_length), ptr(sink), freq_ptr, freq_rows,
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
                              workspace=None, layer_id=None):
    """Direct packed sparse-MLA decode. Returns (out [B, Sq, H, 512] bf16, lse [B, Sq, H])."""
    return _decode(True, q, pool, block_table, indices, seqlens=seqlens,
                   topk_length=topk_length, sink=sink, freqs_cis=freqs_cis,
                   softmax_scale=softmax_scale, out=out, lse=lse, workspace=workspace,
                   layer_id=layer_id)


def native_sparse_decode_fwd(q, pool, block_table, indices, *, seqlens=None, topk_length=None,
                             sink=None, softmax_scale=None, out=None, lse=None, workspace=None,
                             layer_id=None):
    """Native 584-byte control decode on the same harness."""
    return _decode(False, q, pool, block_table, indices, seqlens=seqlens,
                   topk_length=topk_length, sink=sink, freqs_cis=None,
                   softmax_scale=softmax_scale, out=out, lse=lse, workspace=workspace,
                   layer_id=layer_id)


def sparse_decode_fwd(q, pool, block_table, indices, **kwargs):
    """Dispatch on the configured ``--kv-cache-format`` (native | direct)."""
    if config.current().packed:
        return remnant_sparse_decode_fwd(q, pool, block_table, indices, **kwargs)
    kwargs.pop("freqs_cis", None)
    return native_sparse_decode_fwd(q, pool, block_table, indices, **kwargs)
