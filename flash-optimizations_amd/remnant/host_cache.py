"""Host cache (HiCache) for latent records: a pinned-host copy of the pool and
the coordinated record transfers between it and the device pool.

Reference: SGLang's host pool ``srt/mem_cache/memory_pool_host.py`` with the
hybrid pool assembler (third_party/README.md:261): a Packed record's value,
bitmap and scale planes move together, indexed by token slots on each side.
Here a Packed record is one contiguous span, so one transfer unit carries all
three planes; Native records move their data and scale rows together.

The host pool has the device pool's geometry ([layers, pages, page_bytes],
64-record pages) in pinned memory (``torch.empty(..., pin_memory=True)``,
i.e. hipHostMalloc), which the GPU reads and writes directly: backup and
restore are one ``rm_copy_records`` launch each, on the current stream, with
the slot lists on the device.
"""

from __future__ import annotations

import torch

from . import _lib, config
from .packed import _check_cuda, _stream
from .pool import LatentPool


class HostLatentPool:
    """Pinned-host mirror of a ``LatentPool`` geometry (same format, survivor
    count and layer count; its own number of pages)."""

    def __init__(self, pages: int, layers: int = 1, fmt: str = "remnant",
                 keep_count: int = config.KEEP_COUNT, pin_memory: bool = True):
        geometry = LatentPool(0, layers, fmt, device="cpu", keep_count=keep_count)
        self.fmt = geometry.fmt
        self.keep_count = keep_count
        self.layers = layers
        self.pages = pages
        self.page_bytes = geometry.page_bytes
        self.buffer = torch.zeros((layers, pages, self.page_bytes), dtype=torch.uint8,
                                  pin_memory=pin_memory)

    @classmethod
    def like(cls, device_pool: LatentPool, pages: int | None = None, pin_memory: bool = True):
        return cls(device_pool.pages if pages is None else pages, device_pool.layers,
                   device_pool.fmt, device_pool.keep_count, pin_memory)

    @property
    def packed(self) -> bool:
        return self.fmt == "remnant"

    @property
    def rows(self) -> int:
        return self.pages * config.PAGE_RECORDS

    def layer(self, layer_id: int | None = None) -> torch.Tensor:
        return self.buffer[0 if layer_id is None else layer_id]

    # SGLang host-pool spellings
    def backup_from_device_all_layer(self, device_pool: LatentPool, host_indices: torch.Tensor,
                                     device_indices: torch.Tensor) -> None:
        """Copy records device_indices[i] -> host_indices[i] in every layer."""
        copy_records(device_pool, device_indices, self, host_indices)

    def load_to_device_per_layer(self, device_pool: LatentPool, host_indices: torch.Tensor,
                                 device_indices: torch.Tensor, layer_id: int) -> None:
        """Copy records host_indices[i] -> device_indices[i] of one layer."""
        copy_records(self, host_indices, device_pool, device_indices, layer_id=layer_id)

    def load_to_device_all_layer(self, device_pool: LatentPool, host_indices: torch.Tensor,
                                 device_indices: torch.Tensor) -> None:
        copy_records(self, host_indices, device_pool, device_indices)


def _geometry(pool):
    if not isinstance(pool, (LatentPool, HostLatentPool)):
        raise ValueError("pools must be LatentPool or HostLatentPool objects")
    return pool.fmt, pool.keep_count, pool.layers, pool.pages, pool.page_bytes


def copy_records(src, src_slots: torch.Tensor, dst, dst_slots: torch.Tensor, *,
                 layer_id: int | None = None) -> None:
    """Record transfer between two pools of one format: src_slots[i] ->
    dst_slots[i] in every layer (or only ``layer_id``). Slots outside either
    pool are skipped. Slot lists are int32 tensors on the GPU."""
    sfmt, skeep, slayers, spages, spb = _geometry(src)
    dfmt, dkeep, dlayers, dpages, dpb = _geometry(dst)
    if (sfmt, skeep) != (dfmt, dkeep):
        raise ValueError("source and destination pools hold different record formats")
    if layer_id is None and slayers != dlayers:
        raise ValueError("all-layer transfers need pools with the same layer count")
    for name, t in (("src_slots", src_slots), ("dst_slots", dst_slots)):
        if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous int32 vector")
    if src_slots.shape != dst_slots.shape:
        raise ValueError("src_slots and dst_slots must have equal length")
    n = src_slots.shape[0]
    if n == 0:
        return
    if layer_id is not None and not (0 <= layer_id < min(slayers, dlayers)):
        raise ValueError("layer_id out of range")
    _check_cuda(src_slots, dst_slots)
    for pool in (src, dst):
        # the kernel reads and writes both pools directly: device memory or
        # pinned host memory only (a pageable buffer would fault the GPU)
        if not (pool.buffer.is_cuda or pool.buffer.is_pinned()):
            raise ValueError("pools used in a transfer must live on the GPU or in pinned host "
                             "memory")
    sbuf = src.buffer if layer_id is None else src.buffer[layer_id]
    dbuf = dst.buffer if layer_id is None else dst.buffer[layer_id]
    fmt = 0 if sfmt == "remnant" else 1
    _lib.check(_lib.load().rm_copy_records(
        sbuf.data_ptr(), spages, spages * spb, src_slots.data_ptr(), dbuf.data_ptr(), dpages,
        dpages * dpb, dst_slots.data_ptr(), n, slayers if layer_id is None else 1, fmt, skeep,
        _stream()), "rm_copy_records")
