"""Paged C4 latent pool (per-layer planes in HBM).

Reference: fork ``srt/mem_cache/deepseek_v4_memory_pool.py`` allocates per-layer
Packed planes ``values`` u8 [rows, 256], ``bitmaps`` u64 [rows, 8] and
``scales`` u8 [rows, 8] (candidate-sglang.patch:900-904) in pages of 64 C4
records (decode-store timing.json ``page_size: 64``).

MI355X layout: one contiguous uint8 buffer [layers, pages, page_bytes]. A
Packed page holds 64 contiguous 328-byte records (256 codes, 64 bitmap bytes,
8 scales), so a gathered record is one 328-byte span touching as few HBM
lines as its size allows. A Native page keeps the reference's layout: 64 data
rows of 576 bytes, then 64 scale rows of 8 bytes (the tail read
``native[page, value_base + 448 : value_base + 576]``, candidate-sglang.patch:701). The reference's planes are exposed as strided views of the
same memory (no copies), which is what a host-cache transfer or an inspection
needs.

A Packed pool may hold a survivor profile other than 256 (``keep_count`` 64..448
in steps of 64, docs/agents/numerical-and-validation.md:10-14): its records are
``keep_count + 72`` bytes with the same code/bitmap/scale order, 64 to a page.
One pool holds one profile; per-layer profiles use one pool per layer.
"""

from __future__ import annotations

import torch

from . import config


class LatentPool:
    def __init__(self, pages: int, layers: int = 1, fmt: str = "remnant", device="cuda",
                 keep_count: int = config.KEEP_COUNT):
        if fmt == "direct":
            fmt = "remnant"
        if fmt not in ("remnant", "native"):
            raise ValueError(f"unsupported cache format: {fmt!r}")
        if pages < 0 or layers < 1:
            raise ValueError("pages must be >= 0 and layers >= 1")
        config.check_keep_count(keep_count)
        if fmt == "native" and keep_count != config.KEEP_COUNT:
            raise ValueError("Native records keep every coordinate; keep_count is Packed-only")
        self.fmt = fmt
        self.pages = pages
        self.layers = layers
        self.keep_count = keep_count
        if fmt == "remnant":
            self.page_bytes = config.packed_page_bytes(keep_count)
            self.data_bytes = keep_count + 8 * config.BITMAP_WORDS
        else:
            self.page_bytes = config.NATIVE_PAGE_BYTES
            self.data_bytes = config.NATIVE_DATA_BYTES
        self.buffer = torch.zeros((layers, pages, self.page_bytes), dtype=torch.uint8,
                                  device=device)

    @property
    def packed(self) -> bool:
        return self.fmt == "remnant"

    @property
    def rows(self) -> int:
        return self.pages * config.PAGE_RECORDS

    @property
    def record_bytes(self) -> int:
        return self.data_bytes + 8

    def layer(self, layer_id: int | None = None) -> torch.Tensor:
        return self.buffer[0 if layer_id is None else layer_id]

    def _data_rows(self, layer_id):
        if self.packed:  # contiguous records: data = all but the last 8 bytes of each
            pg = self.layer(layer_id).reshape(self.pages, config.PAGE_RECORDS,
                                              self.record_bytes)
            return pg[..., : self.data_bytes]
        pg = self.layer(layer_id)[:, : config.PAGE_RECORDS * self.data_bytes]
        return pg.reshape(self.pages, config.PAGE_RECORDS, self.data_bytes)

    def scales(self, layer_id: int | None = None) -> torch.Tensor:
        """Scale plane view [pages, 64, 8] u8."""
        if self.packed:
            pg = self.layer(layer_id).reshape(self.pages, config.PAGE_RECORDS,
                                              self.record_bytes)
            return pg[..., self.data_bytes:]
        pg = self.layer(layer_id)[:, config.PAGE_RECORDS * self.data_bytes:]
        return pg.reshape(self.pages, config.PAGE_RECORDS, 8)

    def values(self, layer_id: int | None = None) -> torch.Tensor:
        """Code plane view: Packed [pages, 64, keep_count] u8, Native [pages, 64, 448] u8."""
        width = self.keep_count if self.packed else config.NOPE_DIM
        return self._data_rows(layer_id)[..., :width]

    def bitmaps(self, layer_id: int | None = None) -> torch.Tensor:
        """Bitmap plane view [pages, 64, 64] u8 (8 little-endian MSB-first uint64 words)."""
        if not self.packed:
            raise ValueError("Native records carry no bitmap")
        return self._data_rows(layer_id)[..., self.keep_count:self.data_bytes]

    def records(self, slots: torch.Tensor, layer_id: int | None = None) -> torch.Tensor:
        """Logical records [n, record_bytes] (data row + scale row) for pool slots."""
        slots = slots.to(torch.long)
        page, row = slots // config.PAGE_RECORDS, slots % config.PAGE_RECORDS
        data = self._data_rows(layer_id)[page, row]
        return torch.cat([data, self.scales(layer_id)[page, row]], dim=-1)

    def capacity_records(self) -> int:
        return self.rows

    def nbytes(self) -> int:
        return self.buffer.numel()


def records_fitting(nbytes: int, fmt: str = "remnant", keep_count: int = config.KEEP_COUNT) -> int:
    """Records (whole pages of 64) that fit in ``nbytes`` of HBM."""
    fmt = "remnant" if fmt == "direct" else fmt
    page = config.packed_page_bytes(keep_count) if fmt == "remnant" else config.NATIVE_PAGE_BYTES
    return (nbytes // page) * config.PAGE_RECORDS
