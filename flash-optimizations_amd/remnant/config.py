"""Cache-format configuration: the ``--kv-cache-format native|direct`` surface.

Mirrors the reference's configuration boundary (fork ``srt/remnant/config.py``:
``configure_cache_format(fmt, decode_impl, store_impl, keep_count=256, ...)``,
constants ``HEAD_DIM=512, NOPE_DIM=448, ROPE_DIM=64, BITMAP_WORDS=8`` at
candidate-sglang.patch:465-477; the CLI translation at
scripts/local/run-server.sh:114-133). ``direct`` selects the Packed 328-byte
records with the Direct decode reader; ``native`` the 584-byte control.

This build implements the 256-survivor profile only: the reference's
optimized store, Adapter and Direct paths are 256-only as well
(docs/agents/numerical-and-validation.md:12-17); other counts are rejected at
configuration time, before any pool is allocated.
"""

from __future__ import annotations

import argparse
import dataclasses

HEAD_DIM = 512
NOPE_DIM = 448
ROPE_DIM = 64
BITMAP_WORDS = 8
KEEP_COUNT = 256
PAGE_RECORDS = 64
PACKED_DATA_BYTES = KEEP_COUNT + 8 * BITMAP_WORDS            # 320
PACKED_RECORD_BYTES = PACKED_DATA_BYTES + 8                  # 328
PACKED_PAGE_BYTES = PAGE_RECORDS * PACKED_RECORD_BYTES       # 20992
NATIVE_DATA_BYTES = NOPE_DIM + 2 * ROPE_DIM                  # 576
NATIVE_RECORD_BYTES = NATIVE_DATA_BYTES + 8                  # 584
NATIVE_PAGE_BYTES = PAGE_RECORDS * NATIVE_RECORD_BYTES       # 37376

FORMATS = ("native", "direct")


@dataclasses.dataclass(frozen=True)
class CacheFormat:
    fmt: str = "native"              # "native" | "remnant" (= direct)
    decode_impl: str = "kernel"      # Direct reader
    store_impl: str = "kernel"       # fused store
    keep_count: int = KEEP_COUNT

    @property
    def packed(self) -> bool:
        return self.fmt == "remnant"

    @property
    def record_bytes(self) -> int:
        return PACKED_RECORD_BYTES if self.packed else NATIVE_RECORD_BYTES

    @property
    def page_bytes(self) -> int:
        return PACKED_PAGE_BYTES if self.packed else NATIVE_PAGE_BYTES


_current = CacheFormat()


def configure_cache_format(fmt: str, decode_impl: str = "kernel", store_impl: str | None = None,
                           keep_count: int = KEEP_COUNT, layer_keep_counts=None) -> CacheFormat:
    """Select the C4 cache format. ``fmt`` is ``native`` or ``remnant``
    (``direct`` is accepted as the v0.5.22 spelling of Packed + Direct)."""
    global _current
    if fmt == "direct":
        fmt = "remnant"
    if fmt not in ("native", "remnant"):
        raise ValueError(f"unsupported cache format: {fmt!r}")
    if decode_impl != "kernel":
        raise ValueError("only the kernel (Direct) decode implementation is built for MI355X")
    store_impl = decode_impl if store_impl is None else store_impl
    if store_impl != "kernel":
        raise ValueError("only the kernel (fused) store implementation is built for MI355X")
    if type(keep_count) is not int or keep_count != KEEP_COUNT:
        raise ValueError("the MI355X store/Direct path supports exactly 256 survivors")
    if layer_keep_counts is not None and any(c != KEEP_COUNT for c in layer_keep_counts):
        raise ValueError("per-layer keep counts other than 256 are not supported")
    _current = CacheFormat(fmt, decode_impl, store_impl, keep_count)
    return _current


def current() -> CacheFormat:
    return _current


def packed_profile() -> dict:
    c = _current
    return {"format": c.fmt, "keep_count": c.keep_count, "record_bytes": c.record_bytes,
            "page_records": PAGE_RECORDS, "page_bytes": c.page_bytes}


def add_cli_arguments(parser: argparse.ArgumentParser) -> None:
    parser.add_argument("--kv-cache-format", choices=FORMATS, default="native",
                        help="native: 584-byte records; direct: Packed 328-byte records "
                             "read by the Direct decode kernel")


def configure_from_args(args: argparse.Namespace) -> CacheFormat:
    return configure_cache_format(args.kv_cache_format)
