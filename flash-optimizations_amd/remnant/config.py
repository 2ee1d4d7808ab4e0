"""Cache-format configuration: the ``--kv-cache-format native|direct`` surface.

Mirrors the reference's configuration boundary (fork ``srt/remnant/config.py``:
``configure_cache_format(fmt, decode_impl, store_impl, keep_count=256, ...)``,
constants ``HEAD_DIM=512, NOPE_DIM=448, ROPE_DIM=64, BITMAP_WORDS=8`` at
candidate-sglang.patch:465-477; the CLI translation at
scripts/local/run-server.sh:114-133). ``direct`` selects the Packed 328-byte
records with the Direct decode reader; ``native`` the 584-byte control.

Survivor profiles (docs/agents/numerical-and-validation.md:10-17): the
default Packed record keeps 256 of 512 coordinates; startup counts 64..448 in
steps of 64 (``keep_count``, or per C4 layer ``layer_keep_counts``) give
``count + 72``-byte records, stored and reconstructed by the same HIP kernels.
As in the reference, the Direct decode reader is 256-only: a non-256 profile
needs the reconstruct reader (``decode_impl="reconstruct"``; the reference's
spelling ``"triton"`` is accepted for it) and is rejected with the Direct
reader at configuration time, before any pool is allocated. 512 survivors is
not a profile.
"""

from __future__ import annotations

import argparse
import dataclasses

HEAD_DIM = 512
NOPE_DIM = 448
ROPE_DIM = 64
BITMAP_WORDS = 8
KEEP_COUNT = 256
KEEP_COUNTS = tuple(range(64, 449, 64))  # training/losses.py:17 RETENTION_COUNTS
PAGE_RECORDS = 64
PACKED_DATA_BYTES = KEEP_COUNT + 8 * BITMAP_WORDS            # 320
PACKED_RECORD_BYTES = PACKED_DATA_BYTES + 8                  # 328
PACKED_PAGE_BYTES = PAGE_RECORDS * PACKED_RECORD_BYTES       # 20992
NATIVE_DATA_BYTES = NOPE_DIM + 2 * ROPE_DIM                  # 576
NATIVE_RECORD_BYTES = NATIVE_DATA_BYTES + 8                  # 584
NATIVE_PAGE_BYTES = PAGE_RECORDS * NATIVE_RECORD_BYTES       # 37376

FORMATS = ("native", "direct")
DECODE_IMPLS = ("kernel", "reconstruct")


def packed_record_bytes(keep_count: int = KEEP_COUNT) -> int:
    """Bytes of a Packed record with ``keep_count`` survivors (codes, bitmap, scales)."""
    return keep_count + 8 * BITMAP_WORDS + 8


def packed_page_bytes(keep_count: int = KEEP_COUNT) -> int:
    return PAGE_RECORDS * packed_record_bytes(keep_count)


def keep_count_of_page_bytes(page_bytes: int) -> int | None:
    """Survivor count whose Packed page is ``page_bytes`` long (None if none is)."""
    for k in KEEP_COUNTS:
        if packed_page_bytes(k) == page_bytes:
            return k
    return None


def check_keep_count(keep_count) -> int:
    if type(keep_count) is not int or keep_count not in KEEP_COUNTS:
        raise ValueError(f"keep_count must be one of {KEEP_COUNTS} (512 survivors is not a "
                         "profile)")
    return keep_count


@dataclasses.dataclass(frozen=True)
class CacheFormat:
    fmt: str = "native"              # "native" | "remnant" (= direct)
    decode_impl: str = "kernel"      # "kernel" = Direct reader, "reconstruct"
    store_impl: str = "kernel"       # fused store
    keep_count: int = KEEP_COUNT
    layer_keep_counts: tuple | None = None

    @property
    def packed(self) -> bool:
        return self.fmt == "remnant"

    def keep_count_for(self, layer_id: int | None = None) -> int:
        if self.layer_keep_counts is None or layer_id is None:
            return self.keep_count
        return self.layer_keep_counts[layer_id]

    def record_bytes_for(self, layer_id: int | None = None) -> int:
        if not self.packed:
            return NATIVE_RECORD_BYTES
        return packed_record_bytes(self.keep_count_for(layer_id))

    @property
    def record_bytes(self) -> int:
        return self.record_bytes_for(None)

    @property
    def page_bytes(self) -> int:
        return PAGE_RECORDS * self.record_bytes


_current = CacheFormat()


def configure_cache_format(fmt: str, decode_impl: str = "kernel", store_impl: str | None = None,
                           keep_count: int = KEEP_COUNT, layer_keep_counts=None) -> CacheFormat:
    """Select the C4 cache format. ``fmt`` is ``native`` or ``remnant``
    (``direct`` is accepted as the v0.5.22 spelling of Packed + Direct).
    ``decode_impl`` is ``kernel`` (the Direct reader) or ``reconstruct`` (gather
    + dequantize + RoPE rows for a dense reader; ``triton`` is the reference's
    name for it). Survivor counts other than 256 need the reconstruct reader."""
    global _current
    if fmt == "direct":
        fmt = "remnant"
    if fmt not in ("native", "remnant"):
        raise ValueError(f"unsupported cache format: {fmt!r}")
    if decode_impl == "triton":
        decode_impl = "reconstruct"
    if decode_impl not in DECODE_IMPLS:
        raise ValueError(f"unsupported decode implementation: {decode_impl!r}")
    # one fused store kernel serves every profile ("triton" is the reference's
    # name for its store of non-256 profiles)
    if store_impl not in (None, "kernel", "triton"):
        raise ValueError("only the fused store kernel is built for MI355X")
    store_impl = "kernel"
    check_keep_count(keep_count)
    if layer_keep_counts is not None:
        layer_keep_counts = tuple(layer_keep_counts)
        for c in layer_keep_counts:
            check_keep_count(c)
    counts = (keep_count,) + (layer_keep_counts or ())
    if fmt == "remnant" and decode_impl == "kernel" and any(c != KEEP_COUNT for c in counts):
        raise ValueError("the Direct decode reader supports exactly 256 survivors; use the "
                         "reconstruct reader for other counts")
    _current = CacheFormat(fmt, decode_impl, store_impl, keep_count, layer_keep_counts)
    return _current


def current() -> CacheFormat:
    return _current


def packed_profile() -> dict:
    c = _current
    return {"format": c.fmt, "decode_impl": c.decode_impl, "keep_count": c.keep_count,
            "layer_keep_counts": c.layer_keep_counts, "record_bytes": c.record_bytes,
            "page_records": PAGE_RECORDS, "page_bytes": c.page_bytes}


def add_cli_arguments(parser: argparse.ArgumentParser) -> None:
    parser.add_argument("--kv-cache-format", choices=FORMATS, default="native",
                        help="native: 584-byte records; direct: Packed 328-byte records "
                             "read by the Direct decode kernel")


def configure_from_args(args: argparse.Namespace) -> CacheFormat:
    return configure_cache_format(args.kv_cache_format)
