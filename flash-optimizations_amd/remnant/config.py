"""Cache-format configuration: the ``--kv-cache-format native|direct`` surface.

Mirrors the reference's configuration boundary (fork ``srt/remnant/config.py``:
``configure_cache_format(fmt, decode_impl, store_impl, keep_count=256,
layer_keep_counts=None, compression_ratios=None)``, called as in
scripts/local/serve.sh:178-183 and printed through ``packed_profile()`` at :186;
constants ``HEAD_DIM=512, NOPE_DIM=448, ROPE_DIM=64, BITMAP_WORDS=8`` at
candidate-sglang.patch:465-477; the CLI translation at
scripts/local/run-server.sh:114-133). ``direct`` selects the Packed 328-byte
records with the Direct decode reader; ``native`` the 584-byte control.

Survivor profiles (docs/agents/numerical-and-validation.md:10-17;
scripts/local/README.md:993-1013): the default Packed record keeps 256 of 512
coordinates; startup counts 64..448 in steps of 64 give ``count + 72``-byte
records, stored and reconstructed by the same HIP kernels. ``keep_count`` is
the default for every C4 layer; ``layer_keep_counts`` overrides it for single
layers, named by their layer id in the loaded model (not by their position in
the C4 pool), and every named layer must be a C4 layer -- compression ratio 4
in the model's ``compress_ratios``, which the caller passes as
``compression_ratios``. Layers of other ratios (SWA-only 0, C128 128) keep
their own layouts and get no Packed profile. As in the reference, the Direct
decode reader is 256-only: any effective non-256 count needs the reconstruct
reader (``decode_impl="reconstruct"``; the reference's spelling ``"triton"`` is
accepted for it) and is rejected with the Direct reader at configuration time,
before any pool is allocated. 512 survivors is not a profile. A rejected call
leaves the previous configuration in place.
"""

from __future__ import annotations

import argparse
import dataclasses
import re

HEAD_DIM = 512
NOPE_DIM = 448
ROPE_DIM = 64
BITMAP_WORDS = 8
KEEP_COUNT = 256
KEEP_COUNTS = tuple(range(64, 449, 64))  # training/losses.py:17 RETENTION_COUNTS
C4_RATIO = 4                              # compress_ratios entry of a C4 layer
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


def _parse_overrides(layer_keep_counts) -> tuple:
    """Per-layer overrides as sorted ((layer_id, count), ...) pairs. Accepted
    spellings: a mapping {layer: count}; (layer, count) pairs; "layer:count" or
    "layer=count" items, as a sequence or one string separated by commas or
    spaces (the launcher passes the environment string through)."""
    if layer_keep_counts is None:
        return ()
    if isinstance(layer_keep_counts, dict):
        items = list(layer_keep_counts.items())
    else:
        if isinstance(layer_keep_counts, str):
            layer_keep_counts = [t for t in re.split(r"[,\s]+", layer_keep_counts.strip()) if t]
        items = []
        for it in layer_keep_counts:
            if isinstance(it, str):
                m = re.fullmatch(r"\s*(-?\d+)\s*[:=]\s*(-?\d+)\s*", it)
                if m is None:
                    raise ValueError(f"layer keep count {it!r} is not 'layer:count'")
                items.append((int(m.group(1)), int(m.group(2))))
            else:
                try:
                    layer, count = it
                except (TypeError, ValueError):
                    raise ValueError("layer_keep_counts entries name a layer and a count "
                                     "('layer:count' or (layer, count))") from None
                items.append((layer, count))
    seen = {}
    for layer, count in items:
        if type(layer) is not int or layer < 0:
            raise ValueError(f"layer id {layer!r} must be a non-negative int")
        if layer in seen:
            raise ValueError(f"layer {layer} has two keep-count overrides")
        seen[layer] = check_keep_count(count)
    return tuple(sorted(seen.items()))


@dataclasses.dataclass(frozen=True)
class PackedProfile:
    """Resolved survivor counts of the model's C4 layers."""
    default_count: int = KEEP_COUNT
    overrides: tuple = ()             # ((layer_id, count), ...) sorted by layer id
    compression_ratios: tuple | None = None

    def c4_layers(self) -> tuple:
        """Model layer ids of the C4 layers, in C4-pool order (None: unknown)."""
        if self.compression_ratios is None:
            return None
        return tuple(i for i, r in enumerate(self.compression_ratios) if r == C4_RATIO)

    def count_for(self, layer_id: int | None = None) -> int:
        """Survivor count of model layer ``layer_id`` (a C4 layer)."""
        if layer_id is None:
            return self.default_count
        c4 = self.c4_layers()
        if c4 is not None and layer_id not in c4:
            raise ValueError(f"layer {layer_id} is not a C4 layer of the model")
        return dict(self.overrides).get(layer_id, self.default_count)

    def count_for_c4_index(self, index: int) -> int:
        """Survivor count of the C4 pool's layer ``index`` (its order in the model)."""
        c4 = self.c4_layers()
        if c4 is None:
            if self.overrides:
                raise ValueError("per-layer counts need the model's compression ratios")
            return self.default_count
        return self.count_for(c4[index])

    def counts(self) -> tuple:
        """Effective count of every C4 layer, in C4-pool order (the default alone
        when the ratios are unknown)."""
        c4 = self.c4_layers()
        if c4 is None:
            return (self.default_count,) + tuple(c for _, c in self.overrides)
        return tuple(self.count_for(i) for i in c4)

    def c4_bytes_per_row(self) -> int:
        """Packed bytes one record slot takes across all C4 layers (the
        allocator sums each layer's own record size; none is padded to 256)."""
        c4 = self.c4_layers()
        if c4 is None:
            return packed_record_bytes(self.default_count)
        return sum(packed_record_bytes(self.count_for(i)) for i in c4)


@dataclasses.dataclass(frozen=True)
class CacheFormat:
    fmt: str = "native"              # "native" | "remnant" (= direct)
    decode_impl: str = "kernel"      # "kernel" = Direct reader, "reconstruct"
    store_impl: str = "kernel"       # fused store
    profile: PackedProfile = PackedProfile()

    @property
    def packed(self) -> bool:
        return self.fmt == "remnant"

    @property
    def keep_count(self) -> int:
        return self.profile.default_count

    def keep_count_for(self, layer_id: int | None = None) -> int:
        return self.profile.count_for(layer_id)

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
                           keep_count: int = KEEP_COUNT, layer_keep_counts=None,
                           compression_ratios=None) -> CacheFormat:
    """Select the C4 cache format. ``fmt`` is ``native`` or ``remnant``
    (``direct`` is accepted as the v0.5.22 spelling of Packed + Direct).
    ``decode_impl`` is ``kernel`` (the Direct reader) or ``reconstruct`` (gather
    + dequantize + RoPE rows for a dense reader; ``triton`` is the reference's
    name for it). ``compression_ratios`` is the model's per-layer
    ``compress_ratios``; ``layer_keep_counts`` overrides the count of single
    C4 layers (see the module docstring). Survivor counts other than 256 need
    the reconstruct reader. Nothing changes when a check fails."""
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
    ratios = None
    if compression_ratios is not None:
        ratios = tuple(compression_ratios)
        if any(type(r) is not int or r < 0 for r in ratios):
            raise ValueError("compression_ratios must be non-negative ints, one per layer")
    overrides = _parse_overrides(layer_keep_counts)
    if overrides:
        if ratios is None:
            raise ValueError("Packed layer counts require model compress_ratios")
        for layer, _ in overrides:
            if layer >= len(ratios) or ratios[layer] != C4_RATIO:
                raise ValueError(f"layer {layer} is not a C4 layer of the model; overrides "
                                 "must name C4 layers")
    profile = PackedProfile(keep_count, overrides, ratios)
    if fmt == "remnant" and decode_impl == "kernel" and \
            any(c != KEEP_COUNT for c in profile.counts()):
        raise ValueError("the Direct decode reader supports exactly 256 survivors; use the "
                         "reconstruct reader for other counts")
    _current = CacheFormat(fmt, decode_impl, store_impl, profile)
    return _current


def current() -> CacheFormat:
    return _current


def packed_profile() -> PackedProfile:
    """The resolved survivor profile (what the reference's launcher prints)."""
    return _current.profile


LEGACY_FORMATS = ("native", "remnant")   # --dsv4-c4-cache-format (v0.5.18 pin)
LEGACY_DECODE_IMPLS = ("kernel", "triton")
STORE_IMPLS = ("triton", "kernel")


def add_cli_arguments(parser: argparse.ArgumentParser) -> None:
    """Register the launcher's cache flags. scripts/local/run-server.sh:114-133
    passes ``--kv-cache-format native|direct`` on the v0.5.22 pin or
    ``--dsv4-c4-cache-format native|remnant --dsv4-c4-cache-implementation
    kernel`` on v0.5.18, and on both pins the store implementation, the
    default keep count and the per-layer counts when their environment
    variables are set (STORE_IMPLEMENTATION, C4_KEEP_COUNT,
    C4_LAYER_KEEP_COUNTS)."""
    parser.add_argument("--kv-cache-format", choices=FORMATS, default=None,
                        help="native: 584-byte records; direct: Packed 328-byte records "
                             "read by the Direct decode kernel (default native)")
    parser.add_argument("--dsv4-c4-cache-format", choices=LEGACY_FORMATS, default=None,
                        help="v0.5.18 spelling of the format: remnant = Packed records")
    parser.add_argument("--dsv4-c4-cache-implementation", choices=LEGACY_DECODE_IMPLS,
                        default=None,
                        help="Packed decode reader: kernel (Direct) or triton (reconstruct)")
    parser.add_argument("--dsv4-c4-cache-store-implementation", choices=STORE_IMPLS,
                        default=None, help="Packed store (one fused kernel serves both)")
    parser.add_argument("--dsv4-c4-cache-keep-count", type=int, default=None,
                        help="survivors per C4 record for every C4 layer (64..448, step 64)")
    parser.add_argument("--dsv4-c4-cache-layer-keep-counts", default=None,
                        help="per-layer overrides, 'layer:count' items separated by commas "
                             "or spaces")


def configure_from_args(args: argparse.Namespace, compression_ratios=None) -> CacheFormat:
    """Resolve the launcher flags into one ``configure_cache_format`` call (the
    same call serve.sh:178-183 makes from the same settings). The two format
    spellings may both be given only when they agree. ``compression_ratios``
    is the model's ``compress_ratios``, needed by per-layer counts. A rejected
    profile raises ValueError before any pool exists and leaves the previous
    configuration in place."""
    fmt = getattr(args, "kv_cache_format", None)
    legacy = getattr(args, "dsv4_c4_cache_format", None)
    if fmt is not None and legacy is not None and \
            ("remnant" if fmt == "direct" else fmt) != legacy:
        raise ValueError(f"--kv-cache-format {fmt} contradicts --dsv4-c4-cache-format {legacy}")
    fmt = fmt or legacy or "native"
    keep = getattr(args, "dsv4_c4_cache_keep_count", None)
    return configure_cache_format(
        fmt, getattr(args, "dsv4_c4_cache_implementation", None) or "kernel",
        getattr(args, "dsv4_c4_cache_store_implementation", None),
        keep_count=KEEP_COUNT if keep is None else keep,
        layer_keep_counts=getattr(args, "dsv4_c4_cache_layer_keep_counts", None),
        compression_ratios=compression_ratios)
