"""MI355X-native Remnant packed-KV hot path.

Store (pack), reconstruct (unpack + tail RoPE) and Direct packed sparse-MLA
decode, each a hand-written gfx950 HIP kernel reached through the C ABI in
``include/remnant_mi355x.h``. Operator names mirror the reference's fork
(``srt/remnant/packed.py``, ``sgl_kernel/flash_mla.py``) so callers can switch.
"""

from . import config
from .config import configure_cache_format, packed_profile
from .flash_mla import (get_decode_metadata, native_sparse_decode_fwd, remnant_buffers,
                        remnant_sparse_decode_fwd, sparse_decode_fwd)
from .packed import (RemnantBuffers, native_store_rows, pack_rows_fused, packed_to_native,
                     unpack_gather_bf16, unpack_rows)
from .host_cache import HostLatentPool, copy_records
from .pool import LatentPool, records_fitting

__all__ = [
    "config", "configure_cache_format", "packed_profile", "get_decode_metadata",
    "native_sparse_decode_fwd", "remnant_sparse_decode_fwd", "sparse_decode_fwd",
    "remnant_buffers", "RemnantBuffers",
    "native_store_rows", "pack_rows_fused", "packed_to_native", "unpack_gather_bf16",
    "unpack_rows",
    "LatentPool", "records_fitting", "HostLatentPool", "copy_records",
]
