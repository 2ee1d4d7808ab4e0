"""CPU tests of the boundary: the C-ABI library loads and exports every symbol
include/remnant_mi355x.h declares, rejects bad arguments with the documented
status codes before touching the GPU, and the Python host layer mirrors the
reference's validation and empty-input behaviour (candidate-sglang.patch:
435-453, 918-930). No kernel is launched here."""

import ctypes
import os
import re

import pytest
import torch

import remnant
from remnant import _lib, config

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "remnant_mi355x.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*int\s+(rm_\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 7
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES)
    assert lib.rm_version() >= 100


def test_header_geometry_matches_python_config():
    text = open(HEADER).read()
    consts = dict(re.findall(r"#define (RM_\w+) (\d+)", text))
    assert int(consts["RM_PACKED_RECORD_BYTES"]) == config.PACKED_RECORD_BYTES == 328
    assert int(consts["RM_NATIVE_RECORD_BYTES"]) == config.NATIVE_RECORD_BYTES == 584
    assert int(consts["RM_PACKED_PAGE_BYTES"]) == config.PACKED_PAGE_BYTES == 64 * 328
    assert int(consts["RM_NATIVE_PAGE_BYTES"]) == config.NATIVE_PAGE_BYTES == 64 * 584
    assert int(consts["RM_KEEP_COUNT"]) + 64 + 8 == 328


def buf(n=64, align=256):
    raw = ctypes.create_string_buffer(n + align)
    addr = ctypes.addressof(raw)
    return raw, addr + (-addr % align)


def test_capi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    keep = []
    _, x = buf(4096)
    _, w = buf(2048)
    _, s = buf(64)
    _, pool = buf(21000)
    keep += [x, w, s, pool]
    assert lib.rm_pack_rows(x, 1, 512, w, 1e-6, s, 0, pool, 1, None) == 0  # empty: no launch
    assert lib.rm_pack_rows(x, 1, 512, w, 1e-6, s, -1, pool, 1, None) == -2
    assert lib.rm_pack_rows(None, 1, 512, w, 1e-6, s, 4, pool, 1, None) == -1
    assert lib.rm_pack_rows(x, 7, 512, w, 1e-6, s, 4, pool, 1, None) == -4
    assert lib.rm_pack_rows(x + 2, 1, 512, w, 1e-6, s, 4, pool, 1, None) == -3
    assert lib.rm_pack_rows(x, 1, 100, w, 1e-6, s, 4, pool, 1, None) == -2
    assert lib.rm_native_store_rows(x, 0, 512, w, 1e-6, s, None, w, 8, 4, pool, 1, None) == -1
    assert lib.rm_unpack_gather_bf16(pool, 1, s, 1, 1, None, 0, 0, s, 1, 0, 5, None, 0, x,
                                     None) == 0
    assert lib.rm_unpack_gather_bf16(pool, 1, s, 1, 1, None, 0, 0, s, 1, 2, 5, w, 8, x,
                                     None) == -1  # freqs without raw
    assert lib.rm_unpack_gather_bf16(pool, 1, s, 1, 1, None, 0, 0, s, 1, 2, 5, None, 0, x + 8,
                                     None) == -3
    for bad in (0, 32, 200, 512, -64):  # survivor counts outside the profiles
        assert lib.rm_pack_rows_k(x, 1, 512, w, 1e-6, s, 4, pool, 1, bad, None) == -2
        assert lib.rm_unpack_gather_bf16_k(pool, 1, bad, s, 1, 1, None, 0, 0, s, 1, 2, 5, None,
                                           0, x, None) == -2
    assert lib.rm_pack_rows_k(x, 1, 512, w, 1e-6, s, 0, pool, 1, 448, None) == 0
    assert lib.rm_pack_rows_k(None, 1, 512, w, 1e-6, s, 4, pool, 1, 64, None) == -1
    assert lib.rm_unpack_gather_bf16_k(pool, 1, 192, s, 1, 1, None, 0, 0, s, 1, 0, 5, None, 0,
                                       x, None) == 0
    args = [x, 1, 1, 17, pool, 1, s, 4, 4, None, s, 8, None, None, None, 0, None, 0.1, x, w,
            None, 0, None]
    assert lib.rm_remnant_sparse_decode_fwd(*args) == -2  # 17 heads
    args[3] = 16
    args[8] = 9  # max_blocks beyond the table stride
    assert lib.rm_remnant_sparse_decode_fwd(*args) == -2
    args[8] = 4
    args[11] = 64  # top-k 64 at batch 1 plans 4 splits
    assert lib.rm_remnant_sparse_decode_fwd(*args) == -5  # split plan needs a workspace
    assert lib.rm_native_sparse_decode_fwd(x, 0, 1, 16, pool, 1, s, 4, 4, None, s, 8, None,
                                           None, 0.1, x, w, None, 0, None) == 0
    args[11] = 32769  # top-k beyond 64 splits of 512 records
    assert lib.rm_remnant_sparse_decode_fwd(*args) == -2
    args[11] = 8
    args[16] = w + 4  # inverse frequencies not 16-byte aligned
    assert lib.rm_remnant_sparse_decode_fwd(*args) == -3
    args[16] = None
    splits, nbytes = ctypes.c_int32(), ctypes.c_size_t()
    assert lib.rm_sparse_decode_workspace(1, 16, 32769, ctypes.byref(splits),
                                          ctypes.byref(nbytes)) == -2
    assert lib.rm_sparse_decode_workspace(1, 16, 32768, ctypes.byref(splits),
                                          ctypes.byref(nbytes)) == 0 and splits.value == 64
    # window rows take one partial slot: the C4 list keeps 63 splits of 512
    assert lib.rm_sparse_decode_workspace_swa(1, 16, 32256, 64, ctypes.byref(splits),
                                              ctypes.byref(nbytes)) == 0 and splits.value == 64
    assert lib.rm_sparse_decode_workspace_swa(1, 16, 32257, 64, ctypes.byref(splits),
                                              ctypes.byref(nbytes)) == -2
    assert lib.rm_sparse_decode_workspace_swa(1, 16, 512, 513, ctypes.byref(splits),
                                              ctypes.byref(nbytes)) == -2
    assert lib.rm_sparse_decode_workspace_swa(300, 16, 512, 64, ctypes.byref(splits),
                                              ctypes.byref(nbytes)) == 0
    assert splits.value == 2 and nbytes.value == 300 * 2 * 16 * 513 * 4
    swa_args = [x, 1, 1, 16, pool, 1, s, 4, 4, None, s, 8, None, None, 0, s, 8, None, None,
                None, 0, None, 0.1, x, w, None, 0, None]
    assert lib.rm_remnant_sparse_decode_swa_fwd(*swa_args) == -1  # window slots without a pool
    swa_args[13], swa_args[14] = pool + 8, 1
    assert lib.rm_remnant_sparse_decode_swa_fwd(*swa_args) == -3  # unaligned window pool
    swa_args[13], swa_args[16] = pool, 600
    assert lib.rm_remnant_sparse_decode_swa_fwd(*swa_args) == -2  # window above 512


def test_decode_split_plan():
    for tokens, topk in ((1, 2048), (64, 2048), (256, 2048), (3, 10), (1000, 16)):
        splits, nbytes = remnant.get_decode_metadata(tokens, 16, topk)
        assert 1 <= splits <= max(1, -(-topk // 16))
        assert nbytes == (0 if splits == 1 else tokens * splits * 16 * 513 * 4)
    assert remnant.get_decode_metadata(1, 16, 2048)[0] > 1  # batch 1 spreads over CUs
    with pytest.raises(RuntimeError):
        remnant.get_decode_metadata(1, 17, 64)


def test_unpack_gather_host_validation_mirrors_reference():
    pool = torch.zeros((1, config.PACKED_PAGE_BYTES), dtype=torch.uint8)
    index = torch.zeros((1, 1), dtype=torch.int32)
    lengths = torch.ones(1, dtype=torch.int32)
    freqs = torch.ones((16, 32), dtype=torch.complex64)
    output = torch.full((1, 512), -91.0, dtype=torch.bfloat16)
    for invalid in (1, 0, "fused", None):
        with pytest.raises(TypeError, match="fused_rope must be a bool"):
            remnant.unpack_gather_bf16(pool, index, index, lengths, freqs, output,
                                       fused_rope=invalid)
    with pytest.raises(ValueError, match="equal shape"):
        remnant.unpack_gather_bf16(pool, index, index[:, :0], lengths, freqs, output)
    with pytest.raises(ValueError, match="complex"):
        remnant.unpack_gather_bf16(pool, index, index, lengths, torch.ones(16, 64), output)
    with pytest.raises(ValueError, match="int32"):
        remnant.unpack_gather_bf16(pool, index.long(), index.long(), lengths, freqs, output)
    # empty selections return the untouched output and launch nothing
    for physical, raw, active in ((index[:0], index[:0], lengths[:0]),
                                  (index[:, :0], index[:, :0], lengths)):
        got = remnant.unpack_gather_bf16(pool, physical, raw, active, freqs, output,
                                         fused_rope=True)
        assert got is output and torch.all(output == -91)
    with pytest.raises(ValueError, match="GPU"):
        remnant.unpack_gather_bf16(pool, index, index, lengths, freqs, output)


def test_pack_and_decode_host_validation():
    pool = remnant.LatentPool(1, device="cpu")
    x = torch.zeros((2, 512))
    loc = torch.zeros(2, dtype=torch.int32)
    w = torch.ones(512)
    with pytest.raises(ValueError, match="loc"):
        remnant.pack_rows_fused(x, w, 1e-6, loc.long(), pool)
    with pytest.raises(ValueError, match="float32 or bfloat16"):
        remnant.pack_rows_fused(x.half(), w, 1e-6, loc, pool)
    remnant.pack_rows_fused(x[:0], w, 1e-6, loc[:0], pool)  # empty: nothing happens
    native = remnant.LatentPool(1, fmt="native", device="cpu")
    with pytest.raises(ValueError, match="Packed"):
        remnant.pack_rows_fused(x, w, 1e-6, loc, native)
    q = torch.zeros((1, 1, 16, 512), dtype=torch.bfloat16)
    bt = torch.zeros((1, 1), dtype=torch.int32)
    idx = torch.zeros((1, 1, 4), dtype=torch.int32)
    with pytest.raises(ValueError, match="format"):
        remnant.remnant_sparse_decode_fwd(q, native, bt, idx)
    with pytest.raises(ValueError, match="multiple of 16"):
        remnant.remnant_sparse_decode_fwd(q[:, :, :8], pool, bt, idx)
    with pytest.raises(ValueError, match="freqs_cis"):
        remnant.flash_mla._decode(False, q, native, bt, idx, seqlens=None, topk_length=None,
                                  sink=None, freqs_cis=torch.ones(4, 32, dtype=torch.complex64),
                                  softmax_scale=None, out=None, lse=None, workspace=None,
                                  layer_id=None)


def test_cache_format_configuration():
    ratios = (0, 128, 4, 128, 4, 0, 4)  # C4 layers 2, 4, 6
    try:
        assert remnant.configure_cache_format("direct").packed
        assert remnant.configure_cache_format("direct").record_bytes == 328
        assert not remnant.configure_cache_format("native").packed
        assert config.current().record_bytes == 584
        # the Direct reader is 256-only; 512 and non-multiples of 64 are no profile
        # (docs/agents/numerical-and-validation.md:11-16)
        for bad in (dict(fmt="fp4"), dict(fmt="remnant", keep_count=192),
                    dict(fmt="remnant", layer_keep_counts={2: 128}, compression_ratios=ratios),
                    dict(fmt="remnant", decode_impl="triton", keep_count=512),
                    dict(fmt="remnant", decode_impl="triton", keep_count=200),
                    dict(fmt="remnant", decode_impl="triton", keep_count=192.0),
                    dict(fmt="remnant", decode_impl="flashinfer"),
                    dict(fmt="remnant", decode_impl="triton", layer_keep_counts={2: 512},
                         compression_ratios=ratios)):
            with pytest.raises(ValueError):
                remnant.configure_cache_format(**bad)
        for count in config.KEEP_COUNTS:
            c = remnant.configure_cache_format("remnant", "triton", keep_count=count)
            assert c.decode_impl == "reconstruct" and c.record_bytes == count + 72
            assert c.page_bytes == 64 * (count + 72)
            assert remnant.packed_profile().default_count == count
        import argparse
        p = argparse.ArgumentParser()
        config.add_cli_arguments(p)
        assert config.configure_from_args(p.parse_args(["--kv-cache-format", "direct"])).packed
        with pytest.raises(SystemExit):
            p.parse_args(["--kv-cache-format", "remnant256"])
    finally:
        remnant.configure_cache_format("native")


def _launcher_args(pin, mode, env):
    """The cache flags scripts/local/run-server.sh:114-133 appends for serving
    mode ``mode`` (native|direct) on pin ``pin`` with environment ``env``."""
    if pin == "v0.5.18":
        args = ["--dsv4-c4-cache-format", "native" if mode == "native" else "remnant",
                "--dsv4-c4-cache-implementation", "kernel"]
    else:
        args = ["--kv-cache-format", mode]
    if env.get("STORE_IMPLEMENTATION"):
        args += ["--dsv4-c4-cache-store-implementation", env["STORE_IMPLEMENTATION"]]
    if env.get("C4_KEEP_COUNT"):
        args += ["--dsv4-c4-cache-keep-count", env["C4_KEEP_COUNT"]]
    if env.get("C4_LAYER_KEEP_COUNTS"):
        args += ["--dsv4-c4-cache-layer-keep-counts", env["C4_LAYER_KEEP_COUNTS"]]
    return args


def test_launcher_flags_resolve_like_configure_cache_format():
    """Every flag run-server.sh passes on either pin parses, and resolves to
    the CacheFormat of the configure_cache_format call serve.sh:178-183 makes
    from the same settings; rejected profiles fail before any pool exists."""
    import argparse
    ratios = (0, 128, 4, 128, 4, 0, 4)  # C4 layers 2, 4, 6
    p = argparse.ArgumentParser()
    config.add_cli_arguments(p)
    p.add_argument("--tp", type=int)  # a server flag of its own, beside ours
    envs = ({}, {"STORE_IMPLEMENTATION": "kernel"}, {"STORE_IMPLEMENTATION": "triton"},
            {"C4_KEEP_COUNT": "256"}, {"C4_LAYER_KEEP_COUNTS": "2:256 6:256"},
            {"STORE_IMPLEMENTATION": "kernel", "C4_KEEP_COUNT": "256",
             "C4_LAYER_KEEP_COUNTS": "4=256,6:256"})
    try:
        for pin in ("v0.5.18", "v0.5.22"):
            for mode in ("native", "direct"):
                for env in envs:
                    argv = ["--tp", "4"] + _launcher_args(pin, mode, env)
                    got = config.configure_from_args(p.parse_args(argv), compression_ratios=ratios)
                    want = remnant.configure_cache_format(
                        "native" if mode == "native" else "remnant", "kernel",
                        env.get("STORE_IMPLEMENTATION") or None,
                        keep_count=int(env.get("C4_KEEP_COUNT") or 256),
                        layer_keep_counts=env.get("C4_LAYER_KEEP_COUNTS") or None,
                        compression_ratios=ratios)
                    assert got == want, (pin, mode, env)
                    assert got.packed == (mode == "direct")
                    assert got.record_bytes == (328 if mode == "direct" else 584)
        # the reconstruct reader through the v0.5.18 implementation flag
        got = config.configure_from_args(p.parse_args(
            ["--dsv4-c4-cache-format", "remnant", "--dsv4-c4-cache-implementation", "triton",
             "--dsv4-c4-cache-keep-count", "192", "--dsv4-c4-cache-layer-keep-counts", "6:448"]),
            compression_ratios=ratios)
        assert got.decode_impl == "reconstruct" and got.profile.counts() == (192, 192, 448)
        # no flag at all: Native
        assert not config.configure_from_args(p.parse_args([])).packed
        prev = config.current()
        # rejected before any pool: non-256 with the Direct reader, counts that are
        # no profile, overrides of non-C4 layers, contradicting format spellings
        for argv in (_launcher_args("v0.5.22", "direct", {"C4_KEEP_COUNT": "192"}),
                     _launcher_args("v0.5.18", "direct", {"C4_KEEP_COUNT": "192"}),
                     _launcher_args("v0.5.18", "direct", {"C4_LAYER_KEEP_COUNTS": "4:128"}),
                     _launcher_args("v0.5.22", "native", {"C4_KEEP_COUNT": "512"}),
                     _launcher_args("v0.5.22", "direct", {"C4_LAYER_KEEP_COUNTS": "3:256"}),
                     ["--kv-cache-format", "direct", "--dsv4-c4-cache-format", "native"]):
            with pytest.raises(ValueError):
                config.configure_from_args(p.parse_args(argv), compression_ratios=ratios)
            assert config.current() == prev
        for argv in (["--dsv4-c4-cache-format", "direct"],
                     ["--dsv4-c4-cache-store-implementation", "cuda"],
                     ["--dsv4-c4-cache-keep-count", "two"]):
            with pytest.raises(SystemExit):
                p.parse_args(argv)
    finally:
        remnant.configure_cache_format("native")


def test_profiles_validate_counts_ids_and_atomic_updates():
    """Per-layer counts name C4 layers of the model (compress_ratios entry 4),
    in any of the launcher's spellings; a rejected call keeps the previous
    profile (reference test of the same name, candidate-sglang.patch:939-940;
    scripts/local/serve.sh:178-185; scripts/local/README.md:993-1013)."""
    ratios = (0, 128, 4, 128, 4, 0, 4)
    try:
        c = remnant.configure_cache_format("remnant", "triton", keep_count=192,
                                           layer_keep_counts="6:448, 2=64",
                                           compression_ratios=ratios)
        prof = remnant.packed_profile()
        assert isinstance(prof, config.PackedProfile)
        assert prof == config.PackedProfile(192, ((2, 64), (6, 448)), ratios)
        assert prof.c4_layers() == (2, 4, 6) and prof.counts() == (64, 192, 448)
        assert [c.record_bytes_for(i) for i in (2, 4, 6)] == [136, 264, 520]
        assert [prof.count_for_c4_index(i) for i in range(3)] == [64, 192, 448]
        assert prof.c4_bytes_per_row() == 136 + 264 + 520  # summed, never padded to 256
        for spelling in ({2: 64, 6: 448}, [(6, 448), (2, 64)], ["2:64", "6:448"], "2:64 6:448"):
            again = remnant.configure_cache_format("remnant", "reconstruct", keep_count=192,
                                                   layer_keep_counts=spelling,
                                                   compression_ratios=ratios)
            assert again.profile == prof
        with pytest.raises(ValueError, match="not a C4 layer"):
            c.keep_count_for(3)  # a C128 layer has no Packed profile
        # rejected updates leave the previous profile untouched
        for bad in (dict(layer_keep_counts={1: 128}),        # C128 layer
                    dict(layer_keep_counts={0: 128}),        # SWA-only layer
                    dict(layer_keep_counts={7: 128}),        # beyond the model
                    dict(layer_keep_counts={2: 512}),        # not a profile
                    dict(layer_keep_counts=[(2, 64), (2, 128)]),  # two counts for one layer
                    dict(layer_keep_counts="2-64"),
                    dict(layer_keep_counts={2: 128}, compression_ratios=None),
                    dict(layer_keep_counts={-2: 128})):
            kw = dict(keep_count=192, compression_ratios=ratios)
            kw.update(bad)
            with pytest.raises(ValueError):
                remnant.configure_cache_format("remnant", "triton", **kw)
            assert remnant.packed_profile() == prof
        # Direct decode: every C4 layer must keep 256, overrides included
        with pytest.raises(ValueError, match="256"):
            remnant.configure_cache_format("remnant", "kernel", layer_keep_counts={4: 128},
                                           compression_ratios=ratios)
        assert remnant.packed_profile() == prof
        d = remnant.configure_cache_format("remnant", "kernel", layer_keep_counts={4: 256},
                                           compression_ratios=ratios)
        assert d.profile.counts() == (256, 256, 256)
        # overrides of non-C4 layers are what the C4-only rule forbids, also for Native
        with pytest.raises(ValueError):
            remnant.configure_cache_format("native", layer_keep_counts={3: 128},
                                           compression_ratios=ratios)
    finally:
        remnant.configure_cache_format("native")


def test_pool_planes_and_capacity():
    pool = remnant.LatentPool(3, device="cpu")
    assert pool.nbytes() == 3 * 20992 and pool.rows == 192
    assert pool.values().shape == (3, 64, 256)
    assert pool.bitmaps().shape == (3, 64, 64)
    assert pool.scales().shape == (3, 64, 8)
    pool.values()[1, 5] = 7
    pool.bitmaps()[1, 5] = 9
    pool.scales()[1, 5] = 11
    rec = pool.records(torch.tensor([69]))
    assert rec.shape == (1, 328)
    assert torch.all(rec[0, :256] == 7) and torch.all(rec[0, 256:320] == 9)
    assert torch.all(rec[0, 320:] == 11)
    # contiguous 328-byte records: slot 69 is bytes 5*328.. of page 1
    assert torch.equal(pool.layer()[1, 5 * 328:6 * 328], rec[0])
    assert config.PACKED_PAGE_BYTES % 16 == 0
    hbm = 288 * 10**9
    packed, native = remnant.records_fitting(hbm, "direct"), remnant.records_fitting(hbm, "native")
    assert abs(packed / 878.0e6 - 1) < 1e-3 and abs(native / 493.2e6 - 1) < 1e-3
    assert abs(packed / native - 584 / 328) < 1e-3


def test_record_transfer_host_validation():
    lib = _lib.load()
    _, a = buf(21000)
    _, b = buf(21000)
    _, s = buf(64)
    assert lib.rm_copy_records(a, 1, 0, s, b, 1, 0, s, 0, 1, 0, 256, None) == 0  # empty
    assert lib.rm_copy_records(a, 1, 0, s, b, 1, 0, s, 4, 1, 2, 256, None) == -4  # format
    assert lib.rm_copy_records(a, 1, 0, s, b, 1, 0, s, 4, 1, 0, 512, None) == -2  # no profile
    assert lib.rm_copy_records(a + 4, 1, 0, s, b, 1, 0, s, 4, 1, 0, 256, None) == -3
    assert lib.rm_copy_records(a, 1, 100, s, b, 1, 20992, s, 4, 2, 0, 256, None) == -2
    assert lib.rm_copy_records(None, 1, 0, s, b, 1, 0, s, 4, 1, 1, 256, None) == -1
    dev = remnant.LatentPool(2, layers=3, device="cpu")
    host = remnant.HostLatentPool.like(dev, pin_memory=False)
    assert host.buffer.shape == (3, 2, 20992) and host.rows == 128
    h448 = remnant.HostLatentPool(1, fmt="remnant", keep_count=448, pin_memory=False)
    assert h448.page_bytes == 64 * 520
    idx = torch.zeros(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="different record formats"):
        remnant.copy_records(dev, idx, h448, idx)
    with pytest.raises(ValueError, match="layer count"):
        remnant.copy_records(dev, idx, remnant.HostLatentPool(2, 1, pin_memory=False), idx)
    with pytest.raises(ValueError, match="equal length"):
        remnant.copy_records(dev, idx, host, idx[:2])
    with pytest.raises(ValueError, match="GPU"):
        host.backup_from_device_all_layer(dev, idx, idx)
    remnant.copy_records(dev, idx[:0], host, idx[:0])  # empty: nothing happens


class _FakeCudaTensor:
    """Stands for a GPU slot list in host-side checks that run before any launch."""

    def __init__(self, t):
        self._t = t
        self.dtype, self.shape, self.is_cuda = t.dtype, t.shape, True

    def dim(self):
        return self._t.dim()

    def is_contiguous(self):
        return True


def test_record_transfer_rejects_pageable_pools():
    """A pool in pageable host memory (a LatentPool on the CPU, an unpinned
    host pool) would hand the kernel an address the GPU cannot reach: it is
    refused before any launch."""
    idx = _FakeCudaTensor(torch.zeros(4, dtype=torch.int32))
    dev_cpu = remnant.LatentPool(2, device="cpu")
    host = remnant.HostLatentPool.like(dev_cpu, pin_memory=False)
    with pytest.raises(ValueError, match="pinned"):
        remnant.copy_records(dev_cpu, idx, host, idx)
    with pytest.raises(ValueError, match="pinned"):
        remnant.copy_records(host, idx, dev_cpu, idx, layer_id=0)


def test_native_store_and_decode_argument_checks():
    native = remnant.LatentPool(1, fmt="native", device="cpu")
    x = torch.zeros((2, 512))
    loc = torch.zeros(2, dtype=torch.int32)
    pos = torch.zeros(2, dtype=torch.int32)
    w = torch.ones(512)
    freqs = torch.ones((8, 32), dtype=torch.complex64)
    with pytest.raises(ValueError, match="weight"):
        remnant.native_store_rows(x, w.bfloat16(), 1e-6, loc, pos, freqs, native)
    with pytest.raises(ValueError, match="weight"):
        remnant.native_store_rows(x, w[:256], 1e-6, loc, pos, freqs, native)
    with pytest.raises(ValueError, match="weight"):
        remnant.native_store_rows(x, torch.ones(1024)[::2], 1e-6, loc, pos, freqs, native)
    with pytest.raises(ValueError, match="positions"):
        remnant.native_store_rows(x, w, 1e-6, loc, pos.long(), freqs, native)
    with pytest.raises(ValueError, match="positions"):
        remnant.native_store_rows(x, w, 1e-6, loc, torch.zeros(4, dtype=torch.int32)[::2],
                                  freqs, native)
    with pytest.raises(ValueError, match="complex64"):
        remnant.native_store_rows(x, w, 1e-6, loc, pos, freqs.to(torch.complex128), native)
    with pytest.raises(ValueError, match="GPU"):  # CPU positions with a GPU launch
        remnant.native_store_rows(x, w, 1e-6, loc, pos, freqs, native)
    pool = remnant.LatentPool(1, device="cpu")
    q = torch.zeros((1, 1, 16, 512), dtype=torch.bfloat16)
    bt = torch.zeros((1, 1), dtype=torch.int32)
    idx = torch.zeros((1, 1, 64), dtype=torch.int32)
    with pytest.raises(ValueError, match="at least one row"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx,
                                          freqs_cis=torch.ones(16, dtype=torch.complex64))
    with pytest.raises(ValueError, match="workspace"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx,
                                          workspace=torch.zeros(1 << 22, dtype=torch.uint8))
    with pytest.raises(ValueError, match="workspace"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx,
                                          workspace=torch.zeros(1 << 20, dtype=torch.float32))
    # the C entry point refuses a frequency table without rows
    lib = _lib.load()
    _, xq = buf(16384)
    _, pg = buf(21000)
    _, s = buf(64)
    _, f = buf(256)
    assert lib.rm_remnant_sparse_decode_fwd(xq, 1, 1, 16, pg, 1, s, 4, 4, None, s, 8, None,
                                            None, f, 0, None, 0.1, xq, f, None, 0, None) == -2


def test_adapter_host_validation():
    lib = _lib.load()
    _, pool = buf(21000)
    _, s = buf(64)
    _, out = buf(37376)
    assert lib.rm_packed_to_native(pool, 1, s, 1, 1, None, 0, 0, s, 1, 0, 5, None, 0, out, 1,
                                   None) == 0  # empty: no launch
    assert lib.rm_packed_to_native(pool, 1, s, 65, 1, None, 0, 0, s, 1, 2, 65, None, 0, out, 2,
                                   None) == -2  # 130 rows do not fit two pages
    assert lib.rm_packed_to_native(pool, 1, s, 1, 1, None, 0, 0, s, 1, 2, 5, None, 0, out + 8, 1,
                                   None) == -3
    packed = remnant.LatentPool(1, device="cpu")
    native = remnant.LatentPool(1, fmt="native", device="cpu")
    idx = torch.zeros((2, 40), dtype=torch.int32)
    lengths = torch.full((2,), 40, dtype=torch.int32)
    with pytest.raises(ValueError, match="Native pool"):
        remnant.packed_to_native(packed, idx, idx, lengths, None, packed)
    with pytest.raises(ValueError, match="fewer records"):
        remnant.packed_to_native(packed, torch.zeros((2, 40), dtype=torch.int32), None, lengths,
                                 None, native)
    with pytest.raises(ValueError, match="256-survivor"):
        remnant.packed_to_native(remnant.LatentPool(1, device="cpu", keep_count=192), idx[:1],
                                 None, lengths[:1], None, native)
    with pytest.raises(ValueError, match="GPU"):
        remnant.packed_to_native(packed, idx[:1], None, lengths[:1], None, native)


def test_decode_window_rows_host_validation():
    pool = remnant.LatentPool(1, device="cpu")
    native = remnant.LatentPool(1, fmt="native", device="cpu")
    q = torch.zeros((2, 1, 16, 512), dtype=torch.bfloat16)
    bt = torch.zeros((2, 1), dtype=torch.int32)
    idx = torch.zeros((2, 1, 4), dtype=torch.int32)
    sidx = torch.zeros((2, 1, 64), dtype=torch.int32)
    with pytest.raises(ValueError, match="together"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx, swa_pool=native)
    with pytest.raises(ValueError, match="Native pool"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx, swa_pool=pool, swa_indices=sidx)
    with pytest.raises(ValueError, match="swa_indices"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx, swa_pool=native,
                                          swa_indices=sidx[:1])
    with pytest.raises(ValueError, match="512"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx, swa_pool=native,
                                          swa_indices=torch.zeros((2, 1, 513), dtype=torch.int32))
    with pytest.raises(ValueError, match="swa_lengths"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx, swa_pool=native, swa_indices=sidx,
                                          swa_lengths=torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="GPU"):
        remnant.remnant_sparse_decode_fwd(q, pool, bt, idx, swa_pool=native, swa_indices=sidx)
    assert remnant.get_decode_metadata(300, 16, 512, 64) == (2, 300 * 2 * 16 * 513 * 4)
    assert remnant.get_decode_metadata(300, 16, 512) == (1, 0)


def test_survivor_profile_pools():
    """(K + 72)-byte records, 64 to a page; planes are views; a raw page tensor's
    size names its profile; the Direct reader refuses non-256 pools."""
    for count in config.KEEP_COUNTS:
        pool = remnant.LatentPool(2, device="cpu", keep_count=count)
        assert pool.page_bytes == 64 * (count + 72) and pool.record_bytes == count + 72
        assert pool.values().shape == (2, 64, count)
        assert pool.bitmaps().shape == (2, 64, 64) and pool.scales().shape == (2, 64, 8)
        pool.values()[1, 3] = 5
        pool.bitmaps()[1, 3] = 6
        pool.scales()[1, 3] = 7
        rec = pool.records(torch.tensor([67]))[0]
        assert torch.equal(pool.layer()[1, 3 * (count + 72):4 * (count + 72)], rec)
        assert torch.all(rec[:count] == 5) and torch.all(rec[count:count + 64] == 6)
        assert torch.all(rec[count + 64:] == 7)
        raw = torch.zeros((1, pool.page_bytes), dtype=torch.uint8)
        assert remnant.packed._as_pool(raw, None)[1:] == (True, count)
        assert config.packed_page_bytes(count) % 16 == 0
    with pytest.raises(ValueError):
        remnant.LatentPool(1, device="cpu", keep_count=512)
    with pytest.raises(ValueError):
        remnant.LatentPool(1, fmt="native", device="cpu", keep_count=192)
    with pytest.raises(ValueError, match="unknown page size"):
        remnant.packed._as_pool(torch.zeros((1, 64 * 300), dtype=torch.uint8), None)
    q = torch.zeros((1, 1, 16, 512), dtype=torch.bfloat16)
    bt = torch.zeros((1, 1), dtype=torch.int32)
    idx = torch.zeros((1, 1, 4), dtype=torch.int32)
    with pytest.raises(ValueError, match="256-survivor"):
        remnant.remnant_sparse_decode_fwd(q, remnant.LatentPool(1, device="cpu", keep_count=192),
                                          bt, idx)
    hbm = 288 * 10**9
    assert remnant.records_fitting(hbm, "direct", 64) > remnant.records_fitting(hbm, "direct")


class _RecordingLib:
    """Stands for the C library: records which entry point a call reaches."""

    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        if not name.startswith("rm_"):
            raise AttributeError(name)
        return lambda *args: self.calls.append((name, args)) or 0


def test_bf16_reader_dispatch_plane_buffers_and_empty_inputs(monkeypatch):
    """Mirror of the reference's test_bf16_reader_opt_in_dispatch_and_empty_inputs
    (candidate-sglang.patch:896-930): the reference's plane tuple (values u8
    [rows, 256], bitmaps u64 [rows, 8], scales u8 [rows, 8]) reaches the plane
    reader with its row count and survivor count, a page tensor the paged
    reader; fused_rope True and False both take the one fused launch; empty
    selections launch nothing; a non-bool flag raises TypeError."""
    from remnant import packed as packed_mod
    rec = _RecordingLib()
    monkeypatch.setattr(_lib, "load", lambda: rec)
    monkeypatch.setattr(packed_mod, "_check_cuda", lambda *t: None)
    monkeypatch.setattr(packed_mod, "_stream", lambda: 0)
    buffers = (torch.zeros((1, 256), dtype=torch.uint8), torch.zeros((1, 8), dtype=torch.uint64),
               torch.zeros((1, 8), dtype=torch.uint8))
    index = torch.zeros((1, 1), dtype=torch.int32)
    lengths = torch.ones(1, dtype=torch.int32)
    freqs = torch.ones((16, 32), dtype=torch.complex64)
    output = torch.empty((1, 512), dtype=torch.bfloat16)
    remnant.unpack_gather_bf16(buffers, index, index, lengths, freqs, output)
    remnant.unpack_gather_bf16(buffers, index, index, lengths, freqs, output, fused_rope=True)
    assert [c[0] for c in rec.calls] == ["rm_unpack_gather_bf16_planes"] * 2
    args = rec.calls[0][1]
    assert args[:3] == tuple(t.data_ptr() for t in buffers) and args[3:5] == (1, 256)
    # ..., n_queries, selected_k, freqs, freq_rows, output, stream
    assert args[-6:-2] == (1, 1, freqs.data_ptr(), 16) and args[-2] == output.data_ptr()
    rec.calls.clear()
    pages = torch.zeros((2, config.PACKED_PAGE_BYTES), dtype=torch.uint8)
    remnant.unpack_gather_bf16(pages, index, index, lengths, freqs, output, fused_rope=True)
    assert [c[0] for c in rec.calls] == ["rm_unpack_gather_bf16_k"]
    assert rec.calls[0][1][:3] == (pages.data_ptr(), 2, 256)
    rec.calls.clear()
    for physical, raw, active in ((index[:0], index[:0], lengths[:0]),
                                  (index[:, :0], index[:, :0], lengths)):
        remnant.unpack_gather_bf16(buffers, physical, raw, active, freqs, output,
                                   fused_rope=True)
    assert rec.calls == []
    for invalid in (1, 0, "fused", None):
        with pytest.raises(TypeError, match="fused_rope must be a bool"):
            remnant.unpack_gather_bf16(buffers, index, index, lengths, freqs, output,
                                       fused_rope=invalid)
    # the store and the Adapter take the same plane tuple
    x = torch.zeros((1, 512))
    remnant.pack_rows_fused(x, torch.ones(512), 1e-6, torch.zeros(1, dtype=torch.int32), buffers)
    native = remnant.LatentPool(1, fmt="native", device="cpu")
    remnant.packed_to_native(buffers, index, index, lengths, freqs, native)
    assert [c[0] for c in rec.calls] == ["rm_pack_rows_planes", "rm_packed_to_native_planes"]
    assert rec.calls[0][1][7:12] == (*(t.data_ptr() for t in buffers), 1, 256)[:5]


def test_plane_buffer_validation_and_remnant_buffers():
    rows = 6
    v = torch.zeros((rows, 192), dtype=torch.uint8)
    b = torch.zeros((rows, 8), dtype=torch.uint64)
    s = torch.zeros((rows, 8), dtype=torch.uint8)
    rb = remnant.remnant_buffers(v, b, s)
    assert isinstance(rb, remnant.RemnantBuffers) and rb.planes
    assert (rb.rows, rb.keep_count) == (rows, 192)
    assert remnant.remnant_buffers((v, b.view(torch.uint8), s)).keep_count == 192  # u8 view
    pool = remnant.LatentPool(2, layers=2, device="cpu")
    pb = remnant.remnant_buffers(pool, layer_id=1)
    assert not pb.planes and pb.pages.data_ptr() == pool.layer(1).data_ptr() and pb.rows == 128
    for bad in ((v[:, :100], b, s), (v.float(), b, s), (v, b[:5], s), (v, b.float(), s),
                (v, b, s[:, :4]), (v, b, s.t().contiguous().t()), (v[:, ::2], b, s),
                (torch.zeros((rows, 512), dtype=torch.uint8), b, s)):
        with pytest.raises(ValueError):
            remnant.unpack_gather_bf16(bad, torch.zeros((1, 1), dtype=torch.int32), None,
                                       torch.ones(1, dtype=torch.int32), None,
                                       torch.empty((1, 512), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="together"):
        remnant.remnant_buffers(v, b)
    with pytest.raises(ValueError, match="Packed"):
        remnant.remnant_buffers(remnant.LatentPool(1, fmt="native", device="cpu"))
    # the Direct decode reads 256-survivor planes with an even row count
    q = torch.zeros((1, 1, 16, 512), dtype=torch.bfloat16)
    bt = torch.zeros((1, 1), dtype=torch.int32)
    idx = torch.zeros((1, 1, 4), dtype=torch.int32)
    with pytest.raises(ValueError, match="256-survivor"):
        remnant.remnant_sparse_decode_fwd(q, rb, bt, idx)
    odd = remnant.remnant_buffers(torch.zeros((5, 256), dtype=torch.uint8),
                                  torch.zeros((5, 8), dtype=torch.uint64),
                                  torch.zeros((5, 8), dtype=torch.uint8))
    with pytest.raises(ValueError, match="even"):
        remnant.remnant_sparse_decode_fwd(q, odd, bt, idx)
    # C ABI: null planes, alignment, odd rows
    lib = _lib.load()
    _, xq = buf(16384)
    _, vp = buf(4096)
    _, bp = buf(1024)
    _, sp = buf(256)
    _, ix = buf(64)
    _, f = buf(256)
    _, out = buf(2048)
    assert lib.rm_unpack_gather_bf16_planes(vp, None, sp, 4, 256, ix, 1, 1, None, 0, 0, ix, 1, 1,
                                            1, None, 0, out, None) == -1
    assert lib.rm_unpack_gather_bf16_planes(vp, bp + 4, sp, 4, 256, ix, 1, 1, None, 0, 0, ix, 1,
                                            1, 1, None, 0, out, None) == -3
    assert lib.rm_unpack_gather_bf16_planes(vp, bp, sp, 4, 200, ix, 1, 1, None, 0, 0, ix, 1, 1,
                                            1, None, 0, out, None) == -2
    assert lib.rm_pack_rows_planes(xq, 1, 512, f, 1e-6, ix, 1, vp, None, sp, 4, 256, None) == -1
    assert lib.rm_pack_rows_planes(xq, 1, 512, f, 1e-6, ix, 1, vp + 4, bp, sp, 4, 256,
                                   None) == -3
    dec = [xq, 1, 1, 16, vp, bp, sp, 5, ix, 4, 4, None, ix, 4, None, None, 0, None, 0, None,
           None, None, 0, None, 0.1, out, f, None, 0, None]
    assert lib.rm_remnant_sparse_decode_planes_fwd(*dec) == -2  # odd rows
    dec[7] = 4
    dec[5] = bp + 8
    assert lib.rm_remnant_sparse_decode_planes_fwd(*dec) == -3  # bitmaps not 16-byte aligned
    dec[5] = None
    assert lib.rm_remnant_sparse_decode_planes_fwd(*dec) == -1
