"""The allocation-free Direct decode (rm_remnant_sparse_decode_swa_noalloc_fwd)
against the workspace entry point it mirrors (rm_remnant_sparse_decode_swa_fwd),
through the C ABI: identical bits on two calls in a row, the second with a
smaller input, a split plan beyond the library's 32 MiB array refused without
a launch, nothing allocated by the call (neither by torch's allocator nor on
the device: its free memory is unchanged across the call), and the call
captured in a HIP graph and replayed with changed inputs."""

import numpy as np
import pytest
import torch

import remnant
from remnant import _lib
from test_gpu_parity import DEV, add_swa, build_decode_case

pytestmark = pytest.mark.gpu


def banner(msg):
    print(f"[gpu-noalloc] {msg}", flush=True)


def ptr(t):
    return None if t is None else t.data_ptr()


def call(lib, c, noalloc, rope="table"):
    q = c["q"].to(DEV)
    b, sq, h, _ = q.shape
    bt = torch.from_numpy(c["table"]).to(DEV)
    idx = torch.from_numpy(c["idx"]).to(DEV)
    lens = torch.from_numpy(c["lens"]).to(DEV)
    seq = torch.tensor(c["contexts"], dtype=torch.int32, device=DEV)
    sink = c["sink"].to(DEV)
    freqs = c["freqs"].to(DEV)
    sidx = torch.from_numpy(c["swa_idx"]).to(DEV) if c.get("swa_pool") is not None else None
    spool = c["swa_pool"].layer() if sidx is not None else None
    width = 0 if sidx is None else sidx.shape[-1]
    out = torch.full_like(q, 7.0)
    lse = torch.full((b, sq, h), 7.0, dtype=torch.float32, device=DEV)
    pool = c["pool"].layer()
    args = [q.data_ptr(), b, sq, h, pool.data_ptr(), pool.shape[0], bt.data_ptr(), bt.stride(0),
            bt.shape[1], seq.data_ptr(), idx.data_ptr(), idx.shape[-1], lens.data_ptr(),
            ptr(spool), 0 if spool is None else spool.shape[0], ptr(sidx), width, None,
            sink.data_ptr(), freqs.data_ptr(), freqs.numel() // 32, None, 1 / np.sqrt(512)]
    if rope == "positions":
        inv = c.setdefault("inv_freq_dev", remnant.synthetic.rope_inv_freq().to(DEV))
        args[19:22] = [None, 0, inv.data_ptr()]
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        before = torch.cuda.memory_allocated()
        free_before = torch.cuda.mem_get_info()[0]
        st = lib.rm_remnant_sparse_decode_swa_noalloc_fwd(*args, out.data_ptr(), lse.data_ptr(),
                                                          stream)
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == before
        if c.get("warm"):  # device-wide free memory, after a first call on this device
            assert torch.cuda.mem_get_info()[0] == free_before
    else:
        _, need = remnant.get_decode_metadata(b * sq, h, idx.shape[-1], width)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=DEV)
        st = lib.rm_remnant_sparse_decode_swa_fwd(*args, out.data_ptr(), lse.data_ptr(),
                                                  ws.data_ptr(), need, stream)
    assert st == 0, st
    torch.cuda.synchronize()
    return out, lse


def test_noalloc_decode_equals_workspace_decode_on_two_calls():
    lib = _lib.load()
    banner("noalloc: large call (B=4, H=32, top-k 2048, window 64)")
    big = build_decode_case([9000, 3000, 5000, 2500], q_len=1, heads=32, topk=2048, seed=501)
    add_swa(big, 64, seed=502)
    small = build_decode_case([700, 300], q_len=2, heads=16, topk=256, seed=503)
    assert remnant.get_decode_metadata(4, 32, 2048, 64)[0] > 1  # partials in the array
    call(lib, small, True)  # warm-up: the library's first call on this device
    big["warm"] = small["warm"] = True
    for case, name in ((big, "large"), (small, "smaller")):
        banner(f"noalloc: {name} call")
        out_n, lse_n = call(lib, case, True)
        out_w, lse_w = call(lib, case, False)
        assert torch.equal(out_n.view(torch.int16), out_w.view(torch.int16)), name
        assert torch.equal(lse_n, lse_w), name
        assert torch.isfinite(out_n.float()).all()


def test_noalloc_decode_refuses_split_plans_beyond_its_array():
    banner("noalloc: oversized plan refused")
    lib = _lib.load()
    # 1,024 tokens x 16 heads: one C4 split each plus the window rows' slot,
    # 2 partial rows of 2 KiB per (token, head): 64 MiB, beyond the 32 MiB array
    tokens, heads, topk, wtop = 1024, 16, 512, 64
    slots, need = remnant.get_decode_metadata(tokens, heads, topk, wtop)
    assert slots == 2 and need > (32 << 20)
    q = torch.zeros((tokens, 1, heads, 512), dtype=torch.bfloat16, device=DEV)
    pool = remnant.LatentPool(1, device=DEV).layer()
    swa_pool = remnant.LatentPool(1, fmt="native", device=DEV).layer()
    bt = torch.zeros((tokens, 1), dtype=torch.int32, device=DEV)
    idx = torch.full((tokens, 1, topk), -1, dtype=torch.int32, device=DEV)
    widx = torch.full((tokens, 1, wtop), -1, dtype=torch.int32, device=DEV)
    out = torch.full_like(q, 3.0)
    lse = torch.zeros((tokens, 1, heads), dtype=torch.float32, device=DEV)
    st = lib.rm_remnant_sparse_decode_swa_noalloc_fwd(
        q.data_ptr(), tokens, 1, heads, pool.data_ptr(), 1, bt.data_ptr(), 1, 1, None,
        idx.data_ptr(), topk, None, swa_pool.data_ptr(), 1, widx.data_ptr(), wtop, None, None,
        None, 0, None, 0.1, out.data_ptr(), lse.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert st == -5
    torch.cuda.synchronize()
    assert torch.all(out.float() == 3.0)  # nothing was launched


@pytest.mark.parametrize("rope", ["table", "positions"])
def test_noalloc_decode_graph_replay_with_changed_inputs(rope):
    """The allocation-free call captured once in a HIP graph (after one eager
    call on the device); q, indices and lengths change in place between
    replays, and every replay equals the workspace entry point's eager result
    bit for bit."""
    banner(f"noalloc: graph replay rope={rope}")
    lib = _lib.load()
    c = build_decode_case([3000, 1200, 2500], q_len=2, heads=16, topk=1024, seed=521)
    add_swa(c, 64, seed=522)
    b, sq, h, _ = c["q"].shape
    assert remnant.get_decode_metadata(b * sq, h, 1024, 64)[0] > 1  # partials in the array
    q = c["q"].to(DEV)
    bt = torch.from_numpy(c["table"]).to(DEV)
    idx = torch.from_numpy(c["idx"]).to(DEV)
    lens = torch.from_numpy(c["lens"]).to(DEV)
    seq = torch.tensor(c["contexts"], dtype=torch.int32, device=DEV)
    sink = c["sink"].to(DEV)
    freqs = c["freqs"].to(DEV)
    inv = remnant.synthetic.rope_inv_freq().to(DEV)
    sidx = torch.from_numpy(c["swa_idx"]).to(DEV)
    spool = c["swa_pool"].layer()
    pool = c["pool"].layer()
    rope_args = ([freqs.data_ptr(), freqs.numel() // 32, None] if rope == "table"
                 else [None, 0, inv.data_ptr()])
    args = [q.data_ptr(), b, sq, h, pool.data_ptr(), pool.shape[0], bt.data_ptr(), bt.stride(0),
            bt.shape[1], seq.data_ptr(), idx.data_ptr(), idx.shape[-1], lens.data_ptr(),
            spool.data_ptr(), spool.shape[0], sidx.data_ptr(), sidx.shape[-1], None,
            sink.data_ptr(), *rope_args, 1 / np.sqrt(512)]
    out = torch.empty_like(q)
    lse = torch.empty((b, sq, h), dtype=torch.float32, device=DEV)
    _, need = remnant.get_decode_metadata(b * sq, h, idx.shape[-1], 64)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    ref_out = torch.empty_like(q)
    ref_lse = torch.empty_like(lse)

    def noalloc():
        st = lib.rm_remnant_sparse_decode_swa_noalloc_fwd(
            *args, out.data_ptr(), lse.data_ptr(), torch.cuda.current_stream().cuda_stream)
        assert st == 0, st

    noalloc()  # eager: the scratch address of this device is looked up here
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        noalloc()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        noalloc()
    torch.cuda.synchronize()
    for it in range(3):
        g = torch.Generator().manual_seed(530 + it)
        q.copy_((torch.randn(q.shape, generator=g) * (0.5 + it)).to(torch.bfloat16))
        new_idx, new_lens = remnant.synthetic.topk_indices(c["contexts"], sq, 1024, seed=531 + it)
        new_lens = np.minimum(new_lens, 1024 - 100 * it).astype(np.int32)
        idx.copy_(torch.from_numpy(new_idx))
        lens.copy_(torch.from_numpy(new_lens))
        out.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        st = lib.rm_remnant_sparse_decode_swa_fwd(*args, ref_out.data_ptr(), ref_lse.data_ptr(),
                                                  ws.data_ptr(), need,
                                                  torch.cuda.current_stream().cuda_stream)
        assert st == 0, st
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), it
        assert torch.equal(lse, ref_lse), it
