"""The allocation-free Direct decode (rm_remnant_sparse_decode_swa_noalloc_fwd)
against the workspace entry point it mirrors (rm_remnant_sparse_decode_swa_fwd),
through the C ABI: identical bits on two calls in a row, the second with a
smaller input, a split plan beyond the library's 32 MiB array refused without
a launch, and nothing allocated by the call."""

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


def call(lib, c, noalloc):
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
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        before = torch.cuda.memory_allocated()
        st = lib.rm_remnant_sparse_decode_swa_noalloc_fwd(*args, out.data_ptr(), lse.data_ptr(),
                                                          stream)
        assert torch.cuda.memory_allocated() == before
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
