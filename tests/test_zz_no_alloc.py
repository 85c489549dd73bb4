"""fvsr_lcsa_attention_noalloc through the C ABI: the same results as fvsr_lcsa_attention (the same kernels, with the
row order and work counter in the library's static device scratch instead of the context workspace), on two calls
in a row with the second smaller; a fresh context's workspace stays unallocated; sizes beyond the scratch are refused
before any device work."""
import ctypes as C

import numpy as np
import pytest
import torch

import fvsr_lcsa
from fvsr_lcsa import _abi
from oracle import lcsa as O

pytestmark = pytest.mark.gpu


def _fresh_ctx(dev):
    h = C.c_void_p()
    _abi.call("fvsr_ctx_create", dev.index or 0, C.byref(h))
    return h


def _attend(name, ctx, q, k, v, kidx, kcnt, heads, o):
    code = _abi.DTYPE_BF16 if q.dtype == torch.bfloat16 else _abi.DTYPE_F32
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    _abi.call(name, ctx, code, C.c_void_p(q.data_ptr()), q.shape[0], C.c_void_p(k.data_ptr()),
              C.c_void_p(v.data_ptr()), k.shape[0], heads, C.c_void_p(kidx.data_ptr()), C.c_void_p(kcnt.data_ptr()),
              kidx.shape[-1], C.c_void_p(o.data_ptr()), stream)


def _case(dev, dtype, heads, lqb, lk, seed):
    gen = torch.Generator().manual_seed(seed)
    lq = lqb * 128 - 40                                    # a ragged query tail too
    q = torch.randn((lq, heads * 128), generator=gen).to(dtype)
    k = torch.randn((lk, heads * 128), generator=gen).to(dtype)
    v = torch.randn((lk, heads * 128), generator=gen).to(dtype)
    nk = -(-lk // 128)
    dens = torch.rand((heads, lqb, 1), generator=gen)
    m = (torch.rand((heads, lqb, nk), generator=gen) < dens).float()
    m[0, 1] = 0                                            # one empty row
    kidx, kcnt = O.block_lists(m.numpy())
    return (q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(kidx).to(dev), torch.from_numpy(kcnt).to(dev), m,
            (q, k, v))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_equals_workspace_entry_on_two_calls(dev, dtype):
    ctx = _fresh_ctx(dev)
    try:
        # 12 x 60 = 720 rows (past the persistent grid of 512 workgroups), then 4 x 9 = 36 rows: the second call
        # reuses the scratch the first one left behind
        for heads, lqb, lk, seed in ((12, 60, 20 * 128 + 64, 1), (4, 9, 1000, 2)):
            print(f"  noalloc {dtype} heads {heads} query blocks {lqb} lk {lk}", flush=True)
            q, k, v, kidx, kcnt, m, host = _case(dev, dtype, heads, lqb, lk, seed)
            o_ws = torch.full_like(q, float("nan"))
            o_na = torch.full_like(q, float("nan"))
            ws = _abi.lib.fvsr_ctx_workspace_bytes(ctx)    # 0 on the first call: a fresh context
            _attend("fvsr_lcsa_attention_noalloc", ctx, q, k, v, kidx, kcnt, heads, o_na)
            assert _abi.lib.fvsr_ctx_workspace_bytes(ctx) == ws     # the call grew no workspace
            _attend("fvsr_lcsa_attention", ctx, q, k, v, kidx, kcnt, heads, o_ws)
            torch.cuda.synchronize()
            assert not torch.isnan(o_na).any()
            assert torch.equal(o_na, o_ws)
            if heads == 4:   # the small case against the oracle as well
                ref = O.block_masked_attention(*(t.float().numpy() for t in host), m.numpy(), heads)
                bar = 1e-2 if dtype == torch.bfloat16 else 1e-5
                assert O.compare(o_na.float().cpu().numpy(), ref)["rel"] <= bar
    finally:
        _abi.lib.fvsr_ctx_destroy(ctx)


def test_noalloc_refuses_rows_beyond_its_scratch(dev):
    """4096 heads x 65 query blocks = 266240 rows > 262144: refused with FVSR_ERR_UNSUPPORTED before any device work
    (the pointers are never dereferenced)."""
    ctx = fvsr_lcsa.Context.get(dev)
    t = torch.zeros((128, 128), dtype=torch.bfloat16, device=dev)
    p = C.c_void_p(t.data_ptr())
    rc = _abi.lib.fvsr_lcsa_attention_noalloc(ctx.handle, _abi.DTYPE_BF16, p, 65 * 128, p, p, 128, 4096, p, p, 1, p,
                                              None)
    assert rc == _abi.ERR_UNSUPPORTED
    assert b"static scratch" in _abi.lib.fvsr_last_error()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_replays_under_graph_capture(dev, dtype):
    """The allocation-free call captured into a HIP graph (torch.cuda.CUDAGraph) and replayed three times with new
    q/k/v and new key lists copied into the captured buffers, eager work in between: every replay equals
    fvsr_lcsa_attention on the same inputs bit for bit (the order kernel rewrites the scratch's row order and work
    counter on each replay)."""
    ctx = _fresh_ctx(dev)
    try:
        heads, lqb, lk = 6, 20, 12 * 128 + 64
        q, k, v, kidx, kcnt, _, _ = _case(dev, dtype, heads, lqb, lk, 10)
        o_graph = torch.zeros_like(q)
        o_ws = torch.zeros_like(q)
        _attend("fvsr_lcsa_attention_noalloc", ctx, q, k, v, kidx, kcnt, heads, o_graph)   # eager first call
        torch.cuda.synchronize()
        ws = _abi.lib.fvsr_ctx_workspace_bytes(ctx)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            _attend("fvsr_lcsa_attention_noalloc", ctx, q, k, v, kidx, kcnt, heads, o_graph)
        assert _abi.lib.fvsr_ctx_workspace_bytes(ctx) == ws
        for rep, seed in enumerate((11, 12, 13)):
            print(f"  graph replay {rep} {dtype} seed {seed}", flush=True)
            q2, k2, v2, kidx2, kcnt2, _, _ = _case(dev, dtype, heads, lqb, lk, seed)
            for dst, src in ((q, q2), (k, k2), (v, v2), (kidx, kidx2), (kcnt, kcnt2)):
                dst.copy_(src)
            o_graph.fill_(float("nan"))
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            _attend("fvsr_lcsa_attention", ctx, q, k, v, kidx, kcnt, heads, o_ws)      # eager, between replays
            torch.cuda.synchronize()
            assert not torch.isnan(o_graph).any()
            assert torch.equal(o_graph, o_ws), rep
        del g
    finally:
        torch.cuda.synchronize()
        _abi.lib.fvsr_ctx_destroy(ctx)
