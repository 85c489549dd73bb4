"""GPU parity of the dense DiT-block path (hipBLASLt GEMMs, norm / modulation / residual kernels, cross-attention
on the block-sparse kernel, and the whole streaming blockForward around the LCSA layer call) against the oracle
(oracle/dit.py, DiT.swift:317-381,491-551).

Tolerances: a GEMM's bf16 output may differ from the float64-accumulated reference by one bf16 rounding
(relative Frobenius error <= 4e-3); the whole block passes ~15 bf16 roundings and a GELU evaluated before (GPU) or
after (reference) the bf16 rounding of its input; its output is held to a relative Frobenius error <= 5e-3 per
chunk. The selection in the block tests keeps every in-window key block (top-k above the count of pairs), so the
mask is fixed by the local window and no near-tie can flip it.
"""
import math

import numpy as np
import pytest
import torch

import fvsr_lcsa
from oracle import dit as D
from oracle import lcsa as L

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _bf(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).to(dev)


@pytest.mark.parametrize("rows,n_in,n_out,bias,gelu", [(300, 256, 512, True, False), (77, 512, 256, False, False),
                                                       (300, 256, 512, True, True), (1000, 1536, 8960, True, True)])
def test_linear_matches_reference(dev, rows, n_in, n_out, bias, gelu):
    r = np.random.default_rng(rows + n_out)
    x = L.to_bf16(r.standard_normal((rows, n_in)).astype(np.float32))
    w = L.to_bf16((r.standard_normal((n_out, n_in)) / math.sqrt(n_in)).astype(np.float32))
    b = L.to_bf16((r.standard_normal(n_out) * 0.1).astype(np.float32)) if bias else None
    print(f"linear rows={rows} in={n_in} out={n_out} bias={bias} gelu={gelu}", flush=True)
    y = fvsr_lcsa.linear(_bf(x, dev), _bf(w, dev), None if b is None else _bf(b, dev), gelu=gelu)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    acc = D.linear(x, w, b, bf16=False).astype(np.float64)
    if gelu:
        # the GEMM epilogue applies GELU to the fp32 result (one rounding); the reference rounds first
        np.testing.assert_array_less(_rel(got, L.to_bf16(D.gelu_tanh(acc).astype(np.float32))), 4e-3)
        ref = L.to_bf16(D.gelu_tanh(D.linear(x, w, b)).astype(np.float32))
        assert _rel(got, ref) < 1e-2
    else:
        assert _rel(got, L.to_bf16(acc.astype(np.float32))) < 4e-3


def test_linear_rejects_bad_shapes(dev):
    x = torch.zeros((4, 12), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((16, 12), dtype=torch.bfloat16, device=dev)
    with pytest.raises(fvsr_lcsa.FVSRError):
        fvsr_lcsa.linear(x, w)          # in_features not a multiple of 8
    with pytest.raises(fvsr_lcsa.FVSRError):
        fvsr_lcsa.linear(x, torch.zeros((16, 8), dtype=torch.bfloat16, device=dev))
    x16 = torch.zeros((4, 16), dtype=torch.bfloat16, device=dev)
    w16 = torch.zeros((16, 16), dtype=torch.bfloat16, device=dev)
    with pytest.raises(fvsr_lcsa.FVSRError, match="elements"):
        fvsr_lcsa.linear(x16, w16, torch.zeros(8, dtype=torch.bfloat16, device=dev))   # bias shorter than out
    with pytest.raises(fvsr_lcsa.FVSRError, match="expected a tensor on"):
        fvsr_lcsa.linear(x16, w16.cpu())                                                # weight on the host
    with pytest.raises(fvsr_lcsa.FVSRError, match="elements"):
        fvsr_lcsa.DiTBlock({"q_weight": w16, "ffn1_weight": torch.zeros((32, 16), dtype=torch.bfloat16, device=dev),
                            "ffn2_weight": torch.zeros((16, 16), dtype=torch.bfloat16, device=dev)}, 1)   # not 16 x 32


def _weights(r, c, ffn, heads):
    def m(*shape, scale=1.0):
        return L.to_bf16((r.standard_normal(shape) * scale).astype(np.float32))
    W = {"modulation": m(6, c, scale=0.1)}
    for p in ("q", "k", "v", "o", "cross_q", "cross_k", "cross_v", "cross_o"):
        W[p + "_weight"] = m(c, c, scale=1 / math.sqrt(c))
        W[p + "_bias"] = m(c, scale=0.05)
    for p in ("norm_q", "norm_k", "cross_norm_q", "cross_norm_k"):
        W[p + "_weight"] = L.to_bf16((1 + 0.1 * r.standard_normal(c)).astype(np.float32))
    W["norm3_weight"] = L.to_bf16((1 + 0.1 * r.standard_normal(c)).astype(np.float32))
    W["norm3_bias"] = m(c, scale=0.05)
    W["ffn1_weight"] = m(ffn, c, scale=1 / math.sqrt(c))
    W["ffn1_bias"] = m(ffn, scale=0.05)
    W["ffn2_weight"] = m(c, ffn, scale=1 / math.sqrt(ffn))
    W["ffn2_bias"] = m(c, scale=0.05)
    return W


def test_cross_kv_matches_oracle(dev):
    r = np.random.default_rng(7)
    heads, c = 2, 256
    W = _weights(r, c, 512, heads)
    ctx = L.to_bf16(r.standard_normal((100, c)).astype(np.float32))
    blk = fvsr_lcsa.DiTBlock({k: _bf(v, dev) for k, v in W.items()}, heads)
    blk.set_context(_bf(ctx, dev))
    torch.cuda.synchronize()
    k_ref, v_ref = D.cross_kv(ctx, W["cross_k_weight"], W["cross_k_bias"], W["cross_v_weight"], W["cross_v_bias"],
                              W["cross_norm_k_weight"])
    assert _rel(blk.t["cross_k"].float().cpu().numpy(), k_ref) < 8e-3
    assert _rel(blk.t["cross_v"].float().cpu().numpy(), v_ref) < 4e-3


@pytest.mark.parametrize("heads,ffn,bh,bw,rng,ctx_len,chunks", [
    (2, 512, 3, 3, 3, 100, [(2, 0), (1, 4), (1, 6)]),
    (12, 8960, 2, 2, 1, 128, [(1, 0)]),
])
def test_dit_block_matches_oracle(dev, heads, ffn, bh, bw, rng, ctx_len, chunks):
    """Streaming chunks (n_new_slices, t0) through one block and its ring; the oracle keeps its own window cache."""
    r = np.random.default_rng(heads * 100 + bh)
    c = heads * 128
    W = _weights(r, c, ffn, heads)
    ctx = L.to_bf16(r.standard_normal((ctx_len, c)).astype(np.float32))
    W["cross_k"], W["cross_v"] = D.cross_kv(ctx, W["cross_k_weight"], W["cross_k_bias"], W["cross_v_weight"],
                                            W["cross_v_bias"], W["cross_norm_k_weight"])
    t_mod = L.to_bf16((r.standard_normal((6, c)) * 0.1).astype(np.float32))
    local = L.local_block_mask(bh, bw, rng)   # leaves blocks outside every window (probability 0)
    s = bh * bw
    blk = fvsr_lcsa.DiTBlock({k: _bf(v, dev) for k, v in W.items() if k not in ("cross_k", "cross_v")}, heads)
    blk.set_context(_bf(ctx, dev))
    ring = fvsr_lcsa.KVRing(1, heads, bh, bw, capacity=4, kv_len=3, device=dev.index or 0)
    cache = L.KVWindowCache()
    tm = _bf(t_mod, dev)
    for n_new, t0 in chunks:
        f, h, w = 2 * n_new, 8 * bh, 8 * bw
        x = L.to_bf16(r.standard_normal((f * h * w, c)).astype(np.float32))
        nk = (ring.slices(0) + n_new) * s
        topk = n_new * s * nk + 1   # above the pair count: keep every in-window block
        print(f"dit block heads={heads} ffn={ffn} grid={bh}x{bw} chunk n_new={n_new} t0={t0}", flush=True)
        xg = _bf(x, dev)
        blk.forward(ring, 0, xg, tm, n_new, t0, local, topk, mode=fvsr_lcsa.ATTN_KERNEL)
        torch.cuda.synchronize()
        ref, _ = D.block_forward(x, W, t_mod, cache, f, h, w, heads, t0, local, topk)
        err = _rel(xg.float().cpu().numpy(), ref)
        print(f"  rel err {err:.3e}", flush=True)
        assert err < 5e-3
    ring.close()


def test_chained_blocks_match_oracle(dev):
    """Config 5's shape of the computation at small size: every chunk's tokens through block 0, its output through
    block 1, then block 2 (random-init blocks, each with its own ring layer; the oracle keeps one window cache per
    block), over the streaming schedule 2, 1, 1 slices. The blocks' errors compound, so the bar is the per-block one
    times the depth: relative Frobenius error <= 1.5e-2 after the third block."""
    heads, ffn, bh, bw, rng, ctx_len, depth = 2, 512, 3, 3, 3, 100, 3
    r = np.random.default_rng(31)
    c, s = heads * 128, bh * bw
    local = L.local_block_mask(bh, bw, rng)
    t_mod = L.to_bf16((r.standard_normal((6, c)) * 0.1).astype(np.float32))
    tm = _bf(t_mod, dev)
    ring = fvsr_lcsa.KVRing(depth, heads, bh, bw, capacity=4, kv_len=3, device=dev.index or 0)
    Ws, blks, caches = [], [], []
    for _ in range(depth):
        W = _weights(r, c, ffn, heads)
        ctx = L.to_bf16(r.standard_normal((ctx_len, c)).astype(np.float32))
        W["cross_k"], W["cross_v"] = D.cross_kv(ctx, W["cross_k_weight"], W["cross_k_bias"], W["cross_v_weight"],
                                                W["cross_v_bias"], W["cross_norm_k_weight"])
        blk = fvsr_lcsa.DiTBlock({k: _bf(v, dev) for k, v in W.items() if k not in ("cross_k", "cross_v")}, heads)
        blk.set_context(_bf(ctx, dev))
        Ws.append(W)
        blks.append(blk)
        caches.append(L.KVWindowCache())
    for n_new, t0 in [(2, 0), (1, 4), (1, 6)]:
        f, h, w = 2 * n_new, 8 * bh, 8 * bw
        x = L.to_bf16(r.standard_normal((f * h * w, c)).astype(np.float32))
        nk = (ring.slices(0) + n_new) * s
        topk = n_new * s * nk + 1   # above the pair count: keep every in-window block
        xg = _bf(x, dev)
        ref = x
        for layer in range(depth):
            print(f"chained blocks chunk n_new={n_new} t0={t0} block {layer}", flush=True)
            blks[layer].forward(ring, layer, xg, tm, n_new, t0, local, topk, mode=fvsr_lcsa.ATTN_KERNEL)
            ref, _ = D.block_forward(ref, Ws[layer], t_mod, caches[layer], f, h, w, heads, t0, local, topk)
            ref = L.to_bf16(np.asarray(ref, dtype=np.float32))   # the next block reads bf16 tokens
        torch.cuda.synchronize()
        err = _rel(xg.float().cpu().numpy(), ref)
        print(f"  rel err after {depth} blocks {err:.3e}", flush=True)
        assert err < 1.5e-2
    ring.close()


def test_reserved_block_calls_allocate_nothing(dev):
    """fvsr_ctx_reserve_block sizes the hipBLASLt state, the block workspace and the select/attention workspace up
    front: block calls of at most the reserved size then leave both workspaces as they are (no hipFree / hipMalloc
    inside the call)."""
    heads, ffn, bh, bw, ctx_len = 2, 512, 3, 3, 100
    r = np.random.default_rng(5)
    c, s = heads * 128, bh * bw
    W = _weights(r, c, ffn, heads)
    blk = fvsr_lcsa.DiTBlock({k: _bf(v, dev) for k, v in W.items()}, heads)
    blk.set_context(_bf(L.to_bf16(r.standard_normal((ctx_len, c)).astype(np.float32)), dev))
    ring = fvsr_lcsa.KVRing(1, heads, bh, bw, capacity=4, kv_len=3, device=dev.index or 0)
    fresh = fvsr_lcsa.Context(dev.index or 0)      # a context no earlier call has grown
    ring.ctx = fresh
    # the largest chunk (2 slices) over the fullest window: kv_len 3 held + 1 new = 4 slices = the capacity, exactly
    # what the header asks for (min(capacity, kv_len + largest chunk) slices); the last call below attends over it
    tokens, key_tokens = 2 * s * 128, 4 * s * 128
    fresh.reserve_block(heads, tokens, ffn, ctx_len, key_tokens)
    ws, bws = fresh.workspace_bytes(), fresh.block_workspace_bytes()
    assert ws > 0 and bws > 0
    tm = _bf(L.to_bf16((r.standard_normal((6, c)) * 0.1).astype(np.float32)), dev)
    local = L.local_block_mask(bh, bw, 3)
    for n_new, t0 in [(2, 0), (1, 4), (1, 6)]:
        x = _bf(L.to_bf16(r.standard_normal((2 * n_new * 64 * s, c)).astype(np.float32)), dev)
        blk.forward(ring, 0, x, tm, n_new, t0, local, 40)
        torch.cuda.synchronize()
        assert torch.isfinite(x.float()).all()
        assert (fresh.workspace_bytes(), fresh.block_workspace_bytes()) == (ws, bws)
    ring.close()
