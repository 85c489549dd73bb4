"""GPU parity of the fused projection epilogue (WanRMSNorm + 3-D RoPE + window partition, and the same straight into
the KV ring; DiT.swift:34-47,100-118,496-511) through the C ABI, against the oracle.

Bars (written in each test): V is a copy, bit-exact. Q and K (bfloat16): at least 99 % of the elements identical to
the oracle, and every rotated (re, im) pair within 2^-6 of the pair's length — the sum of squares over 1536 channels
is reduced in a different order than numpy's, which can move one of the three bfloat16 roundings (normalise, weight,
rotate) by an ulp, and a rotation keeps the length of that difference, so the bound is set on the pair, not on an
element that cancels; fp32: rel <= 2e-6. The ring variant must equal the plain epilogue bit for bit (contents,
pooled keys through the selection, and Q).
"""
import numpy as np
import pytest
import torch

import fvsr_lcsa
from oracle import lcsa as O

pytestmark = pytest.mark.gpu


def _inputs(f, h, w, heads, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    L, c = f * h * w, heads * 128
    q, k, v = (torch.randn((L, c), generator=g) * 1.5 for _ in range(3))
    wq = 0.5 + torch.rand(c, generator=g)
    wk = 0.5 + torch.rand(c, generator=g)
    cast = (lambda t: t.to(torch.bfloat16)) if dtype == torch.bfloat16 else (lambda t: t)
    return [cast(t) for t in (q, k, v, wq, wk)]


def _close_pairs(got, ref):
    """Every (re, im) pair within 2^-6 of its length; returns the fraction of identical elements."""
    got = got.float().cpu().numpy()
    d = np.linalg.norm((got - ref).reshape(ref.shape[0], -1, 2), axis=-1)
    n = np.linalg.norm(ref.reshape(ref.shape[0], -1, 2), axis=-1)
    assert (d <= 2.0 ** -6 * n + 1e-30).all(), float((d / np.maximum(n, 1e-30)).max())
    return float((got == ref).mean())


# heads 4, 8, 12, 16, 20: the kernel's register sizing (16-byte vectors per lane) 1, 2, 3, 4 and 5
@pytest.mark.parametrize("f,h,w,heads,t0", [(2, 16, 24, 12, 5), (4, 8, 8, 4, 0), (2, 72, 120, 12, 8),
                                            (2, 8, 8, 8, 1), (2, 8, 16, 16, 2), (2, 8, 8, 20, 0)])
def test_epilogue_bf16_vs_oracle(dev, f, h, w, heads, t0):
    q, k, v, wq, wk = _inputs(f, h, w, heads, torch.bfloat16, seed=f * 1000 + t0)
    qo, ko, vo = fvsr_lcsa.qkv_epilogue(q.to(dev), k.to(dev), v.to(dev), f, h, w, heads, t0, wq.to(dev), wk.to(dev))
    torch.cuda.synchronize()
    rq, rk, rv = O.qkv_epilogue(q.float().numpy(), k.float().numpy(), v.float().numpy(), f, h, w, heads, t0,
                                wq.float().numpy(), wk.float().numpy())
    np.testing.assert_array_equal(vo.float().cpu().numpy(), rv)
    assert _close_pairs(qo, rq) >= 0.99
    assert _close_pairs(ko, rk) >= 0.99


@pytest.mark.parametrize("heads", [12, 4])   # 16-byte vectors per lane: 6 and 2
def test_epilogue_fp32_vs_oracle(dev, heads):
    f, h, w, t0 = 2, 16, 16, 3
    q, k, v, wq, wk = _inputs(f, h, w, heads, torch.float32, seed=7)
    qo, ko, vo = fvsr_lcsa.qkv_epilogue(q.to(dev), k.to(dev), v.to(dev), f, h, w, heads, t0, wq.to(dev), wk.to(dev))
    rq, rk, rv = O.qkv_epilogue(q.numpy(), k.numpy(), v.numpy(), f, h, w, heads, t0, wq.numpy(), wk.numpy(),
                                bf16=False)
    np.testing.assert_array_equal(vo.cpu().numpy(), rv)
    for got, ref in ((qo, rq), (ko, rk)):
        rel = O.compare(got.cpu().numpy(), ref)["rel"]
        assert rel <= 2e-6, rel


def test_ring_append_qkv_equals_plain_epilogue(dev):
    """Chunk 0 (3 slices) then one streaming chunk (1 slice), reference geometry scaled down (bh 3, bw 4): the ring
    holds exactly the plain epilogue's K/V, its pooled keys select exactly as the plain keys do, Q is the same."""
    heads, bh, bw = 12, 3, 4
    h, w, s = 8 * bh, 8 * bw, bh * bw
    ring = fvsr_lcsa.KVRing(1, heads, bh, bw, capacity=4, kv_len=3, dtype=torch.bfloat16)
    local = fvsr_lcsa.local_block_mask(bh, bw, 3)
    held_k, held_v = [], []
    for n, t0, seed in ((3, 0, 11), (1, 6, 12)):
        f = 2 * n
        q, k, v, wq, wk = (t.to(dev) for t in _inputs(f, h, w, heads, torch.bfloat16, seed))
        qp, kp, vp = fvsr_lcsa.qkv_epilogue(q, k, v, f, h, w, heads, t0, wq, wk)
        qr = ring.append_qkv(0, q, k, v, n, t0, wq, wk)
        torch.cuda.synchronize()
        assert torch.equal(qr, qp)
        held_k.append(kp)
        held_v.append(vp)
        rk, rv = ring.read(0)
        assert torch.equal(rk, torch.cat(held_k)) and torch.equal(rv, torch.cat(held_v))
        topk = 5 * n
        m_ring, p_ring, _, _ = ring.select(0, qr, n, local, topk)
        m_plain, p_plain, _, _ = fvsr_lcsa.draft_block_mask_and_probs(qp, rk, heads, n, s, local, topk)
        assert torch.equal(p_ring, p_plain) and torch.equal(m_ring, m_plain)
        ring.evict(0)
    ring.close()


def test_epilogue_rejects_bad_geometry(dev):
    q = torch.zeros((2 * 8 * 8, 1536), dtype=torch.bfloat16, device=dev)
    wq = torch.ones(1536, dtype=torch.bfloat16, device=dev)
    with pytest.raises(fvsr_lcsa.FVSRError):
        fvsr_lcsa.qkv_epilogue(q, q, q, 2, 8, 6, 12, 0, wq, wq)        # w not a multiple of 8
    with pytest.raises(fvsr_lcsa.FVSRError):
        fvsr_lcsa.qkv_epilogue(q, q, q, 2, 8, 8, 12, 1023, wq, wq)     # positions past the 1024-row tables


def test_epilogue_width_limit_is_checked_before_launch(dev):
    """A token of at most 384 16-byte vectors (64 lanes x 6 registers) runs; a wider one is refused by validation
    with FVSR_ERR_UNSUPPORTED. fp32: 12 heads = 384 vectors run, 13 heads = 416 vectors are refused."""
    for heads, ok in ((12, True), (13, False)):
        c = heads * 128
        q = torch.randn((2 * 8 * 8, c), device=dev)
        w = torch.ones(c, device=dev)
        if ok:
            qo, _, _ = fvsr_lcsa.qkv_epilogue(q, q, q, 2, 8, 8, heads, 0, w, w)
            torch.cuda.synchronize()
            assert torch.isfinite(qo).all()
        else:
            with pytest.raises(fvsr_lcsa.FVSRError, match="384") as ei:
                fvsr_lcsa.qkv_epilogue(q, q, q, 2, 8, 8, heads, 0, w, w)
            assert ei.value.status == 2


def test_ring_append_qkv_wrapping_append(dev):
    """An append whose slices wrap past the ring's last slot (capacity 4, kv_len 2: slices 3 and 0) is pooled in two
    pieces; the held window and its pooled keys still equal the plain epilogue's."""
    heads, bh, bw = 4, 2, 3
    h, w, s = 8 * bh, 8 * bw, bh * bw
    ring = fvsr_lcsa.KVRing(1, heads, bh, bw, capacity=4, kv_len=2, dtype=torch.bfloat16)
    local = fvsr_lcsa.local_block_mask(bh, bw, 3)
    window_k, window_v = [], []
    for n, t0, seed in ((2, 0, 21), (1, 4, 22), (2, 6, 23)):
        f = 2 * n
        q, k, v, wq, wk = (t.to(dev) for t in _inputs(f, h, w, heads, torch.bfloat16, seed))
        qp, kp, vp = fvsr_lcsa.qkv_epilogue(q, k, v, f, h, w, heads, t0, wq, wk)
        qr = ring.append_qkv(0, q, k, v, n, t0, wq, wk)
        window_k += list(kp.split(s * 128))
        window_v += list(vp.split(s * 128))
        rk, rv = ring.read(0)
        assert torch.equal(qr, qp)
        assert torch.equal(rk, torch.cat(window_k)) and torch.equal(rv, torch.cat(window_v))
        m_ring, p_ring, _, _ = ring.select(0, qr, n, local, 4)
        m_plain, p_plain, _, _ = fvsr_lcsa.draft_block_mask_and_probs(qp, rk, heads, n, s, local, 4)
        assert torch.equal(p_ring, p_plain) and torch.equal(m_ring, m_plain)
        ring.evict(0)
        while len(window_k) > ring.slices(0):
            window_k.pop(0)
            window_v.pop(0)
    ring.close()


@pytest.mark.parametrize("bh,bw,heads", [(3, 4, 12), (9, 15, 12)])
def test_layer_call_from_projections_equals_manual_sequence(dev, bh, bw, heads):
    """fvsr_lcsa_layer_qkv (epilogue into the ring, select, attend, evict, output in natural order) equals the plain
    epilogue followed by the window-order layer call and a window reverse, bit for bit, over chunk 0 (3 slices) and
    two streaming chunks."""
    h, w, s = 8 * bh, 8 * bw, bh * bw
    local = fvsr_lcsa.local_block_mask(bh, bw, 11)
    ring_a = fvsr_lcsa.KVRing(1, heads, bh, bw, capacity=4, kv_len=3, dtype=torch.bfloat16)
    ring_b = fvsr_lcsa.KVRing(1, heads, bh, bw, capacity=4, kv_len=3, dtype=torch.bfloat16)
    for n, t0, seed in ((3, 0, 31), (1, 6, 32), (1, 8, 33)):
        f = 2 * n
        q, k, v, wq, wk = (t.to(dev) for t in _inputs(f, h, w, heads, torch.bfloat16, seed))
        topk = int(s * s * 0.5) - 1
        o_a, m_a, _ = ring_a.layer_call_qkv(0, q, k, v, n, t0, wq, wk, local, topk, want_mask=True)
        qp, kp, vp = fvsr_lcsa.qkv_epilogue(q, k, v, f, h, w, heads, t0, wq, wk)
        o_b, m_b, _ = ring_b.layer_call(0, qp, kp, vp, n, n, local, topk, want_mask=True)
        torch.cuda.synchronize()
        assert torch.equal(m_a, m_b)
        assert torch.equal(o_a, fvsr_lcsa.window_reverse(o_b, f, h, w))
        assert ring_a.slices(0) == ring_b.slices(0)
    ring_a.close()
    ring_b.close()
