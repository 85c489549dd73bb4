"""GPU parity of the KV ring (append / evict / read) and the window layout kernels, against the oracle's
KVWindowCache (DiT.swift:507-511,532-538) and window_partition (DiT.swift:113-126).

The ring must hold exactly what the reference's concat-then-trim cache holds after every chunk of the streaming
schedule (chunk 0: 3 slices; chunks 1..4: 1 slice each; kv_len 3), and selection / attention over the ring must equal
the same calls over the plain concatenated buffers bit for bit (same kernels, same data, same key order).
"""
import numpy as np
import pytest
import torch

import fvsr_lcsa
from fvsr_lcsa import synth
from oracle import lcsa as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_window_partition_and_reverse(dev, dtype):
    f, h, w, c = 4, 16, 24, 256
    x = torch.randn((f * h * w, c)).to(dtype)
    p = fvsr_lcsa.window_partition(x.to(dev), f, h, w)
    ref = O.window_partition(x.float().numpy()[None], f, h, w).reshape(-1, c)
    np.testing.assert_array_equal(p.float().cpu().numpy(), ref)
    r = fvsr_lcsa.window_reverse(p, f, h, w)
    assert torch.equal(r.cpu(), x)


def _chunks(heads, bh, bw, dtype, schedule=(3, 1, 1, 1, 1), seed=0):
    s = bh * bw
    gen = torch.Generator().manual_seed(seed)
    out = []
    for n in schedule:
        L = n * s * 128
        out.append((n, torch.randn((L, heads * 128), generator=gen).to(dtype),
                    torch.randn((L, heads * 128), generator=gen).to(dtype)))
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_ring_follows_reference_cache_schedule(dev, dtype):
    heads, bh, bw = 2, 2, 3
    ring = fvsr_lcsa.KVRing(layers=2, heads=heads, bh=bh, bw=bw, capacity=4, kv_len=3, dtype=dtype)
    ref = O.KVWindowCache(kv_len=3)
    for n, kn, vn in _chunks(heads, bh, bw, dtype):
        layer = 1
        ring.append(layer, kn.to(dev), vn.to(dev), n)
        kview, vview = ref.attend_view(kn.float().numpy().reshape(-1, 128, heads * 128),
                                       vn.float().numpy().reshape(-1, 128, heads * 128), n)
        k_att, v_att = ring.read(layer)
        np.testing.assert_array_equal(k_att.float().cpu().numpy(), kview.reshape(-1, heads * 128))
        np.testing.assert_array_equal(v_att.float().cpu().numpy(), vview.reshape(-1, heads * 128))
        ring.evict(layer)
        ref.trim()
        k_c, v_c = ring.read(layer)
        np.testing.assert_array_equal(k_c.float().cpu().numpy(), ref.k.reshape(-1, heads * 128))
        np.testing.assert_array_equal(v_c.float().cpu().numpy(), ref.v.reshape(-1, heads * 128))
        assert ring.slices(layer) == ref.k.shape[0] // (bh * bw)
    assert ring.slices(0) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_select_and_attention_over_ring_equal_plain(dev, dtype):
    heads, bh, bw, r = 2, 2, 3, 3
    s = bh * bw
    local = O.local_block_mask(bh, bw, r)
    ring = fvsr_lcsa.KVRing(layers=1, heads=heads, bh=bh, bw=bw, capacity=4, kv_len=3, dtype=dtype)
    chunks = _chunks(heads, bh, bw, dtype, schedule=(3, 1, 1))
    gen = torch.Generator().manual_seed(9)
    for step, (n, kn, vn) in enumerate(chunks):
        ring.append(0, kn.to(dev), vn.to(dev), n)
        q = torch.randn((n * s * 128, heads * 128), generator=gen).to(dtype).to(dev)
        kall, vall = ring.read(0)
        topk = 4 * n * s
        m1, p1, ki1, kc1 = ring.select(0, q, n, local, topk)
        m2, p2, ki2, kc2 = fvsr_lcsa.draft_block_mask_and_probs(q, kall, heads, n, s, local, topk)
        assert torch.equal(p1, p2) and torch.equal(m1, m2)
        assert torch.equal(ki1, ki2) and torch.equal(kc1, kc2)
        o1 = ring.attention(0, q, ki1, kc1, fvsr_lcsa.ATTN_KERNEL)
        o2 = fvsr_lcsa.block_sparse_attention(q, kall, vall, ki2, kc2, heads)
        o3 = ring.attention(0, q, ki1, kc1, fvsr_lcsa.ATTN_DENSE)
        assert torch.equal(o1, o2) and torch.equal(o1, o3)
        ring.evict(0)


# AUTO with top-k 3 n s keeps an expected (3 n s + 1) / (s nk) of the pairs: over 0.45 in chunk 0 (dense walk), under
# it afterwards (the kernel walk); both walks give the kernel's result bit for bit (DiT.swift:517-522)
@pytest.mark.parametrize("mode", ["kernel", "auto"])
def test_layer_call_equals_manual_sequence(dev, mode):
    heads, bh, bw, r = 2, 2, 2, 3
    s = bh * bw
    local = O.local_block_mask(bh, bw, r)
    dtype = torch.bfloat16
    ring_a = fvsr_lcsa.KVRing(1, heads, bh, bw, 4, 3, dtype)
    ring_b = fvsr_lcsa.KVRing(1, heads, bh, bw, 4, 3, dtype)
    gen = torch.Generator().manual_seed(21)
    call_mode = fvsr_lcsa.ATTN_KERNEL if mode == "kernel" else fvsr_lcsa.ATTN_AUTO
    for n, kn, vn in _chunks(heads, bh, bw, dtype, schedule=(3, 1, 1, 1)):
        q = torch.randn((n * s * 128, heads * 128), generator=gen).to(dtype).to(dev)
        kd, vd = kn.to(dev), vn.to(dev)
        topk = 3 * n * s
        o_a, m_a, p_a = ring_a.layer_call(0, q, kd, vd, n, n, local, topk, mode=call_mode,
                                          want_mask=True, want_probs=True)
        ring_b.append(0, kd, vd, n)
        m_b, p_b, ki, kc = ring_b.select(0, q, n, local, topk)
        o_b = ring_b.attention(0, q, ki, kc, fvsr_lcsa.ATTN_KERNEL)
        ring_b.evict(0)
        assert torch.equal(m_a, m_b) and torch.equal(p_a, p_b) and torch.equal(o_a, o_b)
        assert ring_a.slices(0) == ring_b.slices(0)


def test_grid_layout_append_equals_windows(dev):
    heads, bh, bw = 2, 2, 3
    f, h, w = 2, 8 * bh, 8 * bw
    x = torch.randn((f * h * w, heads * 128), device=dev)
    y = torch.randn((f * h * w, heads * 128), device=dev)
    ra = fvsr_lcsa.KVRing(1, heads, bh, bw, 4, 3, torch.float32)
    rb = fvsr_lcsa.KVRing(1, heads, bh, bw, 4, 3, torch.float32)
    ra.append(0, x, y, 1, layout=fvsr_lcsa.LAYOUT_GRID)
    rb.append(0, fvsr_lcsa.window_partition(x, f, h, w), fvsr_lcsa.window_partition(y, f, h, w), 1)
    ka, va = ra.read(0)
    kb, vb = rb.read(0)
    assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_ring_errors(dev):
    ring = fvsr_lcsa.KVRing(1, 1, 1, 2, capacity=4, kv_len=3, dtype=torch.float32)
    q = torch.zeros((2 * 128, 128), device=dev)
    with pytest.raises(fvsr_lcsa.FVSRError) as ei:
        ring.select(0, q, 1, np.ones((2, 2), bool), 1)
    assert ei.value.status == 6                      # empty ring
    kv = torch.zeros((5 * 2 * 128, 128), device=dev)
    with pytest.raises(fvsr_lcsa.FVSRError) as ei:
        ring.append(0, kv, kv, 5)
    assert ei.value.status == 5                      # capacity
    with pytest.raises(fvsr_lcsa.FVSRError):
        fvsr_lcsa.KVRing(1, 1, 1, 2, capacity=3, kv_len=3)
