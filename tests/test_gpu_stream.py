"""The streaming attention stack at the real 1920x1152 geometry against the oracle, chunk by chunk.

Geometry: 12 heads x 128, s = 9 x 15 = 135 blocks per temporal slice; a first chunk of 3 slices, then 4 chunks of 1
slice (Pipeline.swift:95-102); a KV window of 3 slices (DiT.swift:507-538, kvLen 3, Pipeline.swift:129); the
reference's default top-k 16199 (DiT.swift:482, Pipeline.swift:68) and local range 11. Two layers share one KV ring,
each with its own projections, and every layer call starts from the q/k/v projections (fvsr_lcsa_layer_qkv:
WanRMSNorm + 3-D RoPE + window partition + ring append + selection + attention + evict + window reverse,
DiT.swift:496-539). The projections are a smooth field over the 14 latent frames plus noise, with norm weights of
about 2, so every top-k threshold of the schedule has a clear margin.

Per chunk and layer, against the oracle:
  - the epilogue on 512 sampled tokens of Q' and of the new K' (the bfloat16 bar of test_gpu_epilogue: pairs within
    2^-6 of their length), V copied exactly;
  - the ring contents after the evict against the oracle's concat-then-trim cache fed the same new keys/values
    (bit-exact);
  - the block mask against the oracle's selection over the same Q' and key window (bit-exact; every (head, slice)
    row has a threshold margin >= 1e-5, several times the ~1.6e-6 per-element difference of the probabilities);
  - one query block of every head (output in natural token order) against the float64 oracle attention
    (rel <= 1e-2).
"""
import numpy as np
import pytest
import torch

import fvsr_lcsa
from fvsr_lcsa import synth
from oracle import lcsa as O

pytestmark = pytest.mark.gpu

H, BH, BW = 12, 9, 15
S, C = BH * BW, H * 128
LH, LW = 8 * BH, 8 * BW
FRAMES = 14
CHUNKS = [(3, 0), (1, 6), (1, 8), (1, 10), (1, 12)]   # (new slices, first latent frame)
LAYER_SEEDS = (2, 13)
NOISE, WSCALE = 0.5, 2.0
MARGIN = 1e-5
BF16_REL = 1e-2


def projections(seed):
    """Seeded q/k/v projections of every chunk, natural (f, h, w) token order, bfloat16, and the two norm weights."""
    gen = torch.Generator().manual_seed(seed)
    field = synth.smooth_field(FRAMES, LH, LW, C, gen)
    wq = (WSCALE * (0.75 + 0.5 * torch.rand(C, generator=gen))).to(torch.bfloat16)
    wk = (WSCALE * (0.75 + 0.5 * torch.rand(C, generator=gen))).to(torch.bfloat16)
    vgen = torch.Generator().manual_seed(seed + 1000)
    chunks = []
    for n, t0 in CHUNKS:
        f = 2 * n
        sl = slice(t0 * LH * LW, (t0 + f) * LH * LW)
        q = (field[sl] + NOISE * torch.randn((f * LH * LW, C), generator=gen)).to(torch.bfloat16)
        k = (field[sl] + NOISE * torch.randn((f * LH * LW, C), generator=gen)).to(torch.bfloat16)
        v = torch.randn((f * LH * LW, C), generator=vgen).to(torch.bfloat16)
        chunks.append((q, k, v))
    return chunks, wq, wk


def window_rows(f):
    """(natural index of each window-order row, window-order row of each natural token) for an (f, LH, LW) grid."""
    L = f * LH * LW
    nat_of_win = O.window_partition(np.arange(L, dtype=np.int64).reshape(1, L, 1), f, LH, LW).reshape(-1)
    return nat_of_win, np.argsort(nat_of_win)


def check_epilogue_rows(got_win, x_nat, weight, f, t0, win_of_nat, rng):
    """The oracle epilogue (WanRMSNorm, then RoPE at the tokens' positions) on 512 sampled tokens."""
    t = rng.choice(f * LH * LW, 512, replace=False)
    cos, sin = O.rope_grid(f, LH, LW, t0)
    ref = O.rope_apply(O.wan_rms_norm(x_nat[t], weight), H, cos[t], sin[t])
    got = got_win[win_of_nat[t]]
    d = np.linalg.norm((got - ref).reshape(len(t), -1, 2), axis=-1)
    nrm = np.linalg.norm(ref.reshape(len(t), -1, 2), axis=-1)
    assert (d <= 2.0 ** -6 * nrm + 1e-30).all(), float((d / np.maximum(nrm, 1e-30)).max())
    assert (got == ref).mean() >= 0.99


def test_streaming_stack_1920x1152_two_layers_vs_oracle(dev):
    local = O.local_block_mask(BH, BW, 11)
    topk = O.step_topk(S, O.default_topk_ratio(1152, 1920))
    assert topk == 16199
    rng = np.random.default_rng(0)
    layers = [projections(seed) for seed in LAYER_SEEDS]
    ring = fvsr_lcsa.KVRing(len(layers), H, BH, BW, capacity=4, kv_len=3, dtype=torch.bfloat16,
                            device=dev.index or 0)
    caches = [O.KVWindowCache(kv_len=3) for _ in layers]
    try:
        for c, (n, t0) in enumerate(CHUNKS):
            f = 2 * n
            nat_of_win, win_of_nat = window_rows(f)
            for layer, (chunks, wq, wk) in enumerate(layers):
                print(f"  chunk {c} (slices {n}, t0 {t0}) layer {layer}", flush=True)
                q, k, v = chunks[c]
                qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
                qw = torch.empty_like(qd)
                o, mask, _ = ring.layer_call_qkv(layer, qd, kd, vd, n, t0, wq.to(dev), wk.to(dev), local, topk,
                                                 q_work=qw, want_mask=True)
                kh, vh = ring.read(layer)
                torch.cuda.synchronize()
                qw_h = qw.float().cpu().numpy()
                kh_h, vh_h = kh.float().cpu().numpy(), vh.float().cpu().numpy()
                # the epilogue: Q' and the new K' (the ring's last n slices) on sampled tokens, V exactly
                new = slice(kh_h.shape[0] - n * S * 128, kh_h.shape[0])
                check_epilogue_rows(qw_h, q.float().numpy(), wq.float().numpy(), f, t0, win_of_nat, rng)
                check_epilogue_rows(kh_h[new], k.float().numpy(), wk.float().numpy(), f, t0, win_of_nat, rng)
                np.testing.assert_array_equal(vh_h[new], v.float().numpy()[nat_of_win])
                # the window cache: concat then trim, fed the same new keys and values
                cache = caches[layer]
                k_att, v_att = cache.attend_view(kh_h[new].reshape(-1, 128, C), vh_h[new].reshape(-1, 128, C), n)
                cache.trim()
                np.testing.assert_array_equal(kh_h, cache.k.reshape(-1, C))
                np.testing.assert_array_equal(vh_h, cache.v.reshape(-1, C))
                k_att, v_att = k_att.reshape(-1, C), v_att.reshape(-1, C)
                assert k_att.shape[0] == (3 if c == 0 else 4) * S * 128
                # the selection over Q' and the window
                ref_mask, ref_probs = O.draft_block_mask_and_probs(qw_h, k_att, H, n, S, local, topk)
                margin = O.threshold_margin(ref_probs, n, topk)
                print(f"    threshold margin {margin:.2e}, kept {int(ref_mask.sum())} block pairs", flush=True)
                assert margin >= MARGIN
                np.testing.assert_array_equal(mask.cpu().numpy(), ref_mask)
                # one query block per head, output in natural token order
                o_h = o.float().cpu().numpy()
                worst = 0.0
                for h in range(H):
                    b = (37 * h + 11 * c + 5 * layer) % (n * S)
                    ref = O.block_masked_attention(qw_h, k_att, v_att, ref_mask, H, heads_subset=[h],
                                                   qblocks_subset=[b])
                    rows = slice(b * 128, (b + 1) * 128)
                    cols = slice(h * 128, (h + 1) * 128)
                    got = o_h[nat_of_win[rows], cols]
                    worst = max(worst, O.compare(got, ref[rows, cols])["rel"])
                print(f"    attention rel {worst:.2e}", flush=True)
                assert worst <= BF16_REL
                assert ring.slices(layer) == 3
    finally:
        ring.close()
