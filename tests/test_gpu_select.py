"""GPU parity of the block selection (lcsa_select) through the C ABI, against the oracle.

Bar: the block mask is bit-exact wherever the top-k threshold has a margin (relative gap to its nearest neighbour)
well above fp32 rounding; where a row has a near-tie, any flip must satisfy the reference's near-tie rule
(Gates.swift:239-277). Probabilities agree to rel <= 1e-5. kidx/kcnt are the mask's compacted lists
(SparseAttention.swift:175-177).
"""
import os

import numpy as np
import pytest
import torch

import fvsr_lcsa
from fvsr_lcsa import synth
from oracle import lcsa as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "lcsa_tiny.npz")
TIE_FREE = 1e-4


def check_lists(mask, kidx, kcnt):
    m = mask.cpu().numpy() > 0.5
    ki, kc = kidx.cpu().numpy(), kcnt.cpu().numpy()
    np.testing.assert_array_equal(kc, m.sum(-1))
    want_kidx, _ = O.block_lists(m.astype(np.float32))
    np.testing.assert_array_equal(ki, want_kidx)


def check_mask(mask, ref_mask, ref_probs, q_slices, topk):
    got = mask.cpu().numpy()
    margin = O.threshold_margin(ref_probs, q_slices, topk)
    if margin > TIE_FREE:
        np.testing.assert_array_equal(got, ref_mask)
    else:
        rep = O.mask_flip_report(got, ref_mask, ref_probs, q_slices)
        assert rep["legit"], rep
    return margin


def test_golden_fixture_select(dev):
    g = np.load(GOLDEN)
    heads, q_slices, s, topk = (int(x) for x in g["meta"])
    q, k = torch.from_numpy(g["q"]).to(dev), torch.from_numpy(g["k"]).to(dev)
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q, k, heads, q_slices, s, g["local"], topk)
    np.testing.assert_array_equal(mask.cpu().numpy(), g["mask"])
    assert O.compare(probs.cpu().numpy(), g["probs"])["rel"] <= 1e-5
    check_lists(mask, kidx, kcnt)


def test_golden_fixture_select_bf16_inputs(dev):
    g = np.load(GOLDEN)
    heads, q_slices, s, topk = (int(x) for x in g["meta"])
    q = torch.from_numpy(g["q"]).to(dev).to(torch.bfloat16)
    k = torch.from_numpy(g["k"]).to(dev).to(torch.bfloat16)
    mask, probs, _, _ = fvsr_lcsa.draft_block_mask_and_probs(q, k, heads, q_slices, s, g["local"], topk)
    np.testing.assert_array_equal(mask.cpu().numpy(), g["mask"])


def test_draft_mask_kat(dev):
    """FlashVSRStructureTests.swift:60-75 on the GPU: topk 1 keeps nothing, topk 2 keeps [1, 0, 1, 0]."""
    q = torch.ones((2 * 128, 128), device=dev)
    k = torch.zeros((2 * 128, 128), device=dev)
    k[:128] = 2.0
    local = np.ones((2, 2), dtype=bool)
    m1 = fvsr_lcsa.draft_block_mask(q, k, 1, 1, 2, local, 1)
    assert m1.sum().item() == 0
    m2 = fvsr_lcsa.draft_block_mask(q, k, 1, 1, 2, local, 2)
    assert m2.reshape(-1).tolist() == [1, 0, 1, 0]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_c1_select(dev, seed):
    """512x512 fp32 (s = 16, Nq 16, Nk 48, local 3, 50% of in-window pairs)."""
    wl = synth.WORKLOADS["lcsa_512x512_fp32"]
    q, k, _ = synth.make_qkv(wl, seed=seed)
    local = synth.local_mask(wl).numpy()
    topk = synth.workload_topk(wl)
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q.numpy(), k.numpy(), wl.heads, wl.q_slices, wl.s, local,
                                                       topk)
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q.to(dev), k.to(dev), wl.heads, wl.q_slices,
                                                                   wl.s, local, topk)
    assert O.compare(probs.cpu().numpy(), ref_probs)["rel"] <= 1e-5
    check_mask(mask, ref_mask, ref_probs, wl.q_slices, topk)
    check_lists(mask, kidx, kcnt)


def test_c3_select_tie_free_is_bit_exact(dev):
    """1280x768 bf16 with a smooth field + noise, at the workload's seed: every top-k row has a margin >= 1e-3 (the
    BASELINE 'no ties within 1e-3' condition), and the GPU mask must equal the oracle's bit for bit."""
    wl = synth.WORKLOADS["sparse_1280x768_bf16"]
    local = synth.local_mask(wl).numpy()
    topk = synth.workload_topk(wl)
    q, k, _ = synth.make_qkv(wl)
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q.float().numpy(), k.float().numpy(), wl.heads,
                                                       wl.q_slices, wl.s, local, topk)
    assert O.threshold_margin(ref_probs, wl.q_slices, topk) >= 1e-3
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q.to(dev), k.to(dev), wl.heads, wl.q_slices,
                                                                   wl.s, local, topk)
    np.testing.assert_array_equal(mask.cpu().numpy(), ref_mask)
    assert (kcnt.sum(1).cpu().numpy() == topk).all()      # exactly topk kept per (head, slice) row
    check_lists(mask, kidx, kcnt)


C4_MARGIN = 5e-5   # relative gap at every top-k threshold of the 1920x1152 workload (~400 fp32 ulps)


def near_threshold_rel(got, ref, q_slices, topk):
    """Largest per-element relative difference of the probabilities over the entries within a factor 2 of their
    (head, slice) row's top-k threshold: the entries whose order decides the mask."""
    h, nq, nk = ref.shape
    g = got.reshape(h * q_slices, -1).astype(np.float64)
    r = ref.reshape(h * q_slices, -1).astype(np.float64)
    n = r.shape[1]
    thr = np.sort(r, axis=1)[:, n - 1 - min(n - 1, topk)][:, None]
    near = (r >= thr / 2) & (r <= thr * 2) & (r > 0)
    return float((np.abs(g - r)[near] / r[near]).max())


def test_c4_select_tie_free_is_bit_exact(dev):
    """1920x1152 bf16 (Lk 43200 = 337.5 key blocks, the last pooled over its 64 valid tokens, local 11, 30% of the
    in-window pairs): Q/K a smooth field + noise with RMS norm and 3-D RoPE, at the workload's seed. Every (head,
    slice) threshold is >= 5e-5 (relative) from its upper neighbour, far above the measured per-element difference of
    the probabilities, and the GPU mask must equal the oracle's bit for bit (DiT.swift:158-174). The mask is not
    degenerate: rows differ between heads and fewer than 10 % select nothing."""
    wl = synth.WORKLOADS["sparse_1920x1152_bf16"]
    q, k, _ = synth.make_qkv(wl)
    local = synth.local_mask(wl).numpy()
    topk = synth.workload_topk(wl)
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q.float().numpy(), k.float().numpy(), wl.heads,
                                                       wl.q_slices, wl.s, local, topk, lk=wl.lk)
    margin = O.threshold_margin(ref_probs, wl.q_slices, topk)
    assert margin >= C4_MARGIN
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q.to(dev), k.to(dev), wl.heads, wl.q_slices,
                                                                   wl.s, local, topk)
    assert mask.shape == (wl.heads, 135, 338)
    rel_elem = near_threshold_rel(probs.cpu().numpy(), ref_probs, wl.q_slices, topk)
    print(f"  threshold margin {margin:.3e}, probs rel diff near the thresholds {rel_elem:.3e}", flush=True)
    assert rel_elem <= margin / 8
    np.testing.assert_array_equal(mask.cpu().numpy(), ref_mask)
    kc = kcnt.cpu().numpy()
    assert (kc.reshape(wl.heads * wl.q_slices, -1).sum(1) == topk).all()
    assert (kc == 0).mean() < 0.1
    assert any(not np.array_equal(kc[0], kc[h]) for h in range(1, wl.heads))
    check_lists(mask, kidx, kcnt)


def test_c4_iid_select_near_ties(dev):
    """The same geometry with i.i.d. N(0,1) Q/K: pooling 128 independent tokens leaves no signal, so the
    probabilities of a row cluster within a few ulps and the threshold margin is ~1e-6. The mask must equal the
    oracle's except at near-ties, where any flip must satisfy the reference's near-tie rule (Gates.swift:239-277)."""
    wl = synth.WORKLOADS["sparse_1920x1152_bf16_iid"]
    q, k, _ = synth.make_qkv(wl)
    local = synth.local_mask(wl).numpy()
    topk = synth.workload_topk(wl)
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q.float().numpy(), k.float().numpy(), wl.heads,
                                                       wl.q_slices, wl.s, local, topk, lk=wl.lk)
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q.to(dev), k.to(dev), wl.heads, wl.q_slices,
                                                                   wl.s, local, topk)
    assert O.compare(probs.cpu().numpy(), ref_probs)["rel"] <= 1e-5
    check_mask(mask, ref_mask, ref_probs, wl.q_slices, topk)
    check_lists(mask, kidx, kcnt)


def test_topk_beyond_row_length_keeps_all_above_minimum(dev):
    gen = torch.Generator().manual_seed(3)
    q = torch.randn((4 * 128, 256), generator=gen)
    k = torch.randn((8 * 128, 256), generator=gen)
    local = O.local_block_mask(2, 2, 3)
    ref_mask, _ = O.draft_block_mask_and_probs(q.numpy(), k.numpy(), 2, 1, 4, local, 10_000)
    mask = fvsr_lcsa.draft_block_mask(q.to(dev), k.to(dev), 2, 1, 4, local, 10_000)
    np.testing.assert_array_equal(mask.cpu().numpy(), ref_mask)


@pytest.mark.parametrize("topk", [2_000, 44_000])
def test_threshold_bin_paths_1920x1152_local3(dev, topk):
    """1920x1152 geometry with local range 3: ~94 % of each (head, slice) row of 45630 probs are exact zeros. topk
    2000 puts the threshold among the nonzero probs (the histogram bin is gathered in LDS); topk 44000 puts it on
    the zeros, a bin far larger than the LDS candidate buffer, so the full-row radix select runs."""
    wl = synth.WORKLOADS["sparse_1920x1152_bf16_iid"]
    q, k, _ = synth.make_qkv(wl, seed=1)
    local = O.local_block_mask(wl.bh, wl.bw, 3)
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q.float().numpy(), k.float().numpy(), wl.heads,
                                                       wl.q_slices, wl.s, local, topk, lk=wl.lk)
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q.to(dev), k.to(dev), wl.heads, wl.q_slices,
                                                                   wl.s, local, topk)
    zeros = float((ref_probs == 0).mean())
    assert zeros > 0.9
    check_mask(mask, ref_mask, ref_probs, wl.q_slices, topk)
    check_lists(mask, kidx, kcnt)


def test_select_rejects_uneven_slices(dev):
    q = torch.zeros((3 * 128, 128), device=dev)
    k = torch.zeros((4 * 128, 128), device=dev)
    with pytest.raises(fvsr_lcsa.FVSRError) as ei:
        fvsr_lcsa.draft_block_mask(q, k, 1, 2, 2, np.ones((2, 2), bool), 1)
    assert ei.value.status == 1


def test_long_rows_take_the_streaming_paths(dev):
    """One head, 300 blocks per slice, 300 query x 1200 key blocks: rows longer than the emit kernel keeps in
    registers (768 key blocks), a local window wider than the scores kernel's one-pass byte staging (256 columns) and
    a (head, slice) row of 360,000 probs, more than 64 threshold workgroups hold in registers (each then reads its
    share twice). Block means with a wide spread (+ token noise) keep the probabilities apart, so the mask is
    checked as every other: bit-exact where the threshold has a margin, the near-tie rule elsewhere."""
    g = torch.Generator().manual_seed(7)
    s, nq, nk = 300, 300, 1200
    qb = 3.0 * torch.randn((nq, 1, 128), generator=g)
    kb = 3.0 * torch.randn((nk, 1, 128), generator=g)
    q = (qb + torch.randn((nq, 128, 128), generator=g)).reshape(-1, 128)
    k = (kb + torch.randn((nk, 128, 128), generator=g)).reshape(-1, 128)
    yy, xx = np.divmod(np.arange(s), 20)   # a 15 x 20 block grid, local range 7
    local = (np.abs(yy[:, None] - yy[None, :]) <= 3) & (np.abs(xx[:, None] - xx[None, :]) <= 3)
    topk = 20000   # of 47,616 in-window pairs
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q.numpy(), k.numpy(), 1, 1, s, local, topk)
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q.to(dev), k.to(dev), 1, 1, s, local, topk)
    assert O.compare(probs.cpu().numpy(), ref_probs)["rel"] <= 1e-5
    check_mask(mask, ref_mask, ref_probs, 1, topk)
    check_lists(mask, kidx, kcnt)
    assert int(kcnt.sum()) == int(ref_mask.sum())


def test_threshold_on_exact_ties_in_a_large_bin(dev):
    """Sixteen query blocks with zero queries score every key block alike, so their 5408 probs tie at exactly 1/338
    and the (k+1)-th largest (k = 3000, with 2109 probs above the tie) falls on them: the threshold's bin holds 5442
    candidates, most of them in the shares of the row's first two workgroups. The mask keeps the 2109 probs strictly
    above the tie, as the oracle's."""
    g = torch.Generator().manual_seed(3)
    s, nq, nk = 135, 135, 338
    q = torch.randn((nq, 128, 128), generator=g) + 2.0 * torch.randn((nq, 1, 128), generator=g)
    k = torch.randn((nk, 128, 128), generator=g) + 2.0 * torch.randn((nk, 1, 128), generator=g)
    q[:16] = 0.0
    q, k = q.reshape(-1, 128), k.reshape(-1, 128)
    local = np.ones((s, s), dtype=bool)
    topk = 3000
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q.numpy(), k.numpy(), 1, 1, s, local, topk)
    tie = np.float32(1.0) / np.float32(nk)
    assert int((ref_probs == tie).sum()) == 16 * nk and int((ref_probs > tie).sum()) < topk + 1
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(q.to(dev), k.to(dev), 1, 1, s, local, topk)
    assert O.compare(probs.cpu().numpy(), ref_probs)["rel"] <= 1e-5
    check_mask(mask, ref_mask, ref_probs, 1, topk)
    check_lists(mask, kidx, kcnt)
    assert int(mask.sum()) == int((ref_probs > tie).sum())
