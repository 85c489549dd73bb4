"""GPU parity of the block-sparse attention (lcsa_attn) through the C ABI, against the oracle.

Bars (written in each test): fp32 rel <= 1e-5, bf16 rel <= 1e-2 against the float64 oracle on the same (bf16-valued)
inputs, rel = max|got - ref| / max|ref| (Gates.swift:19-29). The kernel and its dense fallback must agree exactly.
The reference's own probe protocol (Diag.swift:86-121: random masks at 0.3-0.6 density with a forced empty query
block, fp32 and bf16) is reproduced.
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
FP32_REL = 1e-5
BF16_REL = 1e-2


def _np(t):
    return t.float().cpu().numpy()


def _rel(got, ref):
    return O.compare(_np(got) if isinstance(got, torch.Tensor) else got, ref)["rel"]


def test_golden_fixture_fp32(dev):
    g = np.load(GOLDEN)
    heads = int(g["meta"][0])
    q, k, v = (torch.from_numpy(g[n]).to(dev) for n in ("q", "k", "v"))
    mask = torch.from_numpy(g["mask"]).to(dev)
    o = fvsr_lcsa.kernel_block_attention(q, k, v, mask, heads)
    od = fvsr_lcsa.block_masked_attention(q, k, v, mask, heads)
    assert _rel(o, g["out"]) <= FP32_REL
    assert torch.equal(o, od)


def test_golden_fixture_bf16(dev):
    g = np.load(GOLDEN)
    heads = int(g["meta"][0])
    # fixture inputs are multiples of 1/16 in [-4, 4]: exact in bf16
    q, k, v = (torch.from_numpy(g[n]).to(dev).to(torch.bfloat16) for n in ("q", "k", "v"))
    assert torch.equal(q.float().cpu(), torch.from_numpy(g["q"]))
    mask = torch.from_numpy(g["mask"]).to(dev)
    o = fvsr_lcsa.kernel_block_attention(q, k, v, mask, heads)
    assert o.dtype == torch.bfloat16
    assert _rel(o, g["out"]) <= BF16_REL


@pytest.mark.parametrize("dtype,lqb,lkb,density", [(torch.float32, 4, 6, 0.5), (torch.float32, 12, 36, 0.3),
                                                   (torch.bfloat16, 12, 36, 0.6)])
def test_reference_probe_protocol(dev, dtype, lqb, lkb, density):
    """Diag.swift:87-97: 2 heads, random q/k/v, uniform random block mask, one forced empty query block."""
    heads = 2
    gen = torch.Generator().manual_seed(lqb * 100 + lkb)
    q = torch.randn((lqb * 128, heads * 128), generator=gen).to(dtype)
    k = torch.randn((lkb * 128, heads * 128), generator=gen).to(dtype)
    v = torch.randn((lkb * 128, heads * 128), generator=gen).to(dtype)
    m = (torch.rand((heads, lqb, lkb), generator=gen) < density).float()
    m[0, 1] = 0
    ref = O.block_masked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), m.numpy(), heads)
    o = fvsr_lcsa.FlashVSRAttentionOps.kernel(q.to(dev), k.to(dev), v.to(dev), m.to(dev), heads)
    od = fvsr_lcsa.FlashVSRAttentionOps.dense(q.to(dev), k.to(dev), v.to(dev), m.to(dev), heads)
    bar = FP32_REL if dtype == torch.float32 else BF16_REL
    assert _rel(o, ref) <= bar
    assert torch.equal(o, od)
    assert (o[128:256, :128] == 0).all()          # the forced empty query block


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("lq,lk", [(200, 300), (128, 129), (77, 1000), (384, 64)])
def test_ragged_tails(dev, dtype, lq, lk):
    heads = 2
    gen = torch.Generator().manual_seed(lq + lk)
    q = torch.randn((lq, heads * 128), generator=gen).to(dtype)
    k = torch.randn((lk, heads * 128), generator=gen).to(dtype)
    v = torch.randn((lk, heads * 128), generator=gen).to(dtype)
    nq, nk = -(-lq // 128), -(-lk // 128)
    m = (torch.rand((heads, nq, nk), generator=gen) < 0.7).float()
    m[:, :, -1] = 1                                # always touch the ragged key block
    ref = O.block_masked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), m.numpy(), heads)
    o = fvsr_lcsa.kernel_block_attention(q.to(dev), k.to(dev), v.to(dev), m.to(dev), heads)
    assert o.shape == (lq, heads * 128)
    assert _rel(o, ref) <= (FP32_REL if dtype == torch.float32 else BF16_REL)


@pytest.mark.parametrize("heads,lqb,oracle", [(12, 42, True), (12, 43, True), (4, 129, True), (12, 86, False)])
def test_rows_around_the_persistent_grid(dev, heads, lqb, oracle):
    """Row counts (heads x query blocks) just below, just above and twice the persistent grid of the bf16 walk
    (2 workgroups per CU): every workgroup's first row is dealt by XCD, the rest come from the longest-first queue.
    Row lengths vary from empty to full. The outputs start as NaN, so a row the walk skipped or repeated into the
    wrong place fails; kernel == dense fallback everywhere, and both against the oracle where it is quick."""
    lk = 3 * 128 + 50
    gen = torch.Generator().manual_seed(heads * 1000 + lqb)
    q = torch.randn((lqb * 128, heads * 128), generator=gen).to(torch.bfloat16)
    k = torch.randn((lk, heads * 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((lk, heads * 128), generator=gen).to(torch.bfloat16)
    dens = torch.rand((heads, lqb, 1), generator=gen)   # per-row density: lengths 0 .. 4 blocks
    m = (torch.rand((heads, lqb, 4), generator=gen) < dens).float()
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), m.to(dev)
    o = torch.full((lqb * 128, heads * 128), float("nan"), dtype=torch.bfloat16, device=dev)
    od = torch.full_like(o, float("nan"))
    print(f"  rows {heads * lqb}, kept blocks {int(m.sum())}", flush=True)
    fvsr_lcsa.kernel_block_attention(qd, kd, vd, md, heads, out=o)
    fvsr_lcsa.block_masked_attention(qd, kd, vd, md, heads, out=od)
    torch.cuda.synchronize()
    assert not torch.isnan(o).any()
    assert torch.equal(o, od)
    empty = (m.sum(-1) == 0)                          # (heads, lqb): rows with no listed block are zeros
    ov = o.float().cpu().view(lqb, 128, heads, 128)
    for h, i in empty.nonzero().tolist():
        assert (ov[i, :, h] == 0).all()
    if oracle:
        ref = O.block_masked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), m.numpy(), heads)
        assert _rel(o, ref) <= BF16_REL


def test_list_and_mask_operands_are_checked(dev):
    """The C ABI cannot see buffer sizes: the binding rejects lists, masks and outputs whose extent or device does
    not match the tokens before any pointer reaches a kernel."""
    heads = 2
    q = torch.zeros((256, heads * 128), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((384, heads * 128), dtype=torch.bfloat16, device=dev)
    kidx = torch.zeros((heads, 2, 3), dtype=torch.int32, device=dev)
    kcnt = torch.zeros((heads, 2), dtype=torch.int32, device=dev)
    fvsr_lcsa.block_sparse_attention(q, k, k, kidx, kcnt, heads)          # the right shapes run
    with pytest.raises(fvsr_lcsa.FVSRError, match="kidx"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx[:, :1], kcnt, heads)   # lists of one query block, two needed
    with pytest.raises(fvsr_lcsa.FVSRError, match="kcnt"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx, kcnt[:1], heads)
    with pytest.raises(fvsr_lcsa.FVSRError, match="expected a tensor on"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx.cpu(), kcnt, heads)
    with pytest.raises(fvsr_lcsa.FVSRError, match="elements"):
        fvsr_lcsa.kernel_block_attention(q, k, k, torch.ones((heads, 2, 2), device=dev), heads)   # 3 key blocks


def test_all_empty_mask_gives_zeros(dev):
    heads = 3
    q = torch.randn((256, heads * 128), device=dev)
    k = torch.randn((512, heads * 128), device=dev)
    m = torch.zeros((heads, 2, 4), device=dev)
    o = torch.full_like(q, 7.0)
    fvsr_lcsa.kernel_block_attention(q, k, k, m, heads, out=o)
    assert (o == 0).all()
    o.fill_(7.0)
    fvsr_lcsa.block_masked_attention(q, k, k, m, heads, out=o)
    assert (o == 0).all()


def test_list_order_does_not_change_the_result(dev):
    heads = 2
    gen = torch.Generator().manual_seed(11)
    q = torch.randn((512, heads * 128), generator=gen)
    k = torch.randn((1024, heads * 128), generator=gen)
    v = torch.randn((1024, heads * 128), generator=gen)
    m = (torch.rand((heads, 4, 8), generator=gen) < 0.5).float()
    kidx, kcnt = O.block_lists(m.numpy())
    rev = kidx.copy()
    for h in range(heads):
        for i in range(4):
            c = kcnt[h, i]
            rev[h, i, :c] = kidx[h, i, :c][::-1]
    a = fvsr_lcsa.block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(kidx).to(dev),
                                         torch.from_numpy(kcnt).to(dev), heads)
    b = fvsr_lcsa.block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(rev).to(dev),
                                         torch.from_numpy(kcnt).to(dev), heads)
    assert O.compare(_np(a), _np(b))["rel"] <= 1e-6


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_rows_whose_exponentials_all_underflow_are_redone(dev, dtype):
    """The walk's exact redo (a row-max pass, then attention with that max): a row whose first listed block lies
    outside [0, nk) gets the reference 0 from that all-masked first tile, and when every real score sits ~196 below
    it (log2 units) all of its exponentials underflow to 0. Such rows must still give the softmax over their valid
    blocks, as the oracle computes it (out-of-range entries take no part). Head 1's rows list valid blocks first and
    share the launch."""
    heads, lq, lk = 2, 256, 4 * 128 - 40
    nk = 4
    gen = torch.Generator().manual_seed(23)
    q = torch.randn((lq, heads * 128), generator=gen)
    k = torch.randn((lk, heads * 128), generator=gen)
    v = torch.randn((lk, heads * 128), generator=gen)
    q[:, :128] = 4.0 + 0.25 * torch.randn((lq, 128), generator=gen)     # head 0: q.k ~ -1536 +- 14
    k[:, :128] = -3.0 + 0.25 * torch.randn((lk, 128), generator=gen)
    q, k, v = (t.to(dtype) for t in (q, k, v))
    lists = {(0, 0): [nk + 5, 0, 3], (0, 1): [-3, 1, 2, 3], (1, 0): [0, 1], (1, 1): [3, 2]}
    kidx = np.zeros((heads, 2, nk), dtype=np.int32)
    kcnt = np.zeros((heads, 2), dtype=np.int32)
    mask = np.zeros((heads, 2, nk), dtype=np.float32)
    for (h, i), l in lists.items():
        kidx[h, i, :len(l)] = l
        kcnt[h, i] = len(l)
        for j in l:
            if 0 <= j < nk:
                mask[h, i, j] = 1.0
    o = fvsr_lcsa.block_sparse_attention(q.to(dev), k.to(dev), v.to(dev), torch.from_numpy(kidx).to(dev),
                                         torch.from_numpy(kcnt).to(dev), heads)
    torch.cuda.synchronize()
    ref = O.block_masked_attention(_np(q), _np(k), _np(v), mask, heads)
    assert np.abs(ref[:, :128]).max() > 0.1                      # head 0 is a real softmax, not zeros
    rel = _rel(o, ref)
    # fp32 (its own kernel, no redo needed): head 0's scores are ~1.5e3 in magnitude, so their fp32 rounding (a few
    # 1e-4 absolute) moves the weights by ~1e-4 relative against the float64 oracle
    assert rel <= (BF16_REL if dtype == torch.bfloat16 else 1e-4), rel


def test_c1_fp32_parity(dev):
    """512x512 fp32 workload: Lq 2048, Lk 6144, 12 heads, the oracle's own mask; rel <= 1e-5."""
    wl = synth.WORKLOADS["lcsa_512x512_fp32"]
    q, k, v = synth.make_qkv(wl, seed=0)
    local = synth.local_mask(wl).numpy()
    topk = synth.workload_topk(wl)
    mask, _ = O.draft_block_mask_and_probs(q.numpy(), k.numpy(), wl.heads, wl.q_slices, wl.s, local, topk)
    ref = O.block_masked_attention(q.numpy(), k.numpy(), v.numpy(), mask, wl.heads)
    md = torch.from_numpy(mask).to(dev)
    o = fvsr_lcsa.kernel_block_attention(q.to(dev), k.to(dev), v.to(dev), md, wl.heads)
    od = fvsr_lcsa.block_masked_attention(q.to(dev), k.to(dev), v.to(dev), md, wl.heads)
    assert _rel(o, ref) <= FP32_REL
    assert torch.equal(o, od)


def _torch_fp32_attention(q, k, v, heads, hsel):
    """Plain torch fp32 attention for the heads in `hsel` (full mask), one head at a time on the device."""
    d = 128
    outs = []
    for h in hsel:
        qh = q[:, h * d:(h + 1) * d].float()
        kh = k[:, h * d:(h + 1) * d].float()
        vh = v[:, h * d:(h + 1) * d].float()
        s = (qh @ kh.t().contiguous()) / d ** 0.5
        outs.append(torch.softmax(s, dim=-1) @ vh)
    return torch.cat(outs, dim=1)


def test_c2_full_mask_sparse_equals_dense_bf16(dev):
    """1280x768 bf16, every block kept: kernel == dense fallback exactly, and both within 1e-2 of torch fp32."""
    wl = synth.WORKLOADS["dense_1280x768_bf16"]
    q, k, v = synth.make_qkv(wl, seed=0, device=dev)
    m = torch.ones((wl.heads, wl.nq, wl.nk), device=dev)
    o = fvsr_lcsa.kernel_block_attention(q, k, v, m, wl.heads)
    od = fvsr_lcsa.block_masked_attention(q, k, v, m, wl.heads)
    assert torch.equal(o, od)
    hsel = [0, 7]
    ref = _torch_fp32_attention(q, k, v, wl.heads, hsel)
    got = torch.cat([o[:, h * 128:(h + 1) * 128] for h in hsel], dim=1)
    rel = ((got.float() - ref).abs().max() / ref.abs().max()).item()
    assert rel <= BF16_REL


def _rows_vs_oracle(q, k, v, mask_np, heads, o, pairs):
    """Worst rel of the GPU output against the float64 oracle over the listed (head, query block) rows."""
    qn, kn, vn = q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy()
    got = _np(o)
    worst = 0.0
    for h, b in pairs:
        ref = O.block_masked_attention(qn, kn, vn, mask_np, heads, heads_subset=[h], qblocks_subset=[b])
        r = slice(b * 128, min((b + 1) * 128, got.shape[0]))
        c = slice(h * 128, (h + 1) * 128)
        worst = max(worst, O.compare(got[r, c], ref[r, c])["rel"])
    return worst


def test_c2_full_mask_every_head_vs_oracle(dev):
    """1280x768 bf16, every block kept (DiT.swift:279-313 with a full mask): three query blocks of EVERY head (the
    first, a middle and the last of the 60) against the float64 oracle at rel <= 1e-2, for the sparse kernel and
    for the dense fallback; the two are equal bit for bit."""
    wl = synth.WORKLOADS["dense_1280x768_bf16"]
    q, k, v = synth.make_qkv(wl, seed=0, device=dev)
    m = torch.ones((wl.heads, wl.nq, wl.nk), device=dev)
    o = fvsr_lcsa.kernel_block_attention(q, k, v, m, wl.heads)
    od = fvsr_lcsa.block_masked_attention(q, k, v, m, wl.heads)
    assert torch.equal(o, od)
    mask_np = np.ones((wl.heads, wl.nq, wl.nk), dtype=np.float32)
    pairs = [(h, b) for h in range(wl.heads) for b in (0, (7 * h + 23) % wl.nq, wl.nq - 1)]
    rel = _rows_vs_oracle(q, k, v, mask_np, wl.heads, o, pairs)
    assert rel <= BF16_REL, rel


def test_c4_bf16_subset_vs_oracle(dev):
    """1920x1152 bf16 (Lq 17280, Lk 43200 with a ragged last key block), the oracle's block mask (equal to the
    GPU selection's, which test_gpu_select checks bit for bit): three query blocks of every head against the float64
    oracle at rel <= 1e-2 (each row non-empty, lists of different lengths), kernel == dense fallback everywhere."""
    wl = synth.WORKLOADS["sparse_1920x1152_bf16"]
    q, k, v = synth.make_qkv(wl)
    local = synth.local_mask(wl).numpy()
    topk = synth.workload_topk(wl)
    mask_np, _ = O.draft_block_mask_and_probs(q.float().numpy(), k.float().numpy(), wl.heads, wl.q_slices, wl.s,
                                              local, topk, lk=wl.lk)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    md = torch.from_numpy(mask_np).to(dev)
    o = fvsr_lcsa.kernel_block_attention(qd, kd, vd, md, wl.heads)
    od = fvsr_lcsa.block_masked_attention(qd, kd, vd, md, wl.heads)
    assert torch.equal(o, od)
    assert torch.isfinite(o.float()).all()
    # per head: the query blocks with the shortest and the longest list, and one in the middle of the grid
    kc = mask_np.sum(-1)
    pairs = []
    for h in range(wl.heads):
        for b in {int(kc[h].argmin()), int(kc[h].argmax()), (11 * h + 67) % wl.nq}:
            assert kc[h, b] > 0
            pairs.append((h, b))
    assert _rows_vs_oracle(q, k, v, mask_np, wl.heads, o, pairs) <= BF16_REL


def test_c3_bf16_attention_vs_oracle(dev):
    """1280x768 bf16 block-sparse (local range 3, 60% of in-window pairs; tie-free smooth Q/K at the workload's
    seed), the oracle's own mask: two query blocks of every head against the float64 oracle at rel <= 1e-2
    (DiT.swift:279-313), kernel == dense fallback everywhere."""
    wl = synth.WORKLOADS["sparse_1280x768_bf16"]
    q, k, v = synth.make_qkv(wl)
    local = synth.local_mask(wl).numpy()
    topk = synth.workload_topk(wl)
    mask_np, probs = O.draft_block_mask_and_probs(q.float().numpy(), k.float().numpy(), wl.heads, wl.q_slices, wl.s,
                                                  local, topk)
    assert O.threshold_margin(probs, wl.q_slices, topk) >= 1e-3
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    md = torch.from_numpy(mask_np).to(dev)
    o = fvsr_lcsa.kernel_block_attention(qd, kd, vd, md, wl.heads)
    od = fvsr_lcsa.block_masked_attention(qd, kd, vd, md, wl.heads)
    assert torch.equal(o, od)
    pairs = [(h, b) for h in range(wl.heads) for b in ((7 * h) % wl.nq, (7 * h + 31) % wl.nq)]
    assert _rows_vs_oracle(q, k, v, mask_np, wl.heads, o, pairs) <= BF16_REL


def test_c4_iid_workload_subset(dev):
    """The i.i.d. 1920x1152 workload (960 of 1620 rows select nothing): empty rows are zeros, non-empty rows match
    the oracle, kernel == dense fallback."""
    wl = synth.WORKLOADS["sparse_1920x1152_bf16_iid"]
    q, k, v = synth.make_qkv(wl)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    local = synth.local_mask(wl).numpy()
    mask, _, _, kcnt = fvsr_lcsa.draft_block_mask_and_probs(qd, kd, wl.heads, wl.q_slices, wl.s, local,
                                                            synth.workload_topk(wl), want_probs=False)
    o = fvsr_lcsa.kernel_block_attention(qd, kd, vd, mask, wl.heads)
    od = fvsr_lcsa.block_masked_attention(qd, kd, vd, mask, wl.heads)
    assert torch.equal(o, od)
    kc = kcnt.cpu().numpy()
    ov = o.float().cpu().view(wl.nq, 128, wl.heads, 128)
    empty = np.argwhere(kc == 0)
    assert len(empty) > 0
    for h, b in empty[:: max(1, len(empty) // 16)]:
        assert (ov[b, :, h] == 0).all()
    full = [tuple(x) for x in np.argwhere(kc > 0)[:: max(1, int((kc > 0).sum()) // 12)]]
    assert _rows_vs_oracle(q, k, v, mask.cpu().numpy(), wl.heads, o, full) <= BF16_REL



@pytest.mark.parametrize("density", [1.0, 0.6])
def test_reference_raise_on_sharp_scores(dev, density):
    """Scores that grow along the walk far past the first tile's max: key block j is scaled by s_j (0.05 .. 8), so a
    row's logits span about 90 in log2 units and the reference is raised several times per row (each raise rescales
    O and l and recomputes the tile). The scores are scaled in fp32 (a bf16-rounded prescaled Q would misplace the
    dominant weights by up to 2^0.2 at these magnitudes). bf16 within its bar of the float64 oracle; the kernel
    equal to the dense fallback (which raises at the same tiles) and to the list entry point, bit for bit."""
    heads, lqb, nkb = 2, 3, 6
    gen = torch.Generator().manual_seed(77)
    scale = torch.tensor([0.05, 0.5, 2.0, 4.0, 6.0, 8.0]).repeat_interleave(128).view(-1, 1)
    q = (3.0 * torch.randn((lqb * 128, heads * 128), generator=gen)).to(torch.bfloat16)
    k = (scale * torch.randn((nkb * 128, heads * 128), generator=gen)).to(torch.bfloat16)
    v = torch.randn((nkb * 128, heads * 128), generator=gen).to(torch.bfloat16)
    m = (torch.rand((heads, lqb, nkb), generator=gen) < density).float()
    m[:, :, 0] = 1.0                          # every row starts on the flat block
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), m.to(dev)
    o = fvsr_lcsa.kernel_block_attention(qd, kd, vd, md, heads)
    od = fvsr_lcsa.block_masked_attention(qd, kd, vd, md, heads)
    kidx, kcnt = O.block_lists(m.numpy())
    ol = fvsr_lcsa.block_sparse_attention(qd, kd, vd, torch.from_numpy(kidx).to(dev), torch.from_numpy(kcnt).to(dev),
                                          heads)
    torch.cuda.synchronize()
    assert torch.equal(o, od)
    assert torch.equal(o, ol)
    ref = O.block_masked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), m.numpy(), heads)
    rel = _rel(o, ref)
    print(f"  density {density}: rel {rel:.2e}", flush=True)
    assert rel <= BF16_REL


_QG2_CHILD = r"""
import sys, numpy as np, torch
sys.path[:0] = sys.argv[3:5]
import fvsr_lcsa
z = np.load(sys.argv[1])
dev = torch.device("cuda:0")
q, k, v = (torch.from_numpy(z[n]).to(dev).to(torch.bfloat16) for n in ("q", "k", "v"))
m = torch.from_numpy(z["mask"]).to(dev)
heads = int(z["heads"])
o = fvsr_lcsa.kernel_block_attention(q, k, v, m, heads)
od = fvsr_lcsa.block_masked_attention(q, k, v, m, heads)
torch.cuda.synchronize()
np.savez(sys.argv[2], o=o.float().cpu().numpy(), od=od.float().cpu().numpy())
"""


def test_64_query_waves_equal_32_query_waves(dev, tmp_path):
    """The bf16 walk's 64-queries-per-wave lane (FVSR_ATTN_QG=2, one wave per SIMD; read once per process, so it runs
    in a child) does the same arithmetic per 32-query group as the default lane: kernel and dense walk bit-identical
    to the default's, on ragged rows with an empty one and listed blocks of every length."""
    import subprocess
    import sys
    heads, lqb, nkb = 4, 20, 60
    gen = torch.Generator().manual_seed(2024)
    q = torch.randn((lqb * 128 - 37, heads * 128), generator=gen).to(torch.bfloat16)
    k = torch.randn((nkb * 128 - 90, heads * 128), generator=gen).to(torch.bfloat16)
    v = torch.randn((nkb * 128 - 90, heads * 128), generator=gen).to(torch.bfloat16)
    m = (torch.rand((heads, lqb, nkb), generator=gen) < torch.linspace(0.05, 0.9, lqb).view(1, lqb, 1)).float()
    m[1, 3] = 0.0                              # an empty row
    inp = tmp_path / "in.npz"
    out = tmp_path / "out.npz"
    np.savez(inp, q=q.float().numpy(), k=k.float().numpy(), v=v.float().numpy(), mask=m.numpy(), heads=heads)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, FVSR_ATTN_QG="2")
    r = subprocess.run([sys.executable, "-c", _QG2_CHILD, str(inp), str(out), os.path.join(root, "mlx-flashvsr-swift_amd"),
                        root], env=env, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    qd, kd, vd, md = q.to(dev), k.to(dev), v.to(dev), m.to(dev)
    o = fvsr_lcsa.kernel_block_attention(qd, kd, vd, md, heads)
    od = fvsr_lcsa.block_masked_attention(qd, kd, vd, md, heads)
    torch.cuda.synchronize()
    z = np.load(out)
    assert np.array_equal(z["o"], _np(o))
    assert np.array_equal(z["od"], _np(od))
    assert torch.equal(o, od)


def _rows_vs_torch(q, k, v, m, heads, o, pairs):
    """Worst rel of the GPU output against a float32 torch softmax over the listed key blocks of a few rows."""
    worst = 0.0
    for h, i in pairs:
        blocks = m[h, i].nonzero().flatten().tolist()
        got = o[i * 128:(i + 1) * 128, h * 128:(h + 1) * 128].float()
        if not blocks:
            assert (got == 0).all()
            continue
        qs = q[i * 128:(i + 1) * 128, h * 128:(h + 1) * 128].float()
        rows = torch.cat([torch.arange(j * 128, min((j + 1) * 128, k.shape[0]), device=k.device) for j in blocks])
        ks, vs = k[rows, h * 128:(h + 1) * 128].float(), v[rows, h * 128:(h + 1) * 128].float()
        ref = torch.softmax(qs @ ks.t() / 128 ** 0.5, dim=-1) @ vs
        worst = max(worst, float((got - ref).abs().max() / ref.abs().max()))
    return worst


@pytest.mark.parametrize("heads,lqb,uniform", [(2, 4200, False), (2, 4200, True), (1, 140000, False),
                                               (1, 140000, True)])
def test_row_counts_beyond_the_order_kernels_lds(dev, heads, lqb, uniform):
    """More rows than the row-order kernel keeps in LDS (8192: the sorted order is staged in the workspace) and, at
    140,000 rows, more than its row-id bitmap covers (131,072: each wave is ranked by scanning its rows). Lists of
    mixed lengths (0 .. 4 blocks) and of one length (2 blocks each: the order is dealt without the sort). Outputs
    start as NaN, so a row the walk skipped fails; kernel == dense fallback everywhere, empty rows are zeros, and a
    few rows match a float32 torch softmax."""
    lk = 3 * 128 + 50
    g = torch.Generator(device=dev).manual_seed(lqb + int(uniform))
    q = torch.randn((lqb * 128, heads * 128), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((lk, heads * 128), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((lk, heads * 128), generator=g, device=dev).to(torch.bfloat16)
    if uniform:
        m = torch.zeros((heads, lqb, 4), device=dev)
        m[..., 1] = 1.0
        m[..., 3] = 1.0
    else:
        dens = torch.rand((heads, lqb, 1), generator=g, device=dev)
        m = (torch.rand((heads, lqb, 4), generator=g, device=dev) < dens).float()
    o = torch.full((lqb * 128, heads * 128), float("nan"), dtype=torch.bfloat16, device=dev)
    od = torch.full_like(o, float("nan"))
    print(f"  rows {heads * lqb}, kept blocks {int(m.sum())}", flush=True)
    fvsr_lcsa.kernel_block_attention(q, k, v, m, heads, out=o)
    fvsr_lcsa.block_masked_attention(q, k, v, m, heads, out=od)
    torch.cuda.synchronize()
    assert not torch.isnan(o).any()
    assert torch.equal(o, od)
    empty = (m.sum(-1) == 0).nonzero().tolist()
    ov = o.view(lqb, 128, heads, 128)
    for h, i in empty[:64]:
        assert (ov[i, :, h] == 0).all()
    pairs = [(h, i) for h in range(heads) for i in (0, 1, lqb // 2, lqb - 2, lqb - 1)]
    assert _rows_vs_torch(q, k, v, m, heads, o, pairs) <= BF16_REL
