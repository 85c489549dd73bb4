"""A seeded sweep of the whole select -> attend path over random small geometries, through the C ABI, against the
oracle.

Each case draws the head count, the spatial block grid (bh, bw), the query and key slice counts, ragged query and
key tails, the local range, the top-k (mostly a random share of the in-window pairs; also 1, past the row, and 0)
and the dtype. Q and K are a per-block random offset plus token noise, so the pooled means of a block differ and
most rows have a clear threshold; V is noise.

Bars, as in test_gpu_select.py and test_gpu_attention.py: probs rel <= 1e-5; the mask bit-exact where the (head,
query slice) threshold margin exceeds 1e-4, else flips only at the reference's legitimate near-ties
(Gates.swift:239-277); kcnt / kidx are the mask's lists (SparseAttention.swift:175-177); the attention over the
GPU's lists against the float64 oracle on the GPU's mask: fp32 rel <= 1e-5, bf16 rel <= 1e-2; the block-sparse
kernel and the dense fallback agree bit for bit.
"""
import numpy as np
import pytest
import torch

import fvsr_lcsa
from oracle import lcsa as O

pytestmark = pytest.mark.gpu
TIE_FREE = 1e-4
FP32_REL = 1e-5
BF16_REL = 1e-2
D = 128


def _case(seed):
    r = np.random.default_rng(1000 + seed)
    heads = int(r.choice([1, 2, 3, 4, 6]))
    bh, bw = int(r.integers(1, 5)), int(r.integers(1, 5))
    s = bh * bw
    q_slices, k_slices = int(r.integers(1, 4)), int(r.integers(1, 5))
    nq, nk = q_slices * s, k_slices * s
    lq = nq * 128 - int(r.integers(0, 128))
    lk = nk * 128 - int(r.integers(0, 128))
    local_range = int(r.choice([1, 2, 3, 5, 11]))
    row = s * nk                                    # elements of one (head, query slice) row
    in_window = O.in_window_pairs(O.local_block_mask(bh, bw, local_range), s, nk)
    kind = seed % 6                                 # mostly a share of the in-window pairs; 1, past the row, 0
    share = max(2, int(r.uniform(0.1, 0.9) * in_window))
    topk = [share, 1, share, row + int(r.integers(0, 5)), share, 0][kind]
    dtype = torch.bfloat16 if seed % 2 else torch.float32
    return dict(heads=heads, bh=bh, bw=bw, s=s, q_slices=q_slices, nq=nq, nk=nk, lq=lq, lk=lk,
                local_range=local_range, topk=topk, dtype=dtype, rng=r)


def _tokens(r, n_blocks, n_tokens, c, scale):
    bias = r.standard_normal((n_blocks, c)).astype(np.float32) * scale
    x = np.repeat(bias, 128, axis=0)[:n_tokens] + r.standard_normal((n_tokens, c)).astype(np.float32) * 0.5
    return x


@pytest.mark.parametrize("seed", range(24))
def test_select_then_attend_random_geometry(dev, seed):
    cs = _case(seed)
    r, heads, dtype = cs["rng"], cs["heads"], cs["dtype"]
    c = heads * D
    q = _tokens(r, cs["nq"], cs["lq"], c, 1.0)
    k = _tokens(r, cs["nk"], cs["lk"], c, 1.0)
    v = r.standard_normal((cs["lk"], c)).astype(np.float32)
    if dtype == torch.bfloat16:   # the oracle sees exactly the values the GPU reads
        q, k, v = O.to_bf16(q), O.to_bf16(k), O.to_bf16(v)
    local = O.local_block_mask(cs["bh"], cs["bw"], cs["local_range"])
    ref_mask, ref_probs = O.draft_block_mask_and_probs(q, k, heads, cs["q_slices"], cs["s"], local, cs["topk"],
                                                       lq=cs["lq"], lk=cs["lk"])
    qd, kd, vd = (torch.from_numpy(x).to(dev).to(dtype) for x in (q, k, v))
    mask, probs, kidx, kcnt = fvsr_lcsa.draft_block_mask_and_probs(qd, kd, heads, cs["q_slices"], cs["s"], local,
                                                                   cs["topk"])
    torch.cuda.synchronize()
    info = {k_: v_ for k_, v_ in cs.items() if k_ != "rng"}
    assert O.compare(probs.cpu().numpy(), ref_probs)["rel"] <= 1e-5, info
    got_mask = mask.cpu().numpy()
    margin = O.threshold_margin(ref_probs, cs["q_slices"], cs["topk"])
    if margin > TIE_FREE:
        np.testing.assert_array_equal(got_mask, ref_mask, err_msg=str(info))
    else:
        rep = O.mask_flip_report(got_mask, ref_mask, ref_probs, cs["q_slices"])
        assert rep["legit"], (rep, info)
    sel = got_mask > 0.5
    np.testing.assert_array_equal(kcnt.cpu().numpy(), sel.sum(-1))
    want_kidx, _ = O.block_lists(got_mask)
    np.testing.assert_array_equal(kidx.cpu().numpy(), want_kidx)

    o = fvsr_lcsa.block_sparse_attention(qd, kd, vd, kidx, kcnt, heads)
    od = fvsr_lcsa.block_masked_attention(qd, kd, vd, mask, heads)
    torch.cuda.synchronize()
    assert torch.equal(o, od), info
    ref = O.block_masked_attention(q, k, v, got_mask, heads)
    rel = O.compare(o.float().cpu().numpy(), ref)["rel"]
    assert rel <= (BF16_REL if dtype == torch.bfloat16 else FP32_REL), (rel, info)
