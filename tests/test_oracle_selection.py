"""Independent pins of the oracle's block selection (oracle/lcsa.py: pool_blocks, block_scores,
draft_block_mask_and_probs), none of which reads the golden fixture or retypes the oracle's array formula.

The selection is `draftBlockMaskAndProbs` (Sources/FlashVSRMLX/DiT.swift:158-174):
  - pq, pk: fp32 mean of each 128-token window, per head, where head h owns channels h*d .. h*d + d - 1
    (`mean(axis: 1).reshaped([n, heads, d])`, :161-162); a ragged last window averages its valid tokens only
    (the slicing of oracle/block_sparse_attn.py:34 carried over to the pooling);
  - scores = pq . pk / sqrt(d), a true divide (:163), plus the local window (0 / -inf) tiled over every
    (query slice, key slice) pair (:165-167);
  - softmax over the key blocks (:168);
  - per (head, query temporal slice) row, keep the pairs strictly above the (k+1)-th largest, k = min(n - 1, topk)
    (:169-173).

Pins, each chosen so that a plausible slip fails one of them:
  - a float64 scalar-loop restatement over explicit index ranges (heads carrying different data, two query slices,
    a ragged last key block) against which the oracle's probabilities and mask are compared;
  - closed forms: a ragged block of constant value c pools to c; channel blocks of distinct constants stay with
    their head; block-constant q/k give analytic softmax probabilities;
  - IEEE correct rounding: each score is the correctly rounded fp32 quotient of an exact dot product by fp32(sqrt d),
    computed here with exact rational arithmetic (a multiply by a rounded reciprocal differs in the last place for
    some dots, and those dots are in the test).
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import lcsa as O

D = 128


# --- float64 scalar-loop restatement -----------------------------------------------------------------------------
def pooled_bruteforce(x, heads, n_tokens):
    """Per head h and block b: the float64 mean of channels h*D .. h*D+D-1 over the block's valid tokens."""
    nb = -(-n_tokens // 128)
    out = np.zeros((heads, nb, D))
    for h in range(heads):
        for b in range(nb):
            t0, t1 = 128 * b, min(n_tokens, 128 * (b + 1))
            for ch in range(D):
                out[h, b, ch] = math.fsum(float(x[t, h * D + ch]) for t in range(t0, t1)) / (t1 - t0)
    return out


def selection_bruteforce(q, k, heads, q_slices, s, local, topk, lq, lk):
    """(mask, probs, margin) of the selection by loops over (head, query block, key block)."""
    pq = pooled_bruteforce(q, heads, lq)
    pk = pooled_bruteforce(k, heads, lk)
    nq, nk = pq.shape[1], pk.shape[1]
    probs = np.zeros((heads, nq, nk))
    for h in range(heads):
        for i in range(nq):
            logits = []
            for j in range(nk):
                if local[i % s][j % s]:
                    dot = math.fsum(pq[h, i, c] * pk[h, j, c] for c in range(D))
                    logits.append(dot / math.sqrt(D))
                else:
                    logits.append(-math.inf)
            m = max(logits)
            e = [math.exp(x - m) if x != -math.inf else 0.0 for x in logits]
            z = math.fsum(e)
            for j in range(nk):
                probs[h, i, j] = e[j] / z
    per_slice = nq // q_slices
    mask = np.zeros((heads, nq, nk))
    margin = math.inf
    for h in range(heads):
        for sl in range(q_slices):
            entries = [(probs[h, i, j], i, j) for i in range(sl * per_slice, (sl + 1) * per_slice)
                       for j in range(nk)]
            vals = sorted((p for p, _, _ in entries), reverse=True)
            kk = min(len(vals) - 1, topk)
            thr = vals[kk]                                  # the (k+1)-th largest
            if kk > 0:
                margin = min(margin, (vals[kk - 1] - thr) / vals[kk - 1])
            for p, i, j in entries:
                mask[h, i, j] = 1.0 if p > thr else 0.0
    return mask, probs, margin


def _structured_case(seed, heads=3, bh=2, bw=3, q_slices=2, k_blocks=13, ragged=40, sigma=0.7):
    """Heads with their own block-level signal plus token noise; the last key block holds `ragged` tokens."""
    rng = np.random.default_rng(seed)
    s = bh * bw
    nq = q_slices * s
    lq, lk = nq * 128, (k_blocks - 1) * 128 + ragged
    c = heads * D
    mq = sigma * rng.standard_normal((nq, 1, c))
    mk = sigma * rng.standard_normal((k_blocks, 1, c))
    q = (np.repeat(mq, 128, axis=1).reshape(nq * 128, c) + 0.5 * rng.standard_normal((nq * 128, c)))[:lq]
    k = (np.repeat(mk, 128, axis=1).reshape(k_blocks * 128, c) + 0.5 * rng.standard_normal((k_blocks * 128, c)))[:lk]
    local = O.local_block_mask(bh, bw, 3)
    return q.astype(np.float32), k.astype(np.float32), local, s, lq, lk


@pytest.fixture(scope="module")
def structured():
    q, k, local, s, lq, lk = _structured_case(seed=11)
    heads, q_slices, topk = 3, 2, 20
    bm, bp, margin = selection_bruteforce(q, k, heads, q_slices, s, local, topk, lq, lk)
    return q, k, local, s, lq, lk, heads, q_slices, topk, bm, bp, margin


def test_case_exercises_heads_slices_and_ragged_tail(structured):
    q, k, local, s, lq, lk, heads, q_slices, topk, bm, bp, margin = structured
    assert heads >= 3 and q_slices == 2 and lk % 128 != 0
    nk = bp.shape[2]
    # the ragged key block is in the window of some rows and kept by some of them, in every head
    assert (bp[:, :, nk - 1] > 0).any(axis=1).all()
    assert (bm[:, :, nk - 1] > 0).any(axis=1).all()
    # the heads select differently (a head-mixing slip changes every head's probabilities)
    assert not np.array_equal(bm[0], bm[1]) and not np.array_equal(bm[1], bm[2])
    assert margin > 1e-3          # no near-ties: any fp32 implementation must give this mask


def test_oracle_probs_match_scalar_loops(structured):
    q, k, local, s, lq, lk, heads, q_slices, topk, bm, bp, margin = structured
    _, probs = O.draft_block_mask_and_probs(q, k, heads, q_slices, s, local, topk, lq=lq, lk=lk)
    # fp32 pooling, products and softmax against float64: a few fp32 ulps of the row's probabilities
    np.testing.assert_allclose(probs, bp, rtol=2e-5, atol=1e-7)


def test_oracle_mask_matches_scalar_loops(structured):
    q, k, local, s, lq, lk, heads, q_slices, topk, bm, bp, margin = structured
    mask, _ = O.draft_block_mask_and_probs(q, k, heads, q_slices, s, local, topk, lq=lq, lk=lk)
    np.testing.assert_array_equal(mask, bm)
    per_row = mask.reshape(heads * q_slices, -1).sum(1)
    assert (per_row == topk).all()


def test_oracle_margin_matches_scalar_loops(structured):
    q, k, local, s, lq, lk, heads, q_slices, topk, bm, bp, margin = structured
    assert O.threshold_margin(bp, q_slices, topk) == pytest.approx(margin, rel=1e-9)
    # top-k 0 keeps nothing: no kept neighbour above the threshold, so no tie is possible
    assert O.threshold_margin(bp, q_slices, 0) == math.inf
    assert selection_bruteforce(q, k, heads, q_slices, s, local, 0, lq, lk)[2] == math.inf


def test_oracle_pooling_matches_scalar_loops(structured):
    q, k, local, s, lq, lk, heads, *_ = structured
    np.testing.assert_allclose(O.pool_blocks(k, heads, lk), pooled_bruteforce(k, heads, lk), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(O.pool_blocks(q, heads, lq), pooled_bruteforce(q, heads, lq), rtol=1e-5, atol=1e-6)


# --- closed forms ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n_valid", [1, 40, 64, 127])
def test_ragged_block_of_constant_pools_to_that_constant(n_valid):
    heads = 2
    c = np.float32(0.375)
    x = np.zeros((128 + n_valid, heads * D), dtype=np.float32)
    x[:128] = np.float32(-1.5)
    x[128:] = c
    p = O.pool_blocks(x, heads, 128 + n_valid)
    assert p.shape == (heads, 2, D)
    assert (p[:, 0] == np.float32(-1.5)).all()
    assert (p[:, 1] == c).all()       # the mean over the valid tokens, not the sum over 128


def test_pooled_channels_stay_with_their_head():
    heads = 4
    x = np.empty((256, heads * D), dtype=np.float32)
    for h in range(heads):
        x[:, h * D:(h + 1) * D] = np.float32(h + 1) + np.arange(D, dtype=np.float32) / 256
    p = O.pool_blocks(x, heads)
    for h in range(heads):
        want = np.float32(h + 1) + np.arange(D, dtype=np.float32) / 256
        np.testing.assert_array_equal(p[h, 0], want)
        np.testing.assert_array_equal(p[h, 1], want)


def test_block_constant_inputs_give_analytic_probabilities():
    """Every token of q block i, head h equals a[h, i] in each channel, every token of key block j b[h, j]; then
    pq . pk = D a b exactly and the probabilities are softmax_j(sqrt(D) a b) over the visible key blocks."""
    heads, bh, bw = 3, 2, 2
    s = bh * bw
    nq, nk = s, 2 * s
    a = np.array([[0.5, -1.0, 0.25, 1.0], [1.5, 0.0, -0.5, 0.75], [-0.25, 2.0, 1.0, -1.0]], dtype=np.float32)
    b = np.array([[(j % 5) * 0.25 - 0.5 + 0.125 * h for j in range(nk)] for h in range(heads)], dtype=np.float32)
    q = np.empty((nq * 128, heads * D), dtype=np.float32)
    k = np.empty((nk * 128, heads * D), dtype=np.float32)
    for h in range(heads):
        for i in range(nq):
            q[128 * i:128 * (i + 1), h * D:(h + 1) * D] = a[h, i]
        for j in range(nk):
            k[128 * j:128 * (j + 1), h * D:(h + 1) * D] = b[h, j]
    local = O.local_block_mask(bh, bw, 1)       # each query block sees its own spatial position only
    _, probs = O.draft_block_mask_and_probs(q, k, heads, 1, s, local, topk=3)
    for h in range(heads):
        for i in range(nq):
            vis = [j for j in range(nk) if j % s == i]
            logit = {j: math.sqrt(D) * float(a[h, i]) * float(b[h, j]) for j in vis}
            m = max(logit.values())
            z = math.fsum(math.exp(x - m) for x in logit.values())
            for j in range(nk):
                want = math.exp(logit[j] - m) / z if j in logit else 0.0
                assert probs[h, i, j] == pytest.approx(want, rel=1e-6, abs=1e-12), (h, i, j)


# --- the divide, by exact rational arithmetic ---------------------------------------------------------------------
def round_to_f32(x: Fraction) -> float:
    """The IEEE binary32 value nearest to the rational x (ties to even); normal range only."""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    x = abs(x)
    e = math.floor(math.log2(x.numerator) - math.log2(x.denominator))
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    scaled = x / Fraction(2) ** (e - 23)          # in [2^23, 2^24)
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(Fraction(n) * Fraction(2) ** (e - 23))


def test_scores_are_correctly_rounded_quotients():
    """score = fl(dot / fl(sqrt(128))): the correctly rounded quotient (IEEE division), computed here exactly. The
    dots are integers (exact in fp32); the set includes dots where a multiply by fl(1 / fl(sqrt(128))) rounds to the
    neighbouring value, so a reciprocal multiply fails this test."""
    sq = Fraction(float(np.float32(math.sqrt(D))))
    inv = np.float32(1.0) / np.float32(math.sqrt(D))
    dots = list(range(1, 400))
    quot = [round_to_f32(Fraction(d) / sq) for d in dots]
    differs = [d for d, qv in zip(dots, quot) if float(np.float32(d) * inv) != qv]
    assert len(differs) >= 5          # the two roundings really do differ on this set
    heads, n = 1, len(dots)
    pq = np.zeros((heads, n, D), dtype=np.float32)
    pk = np.zeros((heads, 1, D), dtype=np.float32)
    pq[0, :, 0] = np.array(dots, dtype=np.float32)
    pk[0, 0, 0] = 1.0
    local = np.ones((1, 1), dtype=bool)
    sc = O.block_scores(pq, pk, local, 1)
    np.testing.assert_array_equal(sc[0, :, 0], np.array(quot, dtype=np.float32))


def test_round_to_f32_agrees_with_numpy_on_doubles():
    rng = np.random.default_rng(5)
    for x in rng.standard_normal(200) * 1e3:
        assert round_to_f32(Fraction(float(x))) == float(np.float32(x))
