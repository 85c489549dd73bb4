"""CPU checks that pin the oracle (oracle/lcsa.py) before the GPU results are compared against it.

Sources of truth, none of which is the oracle's own formula retyped:
  - the reference's structure KATs (Tests/FlashVSRMLXTests/FlashVSRStructureTests.swift:34-75), ported verbatim;
  - the mask densities logged by the reference's parity gate (oracle/reports/s1_sparse_gpu_kernel.log:18,49):
    top-k 114 = Int(144*0.8)-1 keeps exactly 114 of 432 (chunk 0) and of 576 (chunk 1) block pairs per row;
  - the survey's in-window fractions of the reference geometries;
  - float64 brute force over every (head, query, key) on tiny shapes; closed forms (constant keys, full mask,
    empty rows, list order); the golden fixture in tests/golden/.
"""
import math
import os

import numpy as np
import pytest

from oracle import lcsa as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "lcsa_tiny.npz")


# --- window layout (FlashVSRStructureTests.swift:34-44) ---------------------------------------------------------
def test_window_partition_round_trip_and_order():
    f, h, w, c = 4, 16, 24, 3
    x = np.arange(f * h * w * c, dtype=np.float32).reshape(1, f, h, w, c)
    p = O.window_partition(x, f, h, w)
    assert p.shape == ((f // 2) * (h // 8) * (w // 8), 128, c)
    win = (1 * (h // 8) + 1) * (w // 8) + 2
    tok = (1 * 8 + 3) * 8 + 5
    np.testing.assert_array_equal(p[win, tok], x[0, 3, 11, 21])
    r = O.window_reverse(p, 1, f, h, w)
    np.testing.assert_array_equal(r.reshape(x.shape), x)


# --- local window (FlashVSRStructureTests.swift:46-58) -----------------------------------------------------------
@pytest.mark.parametrize("bh,bw,r", [(3, 4, 11), (6, 10, 3), (5, 5, 4)])
def test_local_block_mask_matches_definition(bh, bw, r):
    m = O.local_block_mask(bh, bw, r)
    for q in range(bh * bw):
        for k in range(bh * bw):
            qr, qc, kr, kc = q // bw, q % bw, k // bw, k % bw
            lo = lambda v: v - r // 2  # noqa: E731
            want = lo(qr) <= kr <= lo(qr) + r - 1 and lo(qc) <= kc <= lo(qc) + r - 1
            assert m[q, k] == want


def test_local_block_mask_range_covers_grid_is_dense():
    assert O.local_block_mask(3, 4, 11).all()


@pytest.mark.parametrize("bh,bw,r,frac", [(4, 4, 3, 0.391), (6, 10, 3, 0.124), (9, 15, 3, 0.059),
                                          (4, 4, 11, 1.0), (6, 10, 11, 0.80), (9, 15, 11, 0.511)])
def test_in_window_fraction_of_reference_geometries(bh, bw, r, frac):
    s = bh * bw
    assert O.local_block_mask(bh, bw, r).sum() / (s * s) == pytest.approx(frac, abs=6e-4)


# --- draft mask KAT (FlashVSRStructureTests.swift:60-75) ----------------------------------------------------------
def test_draft_mask_keeps_strictly_above_threshold():
    s = 2
    q = np.ones((2, 128, 128), dtype=np.float32)
    k = np.zeros((2, 128, 128), dtype=np.float32)
    k[0] = 2.0
    local = np.ones((2, 2), dtype=bool)
    m, _ = O.draft_block_mask_and_probs(q, k, 1, 1, s, local, topk=1)
    assert m.sum() == 0                       # threshold = 2nd largest = p0 -> nothing strictly above
    m0, _ = O.draft_block_mask_and_probs(q, k, 1, 1, s, local, topk=2)
    np.testing.assert_array_equal(m0.reshape(-1), [1, 0, 1, 0])


def test_topk_formula_of_sparse_golden():
    # sparse golden: topk_ratio 0.8 on s = 12 -> Int(144 * 0.8) - 1 = 114 (PORTING-SPEC.md:39; receipt densities)
    assert O.step_topk(12, 0.8) == 114
    assert O.step_topk(135, O.default_topk_ratio(1152, 1920)) == 16199


@pytest.mark.parametrize("k_slices,density", [(3, 0.264), (4, 0.198)])
def test_topk_density_matches_reference_receipt(k_slices, density):
    """At the sparse golden's geometry (s = 12 = 3 x 4 blocks, local range 3, topk 114) every (head, query slice)
    row keeps exactly 114 block pairs: 114/432 = 0.264 (chunk 0), 114/576 = 0.198 (chunk 1), the logged densities."""
    rng = np.random.default_rng(7)
    heads, bh, bw = 12, 3, 4
    s = bh * bw
    q_slices = 3 if k_slices == 3 else 1
    q = rng.standard_normal((q_slices * s * 128, heads * 128)).astype(np.float32)
    k = rng.standard_normal((k_slices * s * 128, heads * 128)).astype(np.float32)
    local = O.local_block_mask(bh, bw, 3)
    m, probs = O.draft_block_mask_and_probs(q, k, heads, q_slices, s, local, 114)
    per_row = m.reshape(heads * q_slices, -1).sum(1)
    assert (per_row == 114).all()
    assert round(float(m.mean()), 3) == density


def test_topk_at_least_row_length_keeps_everything_above_minimum():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((4 * 128, 128)).astype(np.float32)
    k = rng.standard_normal((8 * 128, 128)).astype(np.float32)
    local = O.local_block_mask(2, 2, 3)
    m, p = O.draft_block_mask_and_probs(q, k, 1, 1, 4, local, topk=10_000)
    flat = p.reshape(1, -1)
    np.testing.assert_array_equal(m.reshape(1, -1), (flat > flat.min()).astype(np.float32))


def test_softmax_rows_sum_to_one_and_window_zeroes():
    rng = np.random.default_rng(4)
    q = rng.standard_normal((4 * 128, 256)).astype(np.float32)
    k = rng.standard_normal((8 * 128, 256)).astype(np.float32)
    local = O.local_block_mask(2, 2, 1)          # only the own block is visible
    _, p = O.draft_block_mask_and_probs(q, k, 2, 1, 4, local, 3)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-5)
    vis = np.tile(local, (1, 2))
    assert (p[:, :, ~vis[0]][:, 0] == 0).all()


def test_block_lists_selected_first():
    bm = np.array([[[0, 1, 0, 1], [0, 0, 0, 0], [1, 1, 1, 1]]], dtype=np.float32)
    kidx, kcnt = O.block_lists(bm)
    np.testing.assert_array_equal(kcnt, [[2, 0, 4]])
    np.testing.assert_array_equal(kidx[0, 0], [1, 3, 0, 2])
    np.testing.assert_array_equal(kidx[0, 1], [0, 1, 2, 3])


# --- attention --------------------------------------------------------------------------------------------------
def _tiny_case(seed=0, heads=2, lq=130, lk=200):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((lq, heads * 128)).astype(np.float32)
    k = rng.standard_normal((lk, heads * 128)).astype(np.float32)
    v = rng.standard_normal((lk, heads * 128)).astype(np.float32)
    nq, nk = -(-lq // 128), -(-lk // 128)
    bm = np.zeros((heads, nq, nk), dtype=np.float32)
    bm[0, 0, 1] = 1           # ragged key block only
    bm[0, 1, :] = 1
    bm[1, 0, 0] = 1
    # head 1, query block 1: empty -> zeros
    return q, k, v, bm


def test_attention_matches_float64_bruteforce():
    q, k, v, bm = _tiny_case()
    got = O.block_masked_attention(q, k, v, bm, 2)
    ref = O.attention_bruteforce(q, k, v, bm, 2)
    assert O.compare(got, ref)["rel"] < 1e-12
    assert (got[128:, 128:] == 0).all()


def test_attention_constant_keys_give_mean_of_values():
    rng = np.random.default_rng(1)
    heads, lq, lk = 1, 128, 384
    q = rng.standard_normal((lq, 128)).astype(np.float32)
    k = np.tile(rng.standard_normal((1, 128)).astype(np.float32), (lk, 1))
    v = rng.standard_normal((lk, 128)).astype(np.float32)
    bm = np.array([[[1, 0, 1]]], dtype=np.float32)
    got = O.block_masked_attention(q, k, v, bm, heads)
    want = np.concatenate([v[:128], v[256:]]).astype(np.float64).mean(0)
    np.testing.assert_allclose(got, np.broadcast_to(want, got.shape), rtol=0, atol=1e-12)


def test_attention_full_mask_is_softmax_attention():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((256, 128))
    k = rng.standard_normal((300, 128))
    v = rng.standard_normal((300, 128))
    bm = np.ones((1, 2, 3), dtype=np.float32)
    got = O.block_masked_attention(q, k, v, bm, 1)
    s = q @ k.T / math.sqrt(128)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(got, p @ v, rtol=1e-12, atol=1e-12)


def test_attention_list_order_does_not_matter():
    q, k, v, bm = _tiny_case(seed=5)
    kidx, kcnt = O.block_lists(bm)
    a = O.block_sparse_attention_lists(q, k, v, kidx, kcnt, 2)
    kidx2 = kidx.copy()
    kidx2[0, 1, :2] = kidx2[0, 1, :2][::-1]
    b = O.block_sparse_attention_lists(q, k, v, kidx2, kcnt, 2)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)


# --- KV window cache (DiT.swift:507-511, 532-538) ---------------------------------------------------------------
def test_kv_window_cache_follows_chunk_schedule():
    s = 5
    cache = O.KVWindowCache(kv_len=3)
    seen = []
    tag = 0
    for chunk, seqlen in enumerate([3, 1, 1, 1, 1]):
        kW = np.arange(tag, tag + seqlen * s, dtype=np.float32)[:, None, None] * np.ones((1, 128, 2), np.float32)
        tag += seqlen * s
        kview, _ = cache.attend_view(kW, kW, seqlen)
        seen.append(kview.shape[0] // s)
        cache.trim()
        assert cache.k.shape[0] // s == 3
        # the cache always holds the newest three slices
        np.testing.assert_array_equal(cache.k[:, 0, 0], np.arange(tag - 3 * s, tag))
    assert seen == [3, 4, 4, 4, 4]     # Nk = 3s in chunk 0, 4s after (PORTING-SPEC.md:127-129)


# --- comparison helpers (Gates.swift:19-29, 239-277) --------------------------------------------------------------
def test_compare_rel_metric():
    r = O.compare(np.array([1.0, -2.0]), np.array([1.0, -4.0]))
    assert r["rel"] == 0.5 and r["max_abs"] == 2.0 and r["ref_max"] == 4.0


def test_mask_flip_report_near_tie_rule():
    probs = np.array([[[0.5, 0.25, 0.2500001, 0.0]]], dtype=np.float32)
    golden = np.array([[[1, 1, 0, 0]]], dtype=np.float32)
    mine = np.array([[[1, 0, 1, 0]]], dtype=np.float32)
    rep = O.mask_flip_report(mine, golden, probs, 1)
    assert rep["flips"] == 2 and rep["legit"]
    far = np.array([[[0.5, 0.3, 0.2, 0.0]]], dtype=np.float32)
    rep2 = O.mask_flip_report(mine, golden, far, 1)
    assert not rep2["legit"]


# --- golden fixture ----------------------------------------------------------------------------------------------
def test_golden_fixture_reproduces():
    g = np.load(GOLDEN)
    heads, q_slices, s, topk = (int(x) for x in g["meta"])
    mask, probs = O.draft_block_mask_and_probs(g["q"], g["k"], heads, q_slices, s, g["local"], topk)
    np.testing.assert_array_equal(mask, g["mask"])
    np.testing.assert_allclose(probs, g["probs"], rtol=1e-6, atol=1e-9)
    o = O.block_masked_attention(g["q"], g["k"], g["v"], g["mask"], heads)
    np.testing.assert_allclose(o, g["out"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(o, O.attention_bruteforce(g["q"], g["k"], g["v"], g["mask"], heads), atol=1e-12)
