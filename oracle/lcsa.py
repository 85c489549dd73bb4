"""CPU oracle for FlashVSR's locality-constrained sparse attention (LCSA) hot path.

TEST INFRASTRUCTURE ONLY: the HIP path's results are compared against this module's. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it; the product path never does.

It restates, in numpy, what the reference (xocialize/mlx-flashvsr-swift) computes on the path
`FlashVSRDiT.blockForward` -> window partition -> KV window cache -> draft block mask -> block-sparse attention:

  window_partition / window_reverse   Sources/FlashVSRMLX/DiT.swift:111-126
  local_block_mask                     Sources/FlashVSRMLX/DiT.swift:128-145
  draft_block_mask_and_probs           Sources/FlashVSRMLX/DiT.swift:147-174
  block_lists                          Sources/FlashVSRMLX/SparseAttention.swift:175-177
  block_masked_attention               Sources/FlashVSRMLX/DiT.swift:279-313, oracle/block_sparse_attn.py:20-38
  KVWindowCache                        Sources/FlashVSRMLX/DiT.swift:507-511,532-538; Pipeline.swift:87-91,129
  step_topk / default_topk_ratio       Sources/FlashVSRMLX/DiT.swift:478-485; Pipeline.swift:68
  compare (rel metric)                 Sources/Smoke/Gates.swift:19-29
  mask_flip_report (near-tie rule)     Sources/Smoke/Gates.swift:239-277
  rope_tables                          Sources/FlashVSRMLX/DiT.swift:52-78
  wan_rms_norm                         Sources/FlashVSRMLX/DiT.swift:34-47
  rope_apply                           Sources/FlashVSRMLX/DiT.swift:100-107
  qkv_epilogue                         Sources/FlashVSRMLX/DiT.swift:496-506 (norm -> rope -> window partition)

Ragged extension (not in the reference, which only ever sees whole 128-token windows and whole temporal slices):
a token count that is not a multiple of 128 ends in a partial block. Attention slices the expanded token mask to
`[:lq, :lk]` exactly as `oracle/block_sparse_attn.py:34` does; pooling averages the valid tokens of the partial block
only; a key block j of a key range that is not a whole number of slices takes its local-window row from spatial
position j mod s.

How each function is pinned (tests/test_oracle.py): the reference's own structure KATs
(Tests/FlashVSRMLXTests/FlashVSRStructureTests.swift:34-75), the mask densities logged in
oracle/reports/s1_sparse_gpu_kernel.log:18,49 (top-k of 114 over 432 / 576 pairs), float64 brute-force loops on
tiny shapes, and closed forms (constant keys -> mean of values, full mask -> plain softmax attention, empty query
block -> 0).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

BLOCK = 128          # tokens per LCSA window (win (2, 8, 8)), DiT.swift:111-118
HEAD_DIM = 128       # FlashVSRDiTConfig: dim 1536 / 12 heads, DiT.swift:20-24


# ----------------------------------------------------------------------------------------------------------------
# layout
# ----------------------------------------------------------------------------------------------------------------
def window_partition(x: np.ndarray, f: int, h: int, w: int) -> np.ndarray:
    """(B, F*H*W, C) or (B, F, H, W, C) -> (B*nf*nh*nw, 128, C); windows ordered (nf, nh, nw), tokens (wf, wh, ww).

    DiT.swift:113-118 (`windowPartition`).
    """
    b, c = x.shape[0], x.shape[-1]
    y = x.reshape(b, f // 2, 2, h // 8, 8, w // 8, 8, c).transpose(0, 1, 3, 5, 2, 4, 6, 7)
    return np.ascontiguousarray(y).reshape(b * (f // 2) * (h // 8) * (w // 8), BLOCK, c)


def window_reverse(x: np.ndarray, b: int, f: int, h: int, w: int) -> np.ndarray:
    """Inverse of `window_partition`: (..., C) windows -> (B, F*H*W, C). DiT.swift:121-126 (`windowReverse`)."""
    c = x.shape[-1]
    y = x.reshape(b, f // 2, h // 8, w // 8, 2, 8, 8, c).transpose(0, 1, 4, 2, 5, 3, 6, 7)
    return np.ascontiguousarray(y).reshape(b, f * h * w, c)


# ----------------------------------------------------------------------------------------------------------------
# projection epilogue: WanRMSNorm, RoPE, window partition
# ----------------------------------------------------------------------------------------------------------------
def to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round to nearest, ties to even) and return them as float32."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rope_tables(head_dim: int = HEAD_DIM, end: int = 1024, theta: float = 10000.0) -> list:
    """`RopeTables.init` (DiT.swift:58-78): per axis (t, h, w) with sub-dims (d - 2(d//3), d//3, d//3), pair j has
    frequency theta^(-2j/dim) over its OWN sub-dimension; row p = (cos, sin)(p * freq) computed in float64, stored
    float32. Returns [(cos_t, sin_t), (cos_h, sin_h), (cos_w, sin_w)], each (end, pairs)."""
    out = []
    for dim in (head_dim - 2 * (head_dim // 3), head_dim // 3, head_dim // 3):
        n = dim // 2
        freq = 1.0 / np.power(float(theta), 2.0 * np.arange(n, dtype=np.float64) / dim)
        ang = np.arange(end, dtype=np.float64)[:, None] * freq[None, :]
        out.append((np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)))
    return out


def rope_tables_flat(theta: float = 10000.0) -> np.ndarray:
    """The tables packed as the C ABI's fvsr_rope_tables lays them out: cos_t, sin_t, cos_h, sin_h, cos_w, sin_w."""
    return np.concatenate([a.reshape(-1) for pair in rope_tables(theta=theta) for a in pair])


def wan_rms_norm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6, bf16: bool = True) -> np.ndarray:
    """`WanRMSNorm` (DiT.swift:42-46): fp32 x * rsqrt(mean(x^2, last axis) + eps), cast to the input dtype, times
    the weight (a product rounded to the input dtype). bf16=True models bfloat16 tensors (values exact in bf16)."""
    xf = x.astype(np.float32)
    ms = (xf * xf).mean(axis=-1, keepdims=True, dtype=np.float32)
    n = xf * (np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32))
    if bf16:
        return to_bf16(to_bf16(n) * weight.astype(np.float32))
    return n * weight.astype(np.float32)


def rope_apply(x: np.ndarray, heads: int, cos: np.ndarray, sin: np.ndarray, bf16: bool = True) -> np.ndarray:
    """`ropeApply` (DiT.swift:101-107): view each head as 64 (re = even, im = odd) pairs, multiply by e^{i theta}
    in fp32 (each product and sum rounded once), cast back. x (L, heads*128); cos, sin (L, 64) fp32."""
    L, c = x.shape
    xf = x.astype(np.float32).reshape(L, heads, c // heads // 2, 2)
    re, im = xf[..., 0], xf[..., 1]
    cs, sn = cos[:, None, :].astype(np.float32), sin[:, None, :].astype(np.float32)
    out = np.stack([re * cs - im * sn, re * sn + im * cs], axis=-1).reshape(L, c)
    return to_bf16(out) if bf16 else out


def rope_grid(f: int, h: int, w: int, t0: int, theta: float = 10000.0):
    """`RopeTables.grid` (DiT.swift:81-97): (cos, sin) of shape (f*h*w, 64) for an (f, h, w) token grid whose
    temporal positions start at t0."""
    (ct, st), (ch, sh), (cw, sw) = rope_tables(theta=theta)
    T, Y, X = np.meshgrid(np.arange(t0, t0 + f), np.arange(h), np.arange(w), indexing="ij")
    T, Y, X = T.reshape(-1), Y.reshape(-1), X.reshape(-1)
    return (np.concatenate([ct[T], ch[Y], cw[X]], axis=1), np.concatenate([st[T], sh[Y], sw[X]], axis=1))


def qkv_epilogue(q: np.ndarray, k: np.ndarray, v: np.ndarray, f: int, h: int, w: int, heads: int, t0: int,
                 wq: np.ndarray, wk: np.ndarray, eps: float = 1e-6, bf16: bool = True):
    """The projection epilogue of blockForward (DiT.swift:498-506): q' = ropeApply(normQ(q)), k' =
    ropeApply(normK(k)), then windowPartition of q', k', v. q, k, v (f*h*w, C) natural token order; returns the three
    as (f*h*w, C) window-ordered float32 arrays (bfloat16 values when bf16)."""
    cos, sin = rope_grid(f, h, w, t0)
    qn = rope_apply(wan_rms_norm(q, wq, eps, bf16), heads, cos, sin, bf16)
    kn = rope_apply(wan_rms_norm(k, wk, eps, bf16), heads, cos, sin, bf16)
    c = q.shape[-1]
    return tuple(window_partition(x[None].astype(np.float32), f, h, w).reshape(-1, c) for x in (qn, kn, v))


# ----------------------------------------------------------------------------------------------------------------
# selection
# ----------------------------------------------------------------------------------------------------------------
def local_block_mask(bh: int, bw: int, r: int) -> np.ndarray:
    """(s, s) bool, s = bh*bw: key block (kr, kc) visible to query block (qr, qc) iff kr in [qr - r//2, qr - r//2 + r - 1]
    and likewise for columns, unclamped. DiT.swift:130-145 (`localBlockMask`)."""
    half = r // 2
    qr = np.arange(bh)[:, None, None, None]
    qc = np.arange(bw)[None, :, None, None]
    kr = np.arange(bh)[None, None, :, None]
    kc = np.arange(bw)[None, None, None, :]
    in_row = (kr >= qr - half) & (kr <= qr - half + r - 1)
    in_col = (kc >= qc - half) & (kc <= qc - half + r - 1)
    return (in_row & in_col).reshape(bh * bw, bh * bw)


def pool_blocks(x: np.ndarray, heads: int, n_tokens: int | None = None) -> np.ndarray:
    """fp32 mean over each 128-token window, per head: (L, H*D) -> (H, N, D). DiT.swift:161-162.

    `n_tokens` (ragged extension): only the first n_tokens rows are real; a partial last block averages its valid rows.
    """
    x = np.asarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
    L = x.shape[0] if n_tokens is None else n_tokens
    c = x.shape[-1]
    d = c // heads
    nb = -(-L // BLOCK)
    out = np.empty((nb, c), dtype=np.float32)
    full = L // BLOCK
    if full:
        out[:full] = x[: full * BLOCK].reshape(full, BLOCK, c).mean(axis=1, dtype=np.float32)
    if nb > full:
        out[full] = x[full * BLOCK: L].mean(axis=0, dtype=np.float32)
    return np.ascontiguousarray(out.reshape(nb, heads, d).transpose(1, 0, 2))


def block_scores(pq: np.ndarray, pk: np.ndarray, local: np.ndarray, s: int) -> np.ndarray:
    """scores = pq @ pk^T / sqrt(d) (a divide, DiT.swift:163), plus the local mask (0 / -inf) tiled over every
    (query slice, key slice) pair (DiT.swift:165-167). (H, Nq, Nk) fp32."""
    d = pq.shape[-1]
    sc = np.matmul(pq, pk.transpose(0, 2, 1)) / np.float32(math.sqrt(d))
    nq, nk = pq.shape[1], pk.shape[1]
    lm = np.where(np.asarray(local, dtype=bool).reshape(s, s), np.float32(0), np.float32(-np.inf))
    qi = np.arange(nq) % s
    kj = np.arange(nk) % s
    return (sc + lm[qi][:, kj][None]).astype(np.float32)


def softmax_rows(x: np.ndarray) -> np.ndarray:
    """fp32 softmax over the last axis (DiT.swift:168)."""
    m = x.max(axis=-1, keepdims=True)
    e = np.exp(x - m, dtype=np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def topk_threshold(flat: np.ndarray, topk: int) -> np.ndarray:
    """Per row: the (k+1)-th largest value, k = min(n - 1, topk) (DiT.swift:170-172). Returns (rows, 1)."""
    n = flat.shape[1]
    k = min(n - 1, topk)
    return np.sort(flat, axis=1)[:, n - 1 - k: n - k]


def draft_block_mask_and_probs(qW: np.ndarray, kW: np.ndarray, heads: int, q_slices: int, s: int,
                               local: np.ndarray, topk: int, lq: int | None = None, lk: int | None = None):
    """`draftBlockMaskAndProbs` (DiT.swift:158-174): returns (mask (H, Nq, Nk) fp32 0/1, probs (H, Nq, Nk) fp32).

    qW: (Lq, C) or (Nq, 128, C) window-order queries; kW likewise for keys (cache + new).
    Keeps, per (head, query temporal slice), the block pairs STRICTLY above the (k+1)-th largest probability.
    """
    pq = pool_blocks(qW, heads, lq)
    pk = pool_blocks(kW, heads, lk)
    nq, nk = pq.shape[1], pk.shape[1]
    if nq % q_slices:
        raise ValueError("query blocks must split evenly into temporal slices")
    probs = softmax_rows(block_scores(pq, pk, local, s))
    flat = probs.reshape(heads * q_slices, (nq // q_slices) * nk)
    thr = topk_threshold(flat, topk)
    mask = (flat > thr).astype(np.float32).reshape(heads, nq, nk)
    return mask, probs


def block_lists(block_mask: np.ndarray):
    """`kernelBlockAttention`'s list build (SparseAttention.swift:175-177): kcnt (H, Nq) int32 = selected count;
    kidx (H, Nq, Nk) int32 = argsort(!sel), i.e. the selected key blocks first (ascending), then the rest."""
    sel = np.asarray(block_mask) > 0.5
    kcnt = sel.sum(axis=-1).astype(np.int32)
    kidx = np.argsort(~sel, axis=-1, kind="stable").astype(np.int32)
    return kidx, kcnt


# ----------------------------------------------------------------------------------------------------------------
# attention
# ----------------------------------------------------------------------------------------------------------------
def expand_token_mask(bm: np.ndarray, lq: int, lk: int) -> np.ndarray:
    """(Nq, Nk) bool block mask -> (lq, lk) token mask, ragged tails sliced (oracle/block_sparse_attn.py:34)."""
    return np.repeat(np.repeat(bm, BLOCK, axis=0)[:lq], BLOCK, axis=1)[:, :lk]


def block_masked_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, block_mask: np.ndarray, heads: int,
                           dtype=np.float64, heads_subset=None, qblocks_subset=None) -> np.ndarray:
    """Dense attention under the expanded 128x128 block mask, per head; a query block that selects nothing -> 0.

    `blockMaskedAttention` (DiT.swift:279-313) / `block_sparse_attn_func` (oracle/block_sparse_attn.py:20-38).
    q (Lq, H*D), k/v (Lk, H*D) window-order tokens; block_mask (H, Nq, Nk) tested > 0.5; scale 1/sqrt(D)
    (DiT.swift:284). Returns (Lq, H*D) in `dtype`. `heads_subset` / `qblocks_subset` restrict the work (rows not
    computed are left NaN) so large shapes can be spot-checked.
    """
    q = np.asarray(q).reshape(-1, q.shape[-1])
    k = np.asarray(k).reshape(-1, k.shape[-1])
    v = np.asarray(v).reshape(-1, v.shape[-1])
    lq, c = q.shape
    lk = k.shape[0]
    d = c // heads
    scale = 1.0 / math.sqrt(d)
    out = np.full((lq, c), np.nan, dtype=dtype)
    bm_all = np.asarray(block_mask) > 0.5
    hs = range(heads) if heads_subset is None else heads_subset
    nq = bm_all.shape[1]
    qbs = range(nq) if qblocks_subset is None else qblocks_subset
    for h in hs:
        kh = k[:, h * d:(h + 1) * d].astype(dtype)
        vh = v[:, h * d:(h + 1) * d].astype(dtype)
        for qb in qbs:
            r0, r1 = qb * BLOCK, min(lq, (qb + 1) * BLOCK)
            if r0 >= r1:
                continue
            sel = bm_all[h, qb]
            if not sel.any():
                out[r0:r1, h * d:(h + 1) * d] = 0
                continue
            tok = np.repeat(sel, BLOCK)[:lk]
            qh = q[r0:r1, h * d:(h + 1) * d].astype(dtype)
            sc = (qh @ kh[tok].T) * dtype(scale)
            sc = sc - sc.max(axis=1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(axis=1, keepdims=True)
            out[r0:r1, h * d:(h + 1) * d] = p @ vh[tok]
    return out


def block_sparse_attention_lists(q, k, v, kidx, kcnt, heads: int, dtype=np.float64):
    """The same result computed from (kidx, kcnt) lists instead of a mask: only kcnt[h, i] leading entries of
    kidx[h, i] are used, in list order (SparseAttention.swift:47-53,71-72)."""
    nq = kcnt.shape[1]
    nk = int(np.max(kidx)) + 1 if kidx.size else 0
    nk = max(nk, kidx.shape[-1])
    bm = np.zeros((heads, nq, nk), dtype=np.float32)
    for h in range(heads):
        for i in range(nq):
            c = int(kcnt[h, i])
            bm[h, i, kidx[h, i, :c]] = 1
    return block_masked_attention(q, k, v, bm, heads, dtype=dtype)


def attention_bruteforce(q, k, v, block_mask, heads: int) -> np.ndarray:
    """float64 scalar loops over every (head, query token): the definition, for tiny shapes only."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    lq, c = q.shape
    lk = k.shape[0]
    d = c // heads
    out = np.zeros((lq, c))
    for h in range(heads):
        hs = slice(h * d, (h + 1) * d)
        for i in range(lq):
            keys = [j for j in range(lk) if block_mask[h, i // BLOCK, j // BLOCK] > 0.5]
            if not keys:
                continue
            logits = [float(np.dot(q[i, hs], k[j, hs])) / math.sqrt(d) for j in keys]
            m = max(logits)
            ws = [math.exp(x - m) for x in logits]
            z = math.fsum(ws)
            acc = np.zeros(d)
            for wj, j in zip(ws, keys):
                acc += wj * v[j, hs]
            out[i, hs] = acc / z
    return out


# ----------------------------------------------------------------------------------------------------------------
# KV window cache
# ----------------------------------------------------------------------------------------------------------------
@dataclass
class KVWindowCache:
    """The per-block window K/V cache of `blockForward` (DiT.swift:507-511 concat, :532-538 trim; state in
    `ChunkState`, Pipeline.swift:87-91; kvLen = Int(kvRatio) = 3, Pipeline.swift:129).

    `attend_view(kW, vW, seqlen)` returns what the attention sees (cache ++ new); `trim()` then applies the rule:
    if the held window count over one slice's windows exceeds kv_len, drop the OLDEST slice (exactly one).
    """
    kv_len: int = 3
    k: np.ndarray | None = None
    v: np.ndarray | None = None
    one_len: int = 0
    _pending: tuple = field(default=None, repr=False)

    def attend_view(self, kW: np.ndarray, vW: np.ndarray, seqlen: int):
        self.one_len = kW.shape[0] // seqlen
        if self.k is not None:
            kW = np.concatenate([self.k, kW], axis=0)
            vW = np.concatenate([self.v, vW], axis=0)
        self._pending = (kW, vW)
        return kW, vW

    def trim(self):
        kW, vW = self._pending
        if kW.shape[0] // self.one_len > self.kv_len:
            self.k, self.v = kW[self.one_len:], vW[self.one_len:]
        else:
            self.k, self.v = kW, vW
        self._pending = None


# ----------------------------------------------------------------------------------------------------------------
# geometry
# ----------------------------------------------------------------------------------------------------------------
def step_topk(s: int, topk_ratio: float) -> int:
    """topk = Int(s^2 * ratio) - 1 (DiT.swift:482)."""
    return int(float(s * s) * topk_ratio) - 1


def default_topk_ratio(height: int, width: int) -> float:
    """2*768*1280 / (H*W) at the output size (Pipeline.swift:68)."""
    return 2.0 * 768 * 1280 / float(height * width)


def in_window_pairs(local: np.ndarray, s: int, nk: int) -> int:
    """Number of in-window (query spatial block, key block) pairs in one (head, query slice) row of the top-k."""
    lm = np.asarray(local, dtype=bool).reshape(s, s)
    return int(lm[:, np.arange(nk) % s].sum())


def topk_for_kept_fraction(local: np.ndarray, s: int, nk: int, fraction: float) -> int:
    """Explicit top-k count that keeps `fraction` of the in-window pairs of a (head, query slice) row."""
    return int(math.floor(fraction * in_window_pairs(local, s, nk)))


def expected_kept_fraction(topk: int, s: int, nk: int) -> float:
    """`auto` dispatch estimate min(1, (topk + 1) / (s * Nk)) (DiT.swift:520)."""
    return min(1.0, float(topk + 1) / float(s * nk))


# ----------------------------------------------------------------------------------------------------------------
# comparison
# ----------------------------------------------------------------------------------------------------------------
def compare(got: np.ndarray, ref: np.ndarray) -> dict:
    """rel = max|got - ref| / max|ref| (Gates.swift:19-29)."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = np.abs(g - r)
    max_abs = float(d.max()) if d.size else 0.0
    ref_max = float(np.abs(r).max()) if r.size else 0.0
    mse = float((d * d).mean()) if d.size else 0.0
    peak = max(ref_max, 1e-12)
    psnr = math.inf if mse == 0 else 10 * math.log10(peak * peak / mse)
    return {"max_abs": max_abs, "ref_max": ref_max, "rel": max_abs / peak, "psnr": psnr}


def mask_flip_report(mine: np.ndarray, golden: np.ndarray, probs: np.ndarray, seqlen: int) -> dict:
    """Block-mask agreement with the near-tie rule of Gates.swift:239-277: a flip is legitimate when the flipped
    probability is below 1e-30 (softmax underflow) or within 1e-3 (relative) of its nearest distinct sorted
    neighbour in its (head, query slice) row."""
    heads, nq, nk = probs.shape
    flat = probs.reshape(heads * seqlen, (nq // seqlen) * nk)
    flips = (np.abs(np.asarray(mine) - np.asarray(golden)) > 0.5).reshape(flat.shape)
    n_flip = int(flips.sum())
    worst_gap, underflow = 0.0, 0
    for r in np.nonzero(flips.any(axis=1))[0]:
        row = flat[r]
        srow = np.sort(row)
        for c in np.nonzero(flips[r])[0]:
            p = row[c]
            if p < 1e-30:
                underflow += 1
                continue
            idx = int(np.searchsorted(srow, p))
            lo = srow[idx - 1] if idx > 0 else p
            hi = srow[idx + 1] if idx + 1 < srow.size else p
            worst_gap = max(worst_gap, min(abs(p - lo), abs(hi - p)) / max(p, 1e-38))
    return {"flips": n_flip, "underflow": underflow, "worst_gap": float(worst_gap),
            "legit": worst_gap <= 1e-3}


def threshold_margin(probs: np.ndarray, seqlen: int, topk: int) -> float:
    """Smallest relative gap, over the (head, slice) rows, between the top-k threshold value and its nearest
    distinct neighbour above it: a mask is bit-exactly reproducible by any fp32 implementation when this margin is
    well above fp32 rounding (the 'no near-ties' condition)."""
    heads, nq, nk = probs.shape
    flat = probs.reshape(heads * seqlen, (nq // seqlen) * nk)
    n = flat.shape[1]
    k = min(n - 1, topk)
    if k <= 0:   # nothing is kept: the threshold is the row's max, with no neighbour above it to tie with
        return math.inf
    srow = np.sort(flat, axis=1)
    thr = srow[:, n - 1 - k]
    above = srow[:, n - k]
    gap = (above - thr) / np.maximum(above, 1e-38)
    return float(gap.min())
