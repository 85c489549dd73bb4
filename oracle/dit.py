"""CPU oracle for the dense parts of one FlashVSR DiT block around the LCSA layer call.

TEST INFRASTRUCTURE ONLY: the HIP path's results are compared against this module's. Only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it; the product path never does.

It restates, in numpy, the streaming `blockForward` of the reference (xocialize/mlx-flashvsr-swift), with bfloat16
tensors modelled as float32 arrays holding bf16 values (each MLX op rounds its result to bf16):

  linear (y = x W^T + b, one rounding)        Sources/FlashVSRMLX/DiT.swift:319-321,341-342 (MLX Linear)
  gelu_tanh                                   Sources/FlashVSRMLX/DiT.swift:371 (GELU(approximation: .tanh))
  layer_norm (affine or not, fp32 inside)     Sources/FlashVSRMLX/DiT.swift:368-370 (MLX LayerNorm)
  modulation rows                             Sources/FlashVSRMLX/DiT.swift:495-497
  cross_kv (CrossAttention.initCache)         Sources/FlashVSRMLX/DiT.swift:346-350
  cross_attention                             Sources/FlashVSRMLX/DiT.swift:352-361
  block_forward                               Sources/FlashVSRMLX/DiT.swift:491-551

The self-attention core (norm + RoPE + window partition, cache, draft mask, block attention, window reverse) is
oracle.lcsa's. Pinned in tests/test_oracle_dit.py: linear, GELU and LayerNorm against torch's CPU float32 routines
(torch.nn.functional.linear / gelu(approximate="tanh") / layer_norm) and the closed forms GELU(0) = 0,
GELU(x) -> x for large x, LayerNorm output mean 0 and variance 1; cross_attention against a float64 brute-force
softmax; block_forward against its own steps composed by hand and the identity cases (zero gates leave x to the
cross-attention residual only).
"""
from __future__ import annotations

import math

import numpy as np

from . import lcsa as L

HEAD_DIM = L.HEAD_DIM
bf = L.to_bf16


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray | None = None, bf16: bool = True) -> np.ndarray:
    """MLX `Linear`: x W^T + b accumulated in fp32 (float64 here), rounded once to the output dtype."""
    y = x.astype(np.float64) @ w.astype(np.float64).T
    if b is not None:
        y = y + b.astype(np.float64)
    y = y.astype(np.float32)
    return bf(y) if bf16 else y


def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in float64."""
    x = x.astype(np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def layer_norm(x: np.ndarray, eps: float = 1e-6, w: np.ndarray | None = None, b: np.ndarray | None = None,
               bf16: bool = True) -> np.ndarray:
    """MLX `LayerNorm` over the last axis: (x - mean) / sqrt(var + eps) in fp32, times w plus b when affine, one
    rounding to the output dtype."""
    xf = x.astype(np.float64)
    mean = xf.mean(axis=-1, keepdims=True)
    var = ((xf - mean) ** 2).mean(axis=-1, keepdims=True)
    n = (xf - mean) / np.sqrt(var + eps)
    if w is not None:
        n = n * w.astype(np.float64)
    if b is not None:
        n = n + b.astype(np.float64)
    n = n.astype(np.float32)
    return bf(n) if bf16 else n


def modulate(n: np.ndarray, scale: np.ndarray, shift: np.ndarray) -> np.ndarray:
    """`norm(x) * (1 + scale) + shift` as three bf16 ops (DiT.swift:498,546)."""
    return bf(bf(n * bf(1.0 + scale)) + shift)


def cross_kv(context: np.ndarray, wk, bk, wv, bv, norm_k_w, eps: float = 1e-6):
    """`CrossAttention.initCache` (DiT.swift:346-350): k = normK(k(ctx)), v = v(ctx)."""
    return L.wan_rms_norm(linear(context, wk, bk), norm_k_w, eps), linear(context, wv, bv)


def cross_attention(x: np.ndarray, wq, bq, norm_q_w, k: np.ndarray, v: np.ndarray, wo, bo, heads: int,
                    eps: float = 1e-6) -> np.ndarray:
    """`CrossAttention.callAsFunction` (DiT.swift:352-361): o(SDPA(normQ(q(x)), cacheK, cacheV)) per head, scale
    1/sqrt(128), no mask; the attention output is rounded to bf16 before the o projection."""
    q = L.wan_rms_norm(linear(x, wq, bq), norm_q_w, eps)
    lq, c = q.shape
    out = np.empty((lq, c), dtype=np.float64)
    d = c // heads
    for h in range(heads):
        s = slice(h * d, (h + 1) * d)
        sc = (q[:, s].astype(np.float64) @ k[:, s].astype(np.float64).T) / math.sqrt(d)
        sc -= sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=1, keepdims=True)
        out[:, s] = p @ v[:, s].astype(np.float64)
    return linear(bf(out.astype(np.float32)), wo, bo)


def block_forward(x: np.ndarray, W: dict, t_mod: np.ndarray, cache: L.KVWindowCache, f: int, h: int, w: int,
                  heads: int, t0: int, local: np.ndarray, topk: int, eps: float = 1e-6):
    """The streaming `blockForward` (DiT.swift:491-551) on natural-order tokens x (f*h*w, C) (bf16 values).
    W holds the block's weights under the C ABI's field names (q_weight, ..., ffn2_bias; cross_k / cross_v the
    cached context K/V). Returns (x_out, mask) and updates `cache` (concat, then trim to kv_len slices)."""
    c = x.shape[1]
    mod = bf(W["modulation"].reshape(6, c) + t_mod.reshape(6, c))                       # DiT.swift:495-497
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = mod
    in_x = modulate(layer_norm(x, eps), scale_msa, shift_msa)                            # :498
    q = linear(in_x, W["q_weight"], W.get("q_bias"))                                     # :500-502
    k = linear(in_x, W["k_weight"], W.get("k_bias"))
    v = linear(in_x, W["v_weight"], W.get("v_bias"))
    qW, kW, vW = L.qkv_epilogue(q, k, v, f, h, w, heads, t0, W["norm_q_weight"], W["norm_k_weight"], eps)
    seqlen = f // 2
    kW, vW = cache.attend_view(kW, vW, seqlen)                                           # :507-511
    s = (h // 8) * (w // 8)
    mask, _ = L.draft_block_mask_and_probs(qW, kW, heads, seqlen, s, local, topk)       # :512-514
    attn = L.block_masked_attention(qW, kW, vW, mask, heads, dtype=np.float64)           # :516-527
    cache.trim()                                                                         # :532-538
    attn = bf(L.window_reverse(attn.astype(np.float32)[None], 1, f, h, w)[0])            # :539
    sa_out = linear(attn, W["o_weight"], W.get("o_bias"))
    x = bf(x + bf(gate_msa * sa_out))                                                    # :541
    ca_in = layer_norm(x, eps, W["norm3_weight"], W.get("norm3_bias"))                   # :542
    ca_out = cross_attention(ca_in, W["cross_q_weight"], W.get("cross_q_bias"), W["cross_norm_q_weight"],
                             W["cross_k"], W["cross_v"], W["cross_o_weight"], W.get("cross_o_bias"), heads, eps)
    x = bf(x + ca_out)                                                                   # :545
    in_f = modulate(layer_norm(x, eps), scale_mlp, shift_mlp)                            # :546
    hid = bf(gelu_tanh(linear(in_f, W["ffn1_weight"], W.get("ffn1_bias"))).astype(np.float32))
    y = linear(hid, W["ffn2_weight"], W.get("ffn2_bias"))
    x = bf(x + bf(gate_mlp * y))                                                         # :547
    return x, mask
