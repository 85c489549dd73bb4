"""CPU checks that pin the oracle's dense DiT-block pieces (oracle/dit.py; DiT.swift:317-381,491-551) before the GPU
results are compared against it.

Sources of truth other than the oracle's own formulas: torch's CPU float32 routines (F.linear, F.gelu with
approximate="tanh", F.layer_norm), float64 brute-force softmax attention, and closed forms (GELU(0) = 0 and
GELU(x) -> x / 0 far out, LayerNorm rows with mean 0 and variance 1, a zero gate leaves the residual stream alone).
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import dit as D
from oracle import lcsa as L


def _rng(seed=0):
    return np.random.default_rng(seed)


def test_linear_matches_torch():
    r = _rng(1)
    x = L.to_bf16(r.standard_normal((37, 64)).astype(np.float32))
    w = L.to_bf16((r.standard_normal((48, 64)) / 8).astype(np.float32))
    b = L.to_bf16(r.standard_normal(48).astype(np.float32))
    ref = F.linear(torch.from_numpy(x).double(), torch.from_numpy(w).double(), torch.from_numpy(b).double())
    np.testing.assert_array_equal(D.linear(x, w, b), L.to_bf16(ref.float().numpy()))
    # a transposed-operand mistake would change the shape or the values
    assert D.linear(x, w).shape == (37, 48)


def test_gelu_tanh_matches_torch_and_closed_forms():
    x = np.linspace(-8, 8, 4001)
    ref = F.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(D.gelu_tanh(x), ref, rtol=0, atol=1e-12)
    assert D.gelu_tanh(np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(D.gelu_tanh(np.array([30.0, -30.0])), [30.0, 0.0], atol=1e-12)
    # differs from the erf form (a plausible mix-up) by ~1e-3 near x = 1.5
    erf = F.gelu(torch.tensor([1.5], dtype=torch.float64)).item()
    assert abs(D.gelu_tanh(np.array([1.5]))[0] - erf) > 1e-5


@pytest.mark.parametrize("affine", [False, True])
def test_layer_norm_matches_torch(affine):
    r = _rng(2)
    x = L.to_bf16((r.standard_normal((9, 256)) * 3 + 1).astype(np.float32))
    w = L.to_bf16(r.standard_normal(256).astype(np.float32)) if affine else None
    b = L.to_bf16(r.standard_normal(256).astype(np.float32)) if affine else None
    ref = F.layer_norm(torch.from_numpy(x).double(), (256,), None if w is None else torch.from_numpy(w).double(),
                       None if b is None else torch.from_numpy(b).double(), eps=1e-6)
    np.testing.assert_array_equal(D.layer_norm(x, 1e-6, w, b), L.to_bf16(ref.float().numpy()))
    if not affine:
        n = D.layer_norm(x, 1e-6, bf16=False).astype(np.float64)
        np.testing.assert_allclose(n.mean(axis=1), 0, atol=1e-6)
        np.testing.assert_allclose(n.var(axis=1), 1, atol=1e-5)


def test_cross_attention_matches_bruteforce():
    r = _rng(3)
    heads, c, lq, lc = 2, 256, 20, 33
    x = L.to_bf16(r.standard_normal((lq, c)).astype(np.float32))
    wq = L.to_bf16((r.standard_normal((c, c)) / 16).astype(np.float32))
    wo = L.to_bf16((r.standard_normal((c, c)) / 16).astype(np.float32))
    nq = L.to_bf16(np.abs(r.standard_normal(c)).astype(np.float32))
    k = L.to_bf16(r.standard_normal((lc, c)).astype(np.float32))
    v = L.to_bf16(r.standard_normal((lc, c)).astype(np.float32))
    got = D.cross_attention(x, wq, None, nq, k, v, wo, None, heads)
    q = L.wan_rms_norm(D.linear(x, wq), nq)
    ref = np.zeros((lq, c))
    for h in range(heads):
        for i in range(lq):
            s = [sum(float(q[i, h * 128 + d]) * float(k[j, h * 128 + d]) for d in range(128)) / math.sqrt(128)
                 for j in range(lc)]
            m = max(s)
            e = [math.exp(t - m) for t in s]
            z = sum(e)
            for d in range(128):
                ref[i, h * 128 + d] = sum(e[j] * float(v[j, h * 128 + d]) for j in range(lc)) / z
    np.testing.assert_array_equal(got, D.linear(L.to_bf16(ref.astype(np.float32)), wo))


def _block_weights(r, c, ffn, ctx_len, heads):
    def m(*shape, scale=1.0):
        return L.to_bf16((r.standard_normal(shape) * scale).astype(np.float32))
    W = {"modulation": m(6, c, scale=0.1)}
    for p in ("q", "k", "v", "o", "cross_q", "cross_k", "cross_v", "cross_o"):
        W[p + "_weight"] = m(c, c, scale=1 / math.sqrt(c))
        W[p + "_bias"] = m(c, scale=0.05)
    for p in ("norm_q", "norm_k", "cross_norm_q", "cross_norm_k"):
        W[p + "_weight"] = L.to_bf16((1 + 0.1 * r.standard_normal(c)).astype(np.float32))
    W["norm3_weight"] = L.to_bf16((1 + 0.1 * r.standard_normal(c)).astype(np.float32))
    W["norm3_bias"] = m(c, scale=0.05)
    W["ffn1_weight"] = m(ffn, c, scale=1 / math.sqrt(c))
    W["ffn1_bias"] = m(ffn, scale=0.05)
    W["ffn2_weight"] = m(c, ffn, scale=1 / math.sqrt(ffn))
    W["ffn2_bias"] = m(c, scale=0.05)
    ctx = m(ctx_len, c)
    W["cross_k"], W["cross_v"] = D.cross_kv(ctx, W["cross_k_weight"], W["cross_k_bias"], W["cross_v_weight"],
                                            W["cross_v_bias"], W["cross_norm_k_weight"])
    return W, ctx


def test_block_forward_composition_and_zero_gates():
    r = _rng(4)
    heads, c, ffn, f, h, w = 2, 256, 512, 2, 16, 16
    W, _ = _block_weights(r, c, ffn, 40, heads)
    x = L.to_bf16(r.standard_normal((f * h * w, c)).astype(np.float32))
    t_mod = L.to_bf16((r.standard_normal((6, c)) * 0.1).astype(np.float32))
    local = L.local_block_mask(2, 2, 3)
    out, mask = D.block_forward(x, W, t_mod, L.KVWindowCache(), f, h, w, heads, 0, local, 10)
    assert out.shape == x.shape and np.isfinite(out).all()
    assert mask.shape == (heads, 4, 4)
    # zero gates (modulation = -t_mod on the gate rows): the self-attention and FFN add nothing, so the output is
    # x + cross-attention(norm3(x)) exactly
    W0 = dict(W)
    mod = W["modulation"].copy()
    mod[2] = -t_mod[2]
    mod[5] = -t_mod[5]
    W0["modulation"] = mod
    out0, _ = D.block_forward(x, W0, t_mod, L.KVWindowCache(), f, h, w, heads, 0, local, 10)
    ca = D.cross_attention(D.layer_norm(x, 1e-6, W["norm3_weight"], W["norm3_bias"]), W["cross_q_weight"],
                           W["cross_q_bias"], W["cross_norm_q_weight"], W["cross_k"], W["cross_v"],
                           W["cross_o_weight"], W["cross_o_bias"], heads)
    np.testing.assert_array_equal(out0, L.to_bf16(x + ca))
    # the cache holds the chunk's window K/V afterwards
    cache = L.KVWindowCache()
    D.block_forward(x, W, t_mod, cache, f, h, w, heads, 0, local, 10)
    assert cache.k.shape == (f * h * w, c)
