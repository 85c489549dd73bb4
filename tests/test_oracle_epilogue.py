"""CPU checks that pin the oracle's projection epilogue (WanRMSNorm, RoPE tables, ropeApply, window partition;
DiT.swift:34-47,52-107,111-118,496-506) before the GPU results are compared against it.

Sources of truth other than the oracle's formulas: torch's bfloat16 conversion and float32 RMS norm
(torch.nn.functional.rms_norm), complex multiplication in complex128, and closed forms (position 0 is the identity,
a rotation keeps each pair's length, cos^2 + sin^2 = 1, the first frequency of every axis is 1 rad per position,
RMS normalisation is scale invariant and leaves unit RMS).
"""
import math

import numpy as np
import pytest
import torch

from oracle import lcsa as O


def test_to_bf16_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10,
                        # exact ties between two bfloat16 values, both parities of the kept mantissa
                        (np.arange(1, 2000, dtype=np.float32) * 2 + 1) * np.float32(2 ** -8) + 1,
                        np.array([0.0, -0.0, 1e-30, -3.0e38], dtype=np.float32)]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.to_bf16(x), ref)


def test_rope_tables_closed_forms():
    (ct, st), (ch, sh), (cw, sw) = O.rope_tables()
    assert ct.shape == (1024, 22) and ch.shape == (1024, 21) and cw.shape == (1024, 21)
    for c, s in ((ct, st), (ch, sh), (cw, sw)):
        np.testing.assert_array_equal(c[0], 1.0)
        np.testing.assert_array_equal(s[0], 0.0)
        # pair 0 turns by 1 rad per position on every axis
        np.testing.assert_allclose(c[1, 0], math.cos(1.0), rtol=1e-7)
        np.testing.assert_allclose(s[1, 0], math.sin(1.0), rtol=1e-7)
        np.testing.assert_allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, 1.0, atol=3e-7)
    # each axis uses its OWN sub-dimension: t pair 5 at position 7 has angle 7 * 10000^(-10/44), h pair 5 10000^(-10/42)
    np.testing.assert_allclose(ct[7, 5], math.cos(7 * 10000 ** (-10 / 44)), rtol=1e-6)
    np.testing.assert_allclose(sh[7, 5], math.sin(7 * 10000 ** (-10 / 42)), rtol=1e-6)
    flat = O.rope_tables_flat()
    assert flat.shape == (2 * 1024 * 22 + 4 * 1024 * 21,)
    np.testing.assert_array_equal(flat[:1024 * 22], ct.reshape(-1))
    np.testing.assert_array_equal(flat[-1024 * 21:], sw.reshape(-1))


def test_wan_rms_norm_matches_torch_rms_norm():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 1536)) * rng.uniform(0.1, 5.0, (64, 1))).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 1536).astype(np.float32)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (1536,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(O.wan_rms_norm(x, w, bf16=False), ref, rtol=2e-6, atol=1e-7)


def test_wan_rms_norm_invariants():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 1536)).astype(np.float32)
    one = np.ones(1536, dtype=np.float32)
    n = O.wan_rms_norm(x, one, eps=0.0, bf16=False)
    np.testing.assert_allclose(np.sqrt((n.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-6)
    np.testing.assert_allclose(O.wan_rms_norm(4 * x, one, eps=0.0, bf16=False), n, rtol=1e-6)
    # bf16 mode: every output is a bfloat16 value
    nb = O.wan_rms_norm(O.to_bf16(x), one)
    np.testing.assert_array_equal(nb, O.to_bf16(nb))


def test_rope_apply_matches_complex_multiplication():
    rng = np.random.default_rng(3)
    f, h, w, heads = 2, 8, 16, 3
    L = f * h * w
    x = rng.standard_normal((L, heads * 128)).astype(np.float32)
    cos, sin = O.rope_grid(f, h, w, t0=5)
    got = O.rope_apply(x, heads, cos, sin, bf16=False)
    z = x.astype(np.float64).reshape(L, heads, 64, 2)
    zc = (z[..., 0] + 1j * z[..., 1]) * (cos.astype(np.float64) + 1j * sin.astype(np.float64))[:, None, :]
    ref = np.stack([zc.real, zc.imag], -1).reshape(L, heads * 128)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-6)
    # rotation keeps each pair's length
    g = got.astype(np.float64).reshape(L, heads, 64, 2)
    np.testing.assert_allclose((g ** 2).sum(-1), (z ** 2).sum(-1), rtol=1e-5)


def test_rope_grid_positions():
    # token (t, y, x) uses table rows t0 + t, y, x; at t0 = 0 the first token is the identity rotation
    cos, sin = O.rope_grid(4, 16, 8, t0=0)
    np.testing.assert_array_equal(cos[0], 1.0)
    np.testing.assert_array_equal(sin[0], 0.0)
    (ct, _), (ch, _), (cw, _) = O.rope_tables()
    c3, _ = O.rope_grid(4, 16, 8, t0=3)
    tok = (2 * 16 + 5) * 8 + 6
    np.testing.assert_array_equal(c3[tok], np.concatenate([ct[5], ch[5], cw[6]]))


def test_qkv_epilogue_composition():
    rng = np.random.default_rng(4)
    f, h, w, heads = 2, 16, 16, 2
    L, c = f * h * w, heads * 128
    q, k, v = (O.to_bf16(rng.standard_normal((L, c)).astype(np.float32)) for _ in range(3))
    wq = O.to_bf16(rng.uniform(0.5, 1.5, c).astype(np.float32))
    wk = O.to_bf16(rng.uniform(0.5, 1.5, c).astype(np.float32))
    qo, ko, vo = O.qkv_epilogue(q, k, v, f, h, w, heads, 7, wq, wk)
    cos, sin = O.rope_grid(f, h, w, 7)
    nat = O.rope_apply(O.wan_rms_norm(k, wk), heads, cos, sin)
    np.testing.assert_array_equal(O.window_reverse(ko, 1, f, h, w)[0], nat)
    np.testing.assert_array_equal(vo, O.window_partition(v[None], f, h, w).reshape(-1, c))
    assert np.array_equal(qo, O.to_bf16(qo))
