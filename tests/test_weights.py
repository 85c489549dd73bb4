"""The weight-lane loader (fvsr_lcsa.weights; Weights.swift:10-71, convert_weights.py:12-17): the 825-key contract of
the released DiT (FlashVSRStructureTests.swift:14-25), lane choice, the upstream-name -> block-field mapping, the
sinusoidal time embedding (DiT.swift:435-443). CPU tests use CPU tensors and temporary safetensors files; the gpu
test runs a tiny checkpoint (dim 128, 1 head, FFN 256, 2 blocks; FlashVSRDiTConfig.tiny, DiT.swift:25-31) through
prepare + one block against the oracle."""
import math
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from fvsr_lcsa import weights as Wt


def _tiny_tensors(layers=2, dim=128, ffn=256, text_dim=64, freq_dim=32, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)

    def r(*shape, scale=1.0):
        return (torch.randn(shape, generator=g) * scale).to(dtype)
    t = {}
    for i in range(layers):
        p = f"blocks.{i}."
        for m in ("self_attn", "cross_attn"):
            for x in "qkvo":
                t[p + f"{m}.{x}.weight"] = r(dim, dim, scale=dim ** -0.5)
                t[p + f"{m}.{x}.bias"] = r(dim, scale=0.05)
            t[p + f"{m}.norm_q.weight"] = 1 + r(dim, scale=0.1)
            t[p + f"{m}.norm_k.weight"] = 1 + r(dim, scale=0.1)
        t[p + "norm3.weight"] = 1 + r(dim, scale=0.1)
        t[p + "norm3.bias"] = r(dim, scale=0.05)
        t[p + "ffn.0.weight"], t[p + "ffn.0.bias"] = r(ffn, dim, scale=dim ** -0.5), r(ffn, scale=0.05)
        t[p + "ffn.2.weight"], t[p + "ffn.2.bias"] = r(dim, ffn, scale=ffn ** -0.5), r(dim, scale=0.05)
        t[p + "modulation"] = r(1, 6, dim, scale=0.1)
    t["patch_embedding.weight"], t["patch_embedding.bias"] = r(dim, 1, 2, 2, 16), r(dim)
    t["text_embedding.0.weight"], t["text_embedding.0.bias"] = r(dim, text_dim, scale=text_dim ** -0.5), r(dim)
    t["text_embedding.2.weight"], t["text_embedding.2.bias"] = r(dim, dim, scale=dim ** -0.5), r(dim)
    t["time_embedding.0.weight"], t["time_embedding.0.bias"] = r(dim, freq_dim, scale=freq_dim ** -0.5), r(dim)
    t["time_embedding.2.weight"], t["time_embedding.2.bias"] = r(dim, dim, scale=dim ** -0.5), r(dim)
    t["time_projection.1.weight"], t["time_projection.1.bias"] = r(6 * dim, dim, scale=dim ** -0.5), r(6 * dim)
    t["head.head.weight"], t["head.head.bias"] = r(64, dim), r(64)
    t["head.modulation"] = r(1, 2, dim)
    return t


def test_key_contract_counts_like_the_released_dit():
    # 27 keys per block x 30 blocks + 15 top-level = 825 (FlashVSRStructureTests.swift:18)
    assert len(Wt.expected_keys(30)) == 825
    keys = Wt.expected_keys(30)
    assert "blocks.29.cross_attn.norm_k.weight" in keys and "blocks.0.ffn.2.bias" in keys
    assert "head.modulation" in keys and "time_projection.1.weight" in keys
    assert not any("norm1" in k or "norm2" in k for k in keys)   # norm1 / norm2 carry no affine
    assert Wt.verify_keys(keys) == 30


def test_verify_rejects_missing_and_unused():
    keys = Wt.expected_keys(3)
    with pytest.raises(Wt.LoadError, match="missing"):
        Wt.verify_keys(keys - {"blocks.1.self_attn.q.bias"})
    with pytest.raises(Wt.LoadError, match="unused"):
        Wt.verify_keys(keys | {"blocks.0.norm1.weight"})
    with pytest.raises(Wt.LoadError):
        Wt.verify_keys(keys - {"head.head.bias"})


def test_block_mapping_and_lane_choice(tmp_path):
    t = _tiny_tensors()
    save_file({k: v.to(torch.bfloat16) for k, v in t.items()}, str(tmp_path / "dit_bf16.safetensors"))
    save_file(t, str(tmp_path / "dit_fp32.safetensors"))
    w32 = Wt.DiTWeights.load(str(tmp_path), dtype=torch.float32, device="cpu")
    assert w32.layers == 2 and w32.dim == 128 and w32.heads == 1
    b1 = w32.block_tensors(1)
    assert set(b1) == set(Wt.BLOCK_KEYS.values())
    torch.testing.assert_close(b1["cross_k_weight"], t["blocks.1.cross_attn.k.weight"], rtol=0, atol=0)
    torch.testing.assert_close(b1["ffn2_bias"], t["blocks.1.ffn.2.bias"], rtol=0, atol=0)
    assert b1["modulation"].shape == (6, 128)
    # fp32 compute reads the fp32 lane; bf16 compute the bf16 lane; a missing lane falls back to the other
    assert Wt.pick_lane_file(str(tmp_path), "dit", torch.float32).endswith("dit_fp32.safetensors")
    assert Wt.pick_lane_file(str(tmp_path), "dit", torch.bfloat16).endswith("dit_bf16.safetensors")
    os.remove(tmp_path / "dit_bf16.safetensors")
    assert Wt.pick_lane_file(str(tmp_path), "dit", torch.bfloat16).endswith("dit_fp32.safetensors")
    with pytest.raises(Wt.LoadError, match="missing"):
        Wt.pick_lane_file(str(tmp_path), "prompt", torch.bfloat16)


def test_sinusoidal_closed_form():
    s = Wt.sinusoidal(256, 1000.0)
    assert s.shape == (1, 256)
    assert s[0, 0] == np.float32(math.cos(1000.0)) and s[0, 128] == np.float32(math.sin(1000.0))
    np.testing.assert_allclose(s[0, 5], math.cos(1000.0 * 10000 ** (-5 / 128)), rtol=1e-6)
    np.testing.assert_allclose(s[0, :128] ** 2 + s[0, 128:] ** 2, 1.0, atol=1e-6)


@pytest.mark.gpu
def test_tiny_checkpoint_block_matches_oracle(tmp_path, dev):
    from oracle import dit as D
    from oracle import lcsa as L

    import fvsr_lcsa

    t = _tiny_tensors(seed=3)
    save_file({k: v.to(torch.bfloat16) for k, v in t.items()}, str(tmp_path / "dit_bf16.safetensors"))
    ctx_raw = torch.randn((1, 40, 64), generator=torch.Generator().manual_seed(5))
    save_file({"context": ctx_raw.to(torch.bfloat16)}, str(tmp_path / "prompt_bf16.safetensors"))
    print("tiny checkpoint: load + prepare + block 0", flush=True)
    w = Wt.DiTWeights.load(str(tmp_path), device=dev)
    w.prepare(Wt.DiTWeights.load_prompt(str(tmp_path), device=dev))
    blk = w.block(0)

    def npy(x):
        return x.float().cpu().numpy()
    T = {k: npy(v) for k, v in w.t.items()}
    # prepare against the oracle: text embedding, time constants
    c_in = npy(ctx_raw.to(torch.bfloat16))[0]
    hid = L.to_bf16(D.gelu_tanh(D.linear(c_in, T["text_embedding.0.weight"], T["text_embedding.0.bias"])).astype(np.float32))
    ctx = D.linear(hid, T["text_embedding.2.weight"], T["text_embedding.2.bias"])
    assert np.linalg.norm(npy(w.context) - ctx) / np.linalg.norm(ctx) < 1e-2
    s = L.to_bf16(Wt.sinusoidal(32, 1000.0))
    e = D.linear(s, T["time_embedding.0.weight"], T["time_embedding.0.bias"])
    e = L.to_bf16((e / (1 + np.exp(-e.astype(np.float64)))).astype(np.float32))
    tv = D.linear(e, T["time_embedding.2.weight"], T["time_embedding.2.bias"])
    p = L.to_bf16((tv / (1 + np.exp(-tv.astype(np.float64)))).astype(np.float32))
    t_mod = D.linear(p, T["time_projection.1.weight"], T["time_projection.1.bias"]).reshape(6, 128)
    assert np.linalg.norm(npy(w.t_mod) - t_mod) / np.linalg.norm(t_mod) < 1e-2
    # one block on a 2 x 16 x 16 chunk, the oracle on the GPU's own context embedding and time constants
    W = {f: npy(v) for f, v in w.block_tensors(0).items()}
    W["cross_k"], W["cross_v"] = D.cross_kv(npy(w.context), W["cross_k_weight"], W["cross_k_bias"],
                                            W["cross_v_weight"], W["cross_v_bias"], W["cross_norm_k_weight"])
    local = L.local_block_mask(2, 2, 1)
    ring = fvsr_lcsa.KVRing(1, 1, 2, 2, capacity=4, kv_len=3, device=dev.index or 0)
    x = L.to_bf16(np.random.default_rng(9).standard_normal((512, 128)).astype(np.float32))
    xg = torch.from_numpy(x).to(torch.bfloat16).to(dev)
    blk.forward(ring, 0, xg, w.t_mod, 1, 0, local, 100)
    torch.cuda.synchronize()
    ref, _ = D.block_forward(x, W, npy(w.t_mod), L.KVWindowCache(), 2, 16, 16, 1, 0, local, 100)
    err = np.linalg.norm(npy(xg) - ref) / np.linalg.norm(ref)
    print(f"  rel err {err:.3e}", flush=True)
    assert err < 1e-2   # 128 channels: fewer elements per norm than the full-width test, so a looser bound
    ring.close()
