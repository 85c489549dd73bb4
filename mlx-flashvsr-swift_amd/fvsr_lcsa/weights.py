"""Weight-lane loader for the DiT blocks: the published FlashVSR v1.1 files (`dit_<lane>.safetensors`,
`prompt_<lane>.safetensors`, lane = bf16 | fp32; Weights.swift:10-71, oracle/convert_weights.py:12-17) with
upstream's parameter names, mapped onto the fields of fvsr_dit_block_weights.

  DiTWeights.load(directory, dtype)   FlashVSRPipeline.load (Weights.swift:49-71): the lane that matches the compute
                                      dtype if present, else the other lane, cast; every key of the 825-key contract
                                      present and no other (the reference's `verify: [.all]`,
                                      FlashVSRStructureTests.swift:14-25)
  DiTWeights.prepare(context)         FlashVSRDiT.prepare (DiT.swift:445-454): text-embed the prompt, cache every
                                      block's cross K/V, and the t = 1000 time constants t and t_mod
  DiTWeights.block(i)                 a fvsr_lcsa.DiTBlock over block i's tensors

Files are read with safetensors (no pickle). The GEMMs of `prepare` run on the device through fvsr_linear; the
two SiLUs of the time MLP act on one (1, C) row each.
"""
from __future__ import annotations

import math
import os
import re

import numpy as np
import torch
from safetensors.torch import load_file

from . import DiTBlock, linear
from ._abi import ERR_INVALID_ARG, FVSRError

LANES = ("bf16", "fp32")

# upstream suffix under blocks.N -> field of fvsr_dit_block_weights (DiT.swift:317-375)
BLOCK_KEYS = {
    "self_attn.q.weight": "q_weight", "self_attn.q.bias": "q_bias",
    "self_attn.k.weight": "k_weight", "self_attn.k.bias": "k_bias",
    "self_attn.v.weight": "v_weight", "self_attn.v.bias": "v_bias",
    "self_attn.o.weight": "o_weight", "self_attn.o.bias": "o_bias",
    "self_attn.norm_q.weight": "norm_q_weight", "self_attn.norm_k.weight": "norm_k_weight",
    "cross_attn.q.weight": "cross_q_weight", "cross_attn.q.bias": "cross_q_bias",
    "cross_attn.k.weight": "cross_k_weight", "cross_attn.k.bias": "cross_k_bias",
    "cross_attn.v.weight": "cross_v_weight", "cross_attn.v.bias": "cross_v_bias",
    "cross_attn.o.weight": "cross_o_weight", "cross_attn.o.bias": "cross_o_bias",
    "cross_attn.norm_q.weight": "cross_norm_q_weight", "cross_attn.norm_k.weight": "cross_norm_k_weight",
    "norm3.weight": "norm3_weight", "norm3.bias": "norm3_bias",
    "ffn.0.weight": "ffn1_weight", "ffn.0.bias": "ffn1_bias",
    "ffn.2.weight": "ffn2_weight", "ffn.2.bias": "ffn2_bias",
    "modulation": "modulation",
}

# the rest of the DiT's parameters (DiT.swift:405-431): patch embedding, text / time embeddings, head
TOP_KEYS = ("patch_embedding.weight", "patch_embedding.bias",
            "text_embedding.0.weight", "text_embedding.0.bias", "text_embedding.2.weight", "text_embedding.2.bias",
            "time_embedding.0.weight", "time_embedding.0.bias", "time_embedding.2.weight", "time_embedding.2.bias",
            "time_projection.1.weight", "time_projection.1.bias",
            "head.head.weight", "head.head.bias", "head.modulation")

_BLOCK_RE = re.compile(r"^blocks\.(\d+)\.(.+)$")


class LoadError(FVSRError):
    def __init__(self, msg: str):
        super().__init__(ERR_INVALID_ARG, "weights", msg)


def lane_file(directory: str, component: str, lane: str) -> str:
    """`<component>_<lane>.safetensors` (Weights.swift:21)."""
    return os.path.join(directory, f"{component}_{lane}.safetensors")


def pick_lane_file(directory: str, component: str, dtype: torch.dtype) -> str:
    """The lane matching the compute dtype when present, else the other one (Weights.swift:52-58)."""
    preferred = "fp32" if dtype == torch.float32 else "bf16"
    for lane in (preferred,) + tuple(x for x in LANES if x != preferred):
        p = lane_file(directory, component, lane)
        if os.path.exists(p):
            return p
    raise LoadError(f"FlashVSR weights missing: {lane_file(directory, component, preferred)}")


def expected_keys(layers: int) -> set:
    return {f"blocks.{i}.{k}" for i in range(layers) for k in BLOCK_KEYS} | set(TOP_KEYS)


def verify_keys(keys) -> int:
    """The key contract: blocks 0..N-1 with every block key, the top-level keys, nothing else. Returns N."""
    keys = set(keys)
    idx = [int(m.group(1)) for m in map(_BLOCK_RE.match, keys) if m]
    layers = max(idx) + 1 if idx else 0
    want = expected_keys(layers)
    missing, unused = sorted(want - keys), sorted(keys - want)
    if missing or unused:
        raise LoadError(f"key contract: {len(missing)} missing {missing[:5]}, {len(unused)} unused {unused[:5]}")
    return layers


def sinusoidal(dim: int, position: float) -> np.ndarray:
    """`sinusoidal_embedding_1d` (DiT.swift:435-443): [cos(p w_j) || sin(p w_j)], w_j = 10000^(-j / (dim/2)), in
    double, stored fp32."""
    half = dim // 2
    a = position * np.power(10000.0, -np.arange(half, dtype=np.float64) / half)
    return np.concatenate([np.cos(a), np.sin(a)]).astype(np.float32)[None, :]


class DiTWeights:
    """The DiT's tensors from one lane file, on the device in the compute dtype (bf16 for the HIP blocks)."""

    def __init__(self, tensors: dict, heads: int | None = None, eps: float = 1e-6):
        self.layers = verify_keys(tensors.keys())
        self.t = tensors
        c = tensors["blocks.0.self_attn.q.weight"].shape[0] if self.layers else 0
        self.dim = c
        self.heads = heads if heads is not None else c // 128
        if self.heads * 128 != c:
            raise LoadError(f"dim {c} is not heads x 128")
        self.eps = eps
        self.t_vec = self.t_mod = self.context = None
        self._blocks: dict = {}

    @classmethod
    def load(cls, directory: str, dtype: torch.dtype = torch.bfloat16, device=None, heads: int | None = None):
        path = pick_lane_file(directory, "dit", dtype)
        raw = load_file(path)   # safetensors: tensors only, nothing executed
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        return cls({k: v.to(dtype).to(dev).contiguous() for k, v in raw.items()}, heads=heads)

    @staticmethod
    def load_prompt(directory: str, dtype: torch.dtype = torch.bfloat16, device=None) -> torch.Tensor:
        """The fixed prompt context (1, 512, text_dim) (`prompt_<lane>.safetensors`, key "context"; Weights.swift:67)."""
        raw = load_file(pick_lane_file(directory, "prompt", dtype))
        if "context" not in raw:
            raise LoadError("prompt context missing")
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        return raw["context"].to(dtype).to(dev).contiguous()

    def block_tensors(self, i: int) -> dict:
        """Block i's tensors under the fvsr_dit_block_weights field names (modulation as (6, C))."""
        out = {f: self.t[f"blocks.{i}.{k}"] for k, f in BLOCK_KEYS.items()}
        out["modulation"] = out["modulation"].reshape(6, self.dim).contiguous()
        return out

    def prepare(self, context: torch.Tensor, stream=None):
        """`FlashVSRDiT.prepare` (DiT.swift:445-454): ctx = text_embedding(context) (Linear, GELU(tanh), Linear);
        every block's cross K/V from it; t = time_embedding(sinusoidal(freq_dim, 1000)) (Linear, SiLU, Linear);
        t_mod = time_projection(t) (SiLU, Linear) as (6, C)."""
        t = self.t
        ctx = context.reshape(-1, context.shape[-1]).to(torch.bfloat16).contiguous()
        h = linear(ctx, t["text_embedding.0.weight"], t["text_embedding.0.bias"], gelu=True, stream=stream)
        self.context = linear(h, t["text_embedding.2.weight"], t["text_embedding.2.bias"], stream=stream)
        dev = ctx.device
        freq_dim = t["time_embedding.0.weight"].shape[1]
        s = torch.from_numpy(sinusoidal(freq_dim, 1000.0)).to(torch.bfloat16).to(dev)
        e = linear(s, t["time_embedding.0.weight"], t["time_embedding.0.bias"], stream=stream)
        e = torch.nn.functional.silu(e.float()).to(torch.bfloat16)
        self.t_vec = linear(e, t["time_embedding.2.weight"], t["time_embedding.2.bias"], stream=stream)
        p = torch.nn.functional.silu(self.t_vec.float()).to(torch.bfloat16)
        self.t_mod = linear(p, t["time_projection.1.weight"], t["time_projection.1.bias"],
                            stream=stream).reshape(6, self.dim)
        self._blocks = {}
        return self

    def block(self, i: int) -> DiTBlock:
        """Block i as a DiTBlock with its cross K/V cached from the prepared context."""
        if i not in self._blocks:
            b = DiTBlock(self.block_tensors(i), self.heads, self.eps)
            if self.context is None:
                raise LoadError("prepare(context) first: the cross-attention K/V come from the prompt")
            b.set_context(self.context)
            self._blocks[i] = b
        return self._blocks[i]
