"""Seeded synthetic Q/K/V for the LCSA workloads (random data of the real shapes; no checkpoint is involved).

Shapes follow the reference's geometry: an output of H x W pixels has (H/16) x (W/16) latent tokens per frame (VAE /8,
patch (1, 2, 2): DiT.swift:422-423,560-562); LCSA windows are (2, 8, 8) = 128 tokens, so one temporal slice of two
latent frames holds s = (H/128) x (W/128) blocks (DiT.swift:111-118,480).

Per-token processing mirrors what produces q/k in `blockForward` (DiT.swift:499-502):
  rms_norm   per-head RMS normalisation (eps 1e-6) or the reference's full-width WanRMSNorm (DiT.swift:34-47)
  rope_apply the 3-D RoPE of `RopeTables` / `ropeApply` (DiT.swift:56-107): head split 44 | 42 | 42 (complex pairs
             22 | 21 | 21), theta 10000, each axis normalised by its own sub-dimension, angles built in float64,
             rotation applied in float32 to (even, odd) pairs.
Tokens are generated in natural (f, h, w) order and then window-partitioned (DiT.swift:113-118).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

HEAD_DIM = 128
BLOCK = 128


@dataclass(frozen=True)
class Workload:
    name: str
    height: int                 # output pixels
    width: int
    q_frames: int               # latent frames of queries
    k_frames: int               # latent frames of keys/values (cache + new); may be odd (ragged, see k_tokens)
    dtype: torch.dtype
    local_range: int
    kept_fraction: float        # of the in-window (query block, key block) pairs per (head, query slice)
    heads: int = 12
    rope: bool = False
    smooth: bool = False        # low-frequency field + noise: pooled scores with distinct margins
    full_mask: bool = False     # every block kept (sparse == dense)
    q_t0: int = 0               # temporal RoPE position of the first query frame
    seed: int = 0               # default generator seed
    noise: float = 0.35         # noise std of the smooth workloads (per element, before the RMS norm)
    description: str = ""

    @property
    def lat_h(self) -> int:
        return self.height // 16

    @property
    def lat_w(self) -> int:
        return self.width // 16

    @property
    def bh(self) -> int:
        return self.lat_h // 8

    @property
    def bw(self) -> int:
        return self.lat_w // 8

    @property
    def s(self) -> int:
        return self.bh * self.bw

    @property
    def tokens_per_frame(self) -> int:
        return self.lat_h * self.lat_w

    @property
    def lq(self) -> int:
        return self.q_frames * self.tokens_per_frame

    @property
    def lk(self) -> int:
        return self.k_frames * self.tokens_per_frame

    @property
    def nq(self) -> int:
        return -(-self.lq // BLOCK)

    @property
    def nk(self) -> int:
        return -(-self.lk // BLOCK)

    @property
    def q_slices(self) -> int:
        return self.q_frames // 2

    @property
    def channels(self) -> int:
        return self.heads * HEAD_DIM


WORKLOADS = {
    "lcsa_512x512_fp32": Workload(
        "lcsa_512x512_fp32", 512, 512, q_frames=2, k_frames=6, dtype=torch.float32, local_range=3,
        kept_fraction=0.5, q_t0=4,
        description="512x512, fp32: Lq 2048 (Q 2 latent frames), Lk 6144 (6 frames incl. cache), 12x128 heads, "
                    "N(0,1) then per-head RMS norm, local range 3, top-k = 50% of in-window pairs"),
    "dense_1280x768_bf16": Workload(
        "dense_1280x768_bf16", 768, 1280, q_frames=2, k_frames=5, dtype=torch.bfloat16, local_range=11,
        kept_fraction=1.0, full_mask=True, q_t0=3,
        description="1280x768, bf16: Lq 7680, Lk 19200 (5 frames), all blocks kept (sparse == dense)"),
    "sparse_1280x768_bf16": Workload(
        "sparse_1280x768_bf16", 768, 1280, q_frames=2, k_frames=5, dtype=torch.bfloat16, local_range=3,
        kept_fraction=0.6, smooth=True, q_t0=3, seed=1,
        description="1280x768, bf16: Lq 7680, Lk 19200, local range 3, 60% of in-window kept, smooth Q/K + noise; "
                    "seed 1 puts every top-k threshold 2.2e-3 (relative) below its upper neighbour"),
    "sparse_1920x1152_bf16": Workload(
        "sparse_1920x1152_bf16", 1152, 1920, q_frames=2, k_frames=5, dtype=torch.bfloat16, local_range=11,
        kept_fraction=0.3, rope=True, smooth=True, noise=1.0, q_t0=3, seed=0,
        description="1920x1152, bf16: Lq 17280, Lk 43200 (337.5 key blocks, ragged tail), local range 11, "
                    "30% of in-window kept, smooth Q/K field + N(0,1) noise, per-head RMS norm + 3-D RoPE; seed 0 "
                    "puts every top-k threshold 8.7e-5 (relative) below its upper neighbour"),
    "sparse_1920x1152_bf16_iid": Workload(
        "sparse_1920x1152_bf16_iid", 1152, 1920, q_frames=2, k_frames=5, dtype=torch.bfloat16, local_range=11,
        kept_fraction=0.3, rope=True, q_t0=3,
        description="1920x1152, bf16: as sparse_1920x1152_bf16 with i.i.d. N(0,1) Q/K (pooled blocks carry no "
                    "signal: the mask follows the window sizes and 960 of 1620 rows select nothing)"),
}


# ----------------------------------------------------------------------------------------------------------------
# token processing
# ----------------------------------------------------------------------------------------------------------------
def rms_norm(x: torch.Tensor, heads: int, per_head: bool = True, eps: float = 1e-6) -> torch.Tensor:
    """fp32 RMS normalisation, per head or over the full width (WanRMSNorm with unit weight, DiT.swift:42-46)."""
    xf = x.float()
    if per_head:
        xh = xf.reshape(*xf.shape[:-1], heads, -1)
        return (xh * torch.rsqrt(xh.pow(2).mean(-1, keepdim=True) + eps)).reshape(xf.shape)
    return xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)


def rope_tables(head_dim: int = HEAD_DIM, end: int = 1024, theta: float = 10000.0):
    """(cos, sin) per axis: lists of three float64 tensors (end, n_axis) for t, h, w (RopeTables.init)."""
    d_t = head_dim - 2 * (head_dim // 3)
    d_hw = head_dim // 3
    out = []
    for dim in (d_t, d_hw, d_hw):
        n = dim // 2
        j = torch.arange(n, dtype=torch.float64)
        freq = 1.0 / torch.pow(torch.tensor(theta, dtype=torch.float64), 2 * j / dim)
        ang = torch.arange(end, dtype=torch.float64)[:, None] * freq[None, :]
        out.append((torch.cos(ang), torch.sin(ang)))
    return out


def rope_grid(f: int, h: int, w: int, t0: int, device=None):
    """(cos, sin) fp32 of shape (f*h*w, 64) for an (f, h, w) token grid starting at temporal position t0
    (RopeTables.grid, DiT.swift:81-97)."""
    (ct, st), (ch, sh), (cw, sw) = rope_tables()
    tt = torch.arange(t0, t0 + f)
    yy = torch.arange(h)
    xx = torch.arange(w)
    T, Y, X = torch.meshgrid(tt, yy, xx, indexing="ij")
    T, Y, X = T.reshape(-1), Y.reshape(-1), X.reshape(-1)
    cos = torch.cat([ct[T], ch[Y], cw[X]], dim=1).float()
    sin = torch.cat([st[T], sh[Y], sw[X]], dim=1).float()
    return cos.to(device), sin.to(device)


def rope_apply(x: torch.Tensor, heads: int, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate (even, odd) pairs per head by e^{i theta} (ropeApply, DiT.swift:101-107). x: (L, H*D)."""
    L, c = x.shape
    xf = x.float().reshape(L, heads, c // heads // 2, 2)
    re, im = xf[..., 0], xf[..., 1]
    cs, sn = cos[:, None, :], sin[:, None, :]
    return torch.stack([re * cs - im * sn, re * sn + im * cs], dim=-1).reshape(L, c)


def window_partition(x: torch.Tensor, f: int, h: int, w: int) -> torch.Tensor:
    """(f*h*w, C) -> (f*h*w, C) in window order (DiT.swift:113-118)."""
    c = x.shape[-1]
    y = x.reshape(f // 2, 2, h // 8, 8, w // 8, 8, c).permute(0, 2, 4, 1, 3, 5, 6)
    return y.reshape(-1, c).contiguous()


def smooth_field(f: int, h: int, w: int, channels: int, gen: torch.Generator, modes: int = 6) -> torch.Tensor:
    """A low-frequency random field over (t, y, x): sum of `modes` random-phase plane waves with per-channel
    amplitudes, (f*h*w, channels) fp32."""
    T, Y, X = torch.meshgrid(torch.arange(f, dtype=torch.float32) / max(f, 1),
                             torch.arange(h, dtype=torch.float32) / h,
                             torch.arange(w, dtype=torch.float32) / w, indexing="ij")
    pos = torch.stack([T.reshape(-1), Y.reshape(-1), X.reshape(-1)], dim=1)           # (L, 3)
    freqs = torch.randint(-2, 3, (modes, 3), generator=gen).float()                   # cycles over the grid
    freqs[freqs.abs().sum(1) == 0, 1] = 1.0
    phase = torch.rand(modes, channels, generator=gen) * 2 * math.pi
    amp = torch.randn(modes, channels, generator=gen)
    arg = 2 * math.pi * (pos @ freqs.T)                                               # (L, modes)
    out = torch.zeros((pos.shape[0], channels))
    for m in range(modes):
        out += torch.cos(arg[:, m:m + 1] + phase[m][None, :]) * amp[m][None, :]
    return out


# ----------------------------------------------------------------------------------------------------------------
# workloads
# ----------------------------------------------------------------------------------------------------------------
def make_qkv(wl: Workload, seed: int | None = None, device="cpu", noise: float | None = None):
    """Seeded (q, k, v) for a workload: q (Lq, C), k/v (Lk, C) in window order, `wl.dtype`, on `device`.
    `seed` and `noise` default to the workload's own.

    Generation happens on the CPU with a torch.Generator (deterministic across machines) in float32, then the
    tensors are cast and moved."""
    seed = wl.seed if seed is None else seed
    noise = wl.noise if noise is None else noise
    gen = torch.Generator().manual_seed(seed)
    c, H = wl.channels, wl.heads
    h, w = wl.lat_h, wl.lat_w
    kf_gen = wl.k_frames + (wl.k_frames % 2)           # whole slices, truncated to k_frames worth of tokens
    qf = wl.q_frames
    if wl.smooth:
        fk = smooth_field(kf_gen, h, w, c, gen)
        # queries see the newest frames of the same field
        fq = fk.reshape(kf_gen, h * w, c)[kf_gen - qf:].reshape(-1, c)
        k = fk + noise * torch.randn(fk.shape, generator=gen)
        q = fq + noise * torch.randn(fq.shape, generator=gen)
    else:
        q = torch.randn((qf * h * w, c), generator=gen)
        k = torch.randn((kf_gen * h * w, c), generator=gen)
    v = torch.randn((kf_gen * h * w, c), generator=gen)
    q = rms_norm(q, H)
    k = rms_norm(k, H)
    if wl.rope:
        cq, sq = rope_grid(qf, h, w, wl.q_t0)
        ck, sk = rope_grid(kf_gen, h, w, 0)
        q = rope_apply(q, H, cq, sq)
        k = rope_apply(k, H, ck, sk)
    q = window_partition(q, qf, h, w)
    k = window_partition(k, kf_gen, h, w)[: wl.lk]
    v = window_partition(v, kf_gen, h, w)[: wl.lk]
    return (q.to(wl.dtype).to(device).contiguous(), k.to(wl.dtype).to(device).contiguous(),
            v.to(wl.dtype).to(device).contiguous())


def local_mask(wl: Workload) -> torch.Tensor:
    """(s, s) bool local window of the workload (localBlockMask semantics, DiT.swift:130-145)."""
    half = wl.local_range // 2
    r = wl.local_range
    qr = torch.arange(wl.bh)[:, None, None, None]
    qc = torch.arange(wl.bw)[None, :, None, None]
    kr = torch.arange(wl.bh)[None, None, :, None]
    kc = torch.arange(wl.bw)[None, None, None, :]
    m = (kr >= qr - half) & (kr <= qr - half + r - 1) & (kc >= qc - half) & (kc <= qc - half + r - 1)
    return m.reshape(wl.s, wl.s)


def in_window_pairs(wl: Workload) -> int:
    lm = local_mask(wl)
    return int(lm[:, torch.arange(wl.nk) % wl.s].sum())


def workload_topk(wl: Workload) -> int:
    """Explicit top-k count keeping `kept_fraction` of the in-window pairs of one (head, query slice) row."""
    return int(math.floor(wl.kept_fraction * in_window_pairs(wl)))


def step_topk(s: int, topk_ratio: float) -> int:
    """topk = Int(s^2 * ratio) - 1 (DiT.swift:482)."""
    return int(float(s * s) * topk_ratio) - 1


def default_topk_ratio(height: int, width: int) -> float:
    """2*768*1280 / (H*W) (Pipeline.swift:68)."""
    return 2.0 * 768 * 1280 / float(height * width)


def kept_flops(kcnt: torch.Tensor, kidx: torch.Tensor, lq: int, lk: int) -> float:
    """Kept-block FLOPs: 4 * 128 * sum over kept (head, q-block, k-block) of valid q tokens x valid k tokens."""
    kc = kcnt.to(torch.int64).cpu()
    ki = kidx.to(torch.int64).cpu()
    H, nq = kc.shape
    q_valid = torch.full((nq,), BLOCK, dtype=torch.int64)
    q_valid[-1] = lq - (nq - 1) * BLOCK
    last = (lk - 1) // BLOCK
    k_short = BLOCK - (lk - last * BLOCK)                   # missing keys of the last (ragged) block
    listed = torch.arange(ki.shape[-1])[None, None, :] < kc[:, :, None]
    has_last = ((ki == last) & listed).any(-1).to(torch.int64)
    keys = kc * BLOCK - k_short * has_last                  # valid keys per (head, q-block)
    return 4.0 * HEAD_DIM * float((keys * q_valid[None, :]).sum())
