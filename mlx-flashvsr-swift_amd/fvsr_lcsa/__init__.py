"""Python host binding of libfvsr_lcsa (the MI355X LCSA path) over torch device tensors.

Names mirror the reference's call surface (xocialize/mlx-flashvsr-swift):
  local_block_mask            localBlockMask(bh:bw:range:)                    DiT.swift:130-145
  draft_block_mask_and_probs  draftBlockMaskAndProbs(qW:kW:heads:qSlices:...)  DiT.swift:158-174
  draft_block_mask            draftBlockMask(...)                              DiT.swift:150-154
  kernel_block_attention      kernelBlockAttention(q:k:v:blockMask:heads:)     SparseAttention.swift:169-187
  block_masked_attention      blockMaskedAttention(q:k:v:blockMask:heads:)     DiT.swift:279-313 (dense fallback)
  FlashVSRAttentionOps        FlashVSRAttentionOps.dense / .kernel             SparseAttention.swift:190-202
  KVRing                      the window K/V cache of blockForward             DiT.swift:507-511,532-538
  window_partition / reverse  windowPartition / windowReverse                  DiT.swift:113-126
  rope_tables                 RopeTables(headDim: 128)                          DiT.swift:52-97
  qkv_epilogue                normQ/normK + ropeApply + windowPartition          DiT.swift:34-47,100-118,496-506
  linear                      Linear (+ GELU tanh) on hipBLASLt                  DiT.swift:319-321,371
  DiTBlock                    DiTBlock + blockForward (streaming)               DiT.swift:363-375,491-551
Token tensors are (L, H*128) or (1, L, H*128), window order, float32 or bfloat16, on a HIP device, contiguous.
Every call runs the HIP kernels of libfvsr_lcsa.so; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _abi
from ._abi import (ATTN_AUTO, ATTN_DENSE, ATTN_KERNEL, DTYPE_BF16, DTYPE_F32, LAYOUT_GRID, LAYOUT_WINDOWS,
                   FVSRError, call, lib)

__all__ = ["FVSRError", "Context", "local_block_mask", "draft_block_mask_and_probs", "draft_block_mask",
           "kernel_block_attention", "block_masked_attention", "block_sparse_attention", "FlashVSRAttentionOps",
           "KVRing", "window_partition", "window_reverse", "attention_mode_auto", "workspace_size",
           "rope_tables", "rope_tables_device", "qkv_epilogue", "linear", "DiTBlock",
           "ATTN_AUTO", "ATTN_DENSE", "ATTN_KERNEL", "LAYOUT_GRID", "LAYOUT_WINDOWS", "lib"]

HEAD_DIM = 128
BLOCK = 128


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise FVSRError(_abi.ERR_INVALID_ARG, "dtype", f"unsupported dtype {t.dtype} (float32 or bfloat16)")


def _tokens(x: torch.Tensor, name: str) -> torch.Tensor:
    """(L, C) view of a token operand (2-D, or 3-D with batch 1), contiguous. Metadata only: where the operands live
    is checked by _devices right before the library call, after every shape check."""
    if x is None:
        raise FVSRError(_abi.ERR_INVALID_ARG, name, "is None")
    if x.dim() == 3:
        if x.shape[0] != 1:
            raise FVSRError(_abi.ERR_UNSUPPORTED, name, "batch 1 only (the reference asserts the same)")
        x = x[0]
    if x.dim() != 2 or not x.is_contiguous():
        raise FVSRError(_abi.ERR_INVALID_ARG, name, f"expected contiguous (L, C) tokens, got {tuple(x.shape)}")
    return x


def _devices(*named) -> torch.device:
    """Every (tensor, name) operand on the HIP device of the first one, contiguous; None entries are skipped. Runs
    before any pointer reaches the library: a host tensor's address handed to a kernel would fault the GPU."""
    first, fname = named[0]
    if not first.is_cuda:
        raise FVSRError(_abi.ERR_INVALID_ARG, fname, f"expected a tensor on a HIP device, got {first.device}")
    for t, n in named:
        if t is not None:
            _on_device(t, n, first.device)
    return first.device


def _ptr(t) -> C.c_void_p:
    return C.c_void_p(0 if t is None else t.data_ptr())


def _on_device(t: torch.Tensor, name: str, device: torch.device, numel: int | None = None) -> torch.Tensor:
    """A caller-supplied operand the kernels read through a raw pointer: it must live on the tokens' device, be
    contiguous and, where the library derives its extent from other arguments, hold exactly `numel` elements (the
    C ABI cannot check a buffer's size, and a short one would be read past its end)."""
    if not t.is_cuda or t.device != device:
        raise FVSRError(_abi.ERR_INVALID_ARG, name, f"expected a tensor on {device}, got {t.device}")
    if not t.is_contiguous():
        raise FVSRError(_abi.ERR_INVALID_ARG, name, "expected a contiguous tensor")
    if numel is not None and t.numel() != numel:
        raise FVSRError(_abi.ERR_INVALID_ARG, name, f"expected {numel} elements, got {t.numel()} (shape {tuple(t.shape)})")
    return t


def _shaped(t: torch.Tensor, name: str, shape: tuple, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Metadata checks of an operand whose extent the library derives from other arguments: exact shape, then
    dtype. They run before any device check, so a wrong operand is named even for host tensors."""
    if t is None:
        raise FVSRError(_abi.ERR_INVALID_ARG, name, "is None")
    if tuple(t.shape) != tuple(shape):
        raise FVSRError(_abi.ERR_INVALID_ARG, name, f"expected shape {tuple(shape)}, got {tuple(t.shape)}")
    if dtype is not None and t.dtype != dtype:
        raise FVSRError(_abi.ERR_INVALID_ARG, name, f"expected dtype {dtype}, got {t.dtype}")
    return t


def _heads_width(x: torch.Tensor, name: str, heads: int) -> None:
    if x.dim() != 2 or x.shape[1] != heads * HEAD_DIM:
        raise FVSRError(_abi.ERR_INVALID_ARG, name,
                        f"expected (L, {heads * HEAD_DIM}) tokens for {heads} heads of {HEAD_DIM}, got {tuple(x.shape)}")


def _stream(stream) -> C.c_void_p:
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream))


class Context:
    """One fvsr_ctx per device (workspace + device binding). Not re-entrant, like the reference's modules."""
    _by_device: dict[int, "Context"] = {}

    def __init__(self, device: int = 0):
        self.device = device
        h = C.c_void_p()
        call("fvsr_ctx_create", device, C.byref(h))
        self.handle = h
        self._local_cache: dict[tuple, torch.Tensor] = {}

    @classmethod
    def get(cls, device: int | torch.device | None = None) -> "Context":
        if device is None:
            device = torch.cuda.current_device()
        if isinstance(device, torch.device):
            device = device.index if device.index is not None else torch.cuda.current_device()
        if device not in cls._by_device:
            cls._by_device[device] = Context(device)
        return cls._by_device[device]

    def reserve(self, nbytes: int):
        call("fvsr_ctx_reserve", self.handle, nbytes)

    def workspace_bytes(self) -> int:
        return int(lib.fvsr_ctx_workspace_bytes(self.handle))

    def reserve_block(self, heads: int, tokens: int, ffn_dim: int, ctx_len: int, key_tokens: int):
        """Size everything a DiT block call of up to `tokens` tokens over a ring window of up to `key_tokens` keys
        needs (hipBLASLt state, block and select/attention workspaces), so later block calls allocate nothing."""
        call("fvsr_ctx_reserve_block", self.handle, heads, tokens, ffn_dim, ctx_len, key_tokens)

    def block_workspace_bytes(self) -> int:
        return int(lib.fvsr_ctx_block_workspace_bytes(self.handle))

    def local_device(self, local, s: int) -> torch.Tensor:
        """Device copy of an (s, s) local window mask, memoised by content (the reference memoises per geometry,
        DiT.swift:464-470). The library reads s * s bytes from it."""
        if isinstance(local, torch.Tensor) and local.is_cuda:
            if local.numel() != s * s:
                raise FVSRError(_abi.ERR_INVALID_ARG, "local", f"expected an ({s}, {s}) mask, got {tuple(local.shape)}")
            return _on_device(local.to(torch.uint8).contiguous(), "local", torch.device(f"cuda:{self.device}"))
        arr = np.ascontiguousarray(np.asarray(local, dtype=np.uint8))
        if arr.size != s * s:
            raise FVSRError(_abi.ERR_INVALID_ARG, "local", f"expected an ({s}, {s}) mask, got {arr.shape}")
        key = (arr.shape, arr.tobytes())
        t = self._local_cache.get(key)
        if t is None:
            t = torch.from_numpy(arr.copy()).to(f"cuda:{self.device}")
            self._local_cache[key] = t
        return t

    def __del__(self):
        try:
            lib.fvsr_ctx_destroy(self.handle)
        except Exception:
            pass


# ------------------------------------------------------------------------------------------------------------------
# host helpers
# ------------------------------------------------------------------------------------------------------------------
def local_block_mask(bh: int, bw: int, r: int) -> np.ndarray:
    """(s, s) bool local window (host). localBlockMask, DiT.swift:130-145."""
    s = bh * bw
    out = np.zeros((s, s), dtype=np.uint8)
    call("fvsr_local_block_mask", bh, bw, r, out.ctypes.data_as(C.c_void_p))
    return out.astype(bool)


def attention_mode_auto(topk: int, s: int, nk: int, threshold: float = 0.45):
    """(expected kept fraction, ATTN_KERNEL | ATTN_DENSE): the `auto` rule of DiT.swift:517-522."""
    e = C.c_double()
    m = C.c_int()
    call("fvsr_attention_mode_auto", topk, s, nk, threshold, C.byref(e), C.byref(m))
    return e.value, m.value


def workspace_size(heads: int, lq: int, lk: int, channels: int) -> int:
    return int(lib.fvsr_workspace_size(heads, lq, lk, channels))


# ------------------------------------------------------------------------------------------------------------------
# selection
# ------------------------------------------------------------------------------------------------------------------
def draft_block_mask_and_probs(qW: torch.Tensor, kW: torch.Tensor, heads: int, q_slices: int, s: int, local,
                               topk: int, stream=None, want_mask: bool = True, want_probs: bool = True):
    """Returns (mask (H, Nq, Nk) f32 0/1 or None, probs (H, Nq, Nk) f32 or None, kidx (H, Nq, Nk) i32,
    kcnt (H, Nq) i32). DiT.swift:158-174 + SparseAttention.swift:175-177."""
    q = _tokens(qW.reshape(-1, qW.shape[-1]) if qW.dim() == 3 and qW.shape[0] != 1 else qW, "qW")
    k = _tokens(kW.reshape(-1, kW.shape[-1]) if kW.dim() == 3 and kW.shape[0] != 1 else kW, "kW")
    _heads_width(q, "qW", heads)
    _heads_width(k, "kW", heads)
    if q.dtype != k.dtype:
        raise FVSRError(_abi.ERR_INVALID_ARG, "kW", f"dtype {k.dtype} differs from qW's {q.dtype}")
    _devices((q, "qW"), (k, "kW"))
    ctx = Context.get(q.device)
    nq = -(-q.shape[0] // BLOCK)
    nk = -(-k.shape[0] // BLOCK)
    dev = q.device
    mask = torch.empty((heads, nq, nk), dtype=torch.float32, device=dev) if want_mask else None
    probs = torch.empty((heads, nq, nk), dtype=torch.float32, device=dev) if want_probs else None
    kidx = torch.empty((heads, nq, nk), dtype=torch.int32, device=dev)
    kcnt = torch.empty((heads, nq), dtype=torch.int32, device=dev)
    loc = ctx.local_device(local, s)
    call("fvsr_lcsa_select", ctx.handle, _dtype_code(q), _ptr(q), q.shape[0], _ptr(k), k.shape[0], heads, q_slices,
         s, _ptr(loc), topk, _ptr(mask), _ptr(probs), _ptr(kidx), _ptr(kcnt), _stream(stream))
    return mask, probs, kidx, kcnt


def draft_block_mask(qW, kW, heads, q_slices, s, local, topk, stream=None) -> torch.Tensor:
    return draft_block_mask_and_probs(qW, kW, heads, q_slices, s, local, topk, stream, want_probs=False)[0]


# ------------------------------------------------------------------------------------------------------------------
# attention
# ------------------------------------------------------------------------------------------------------------------
def _attn_mask(q, k, v, block_mask, heads, mode, stream, out):
    shape = q.shape
    q2, k2, v2 = _qkv_operands(q, k, v, heads)
    nq, nk = -(-q2.shape[0] // 128), -(-k2.shape[0] // 128)
    if block_mask.numel() != heads * nq * nk:
        raise FVSRError(_abi.ERR_INVALID_ARG, "block_mask",
                        f"expected {heads * nq * nk} elements ({heads}, {nq}, {nk}), got {tuple(block_mask.shape)}")
    o = _out_meta(out, q2)
    _devices((q2, "q"), (k2, "k"), (v2, "v"), (block_mask, "block_mask"), (o, "out"))
    bm = block_mask.to(torch.float32).contiguous()
    o = torch.empty_like(q2) if o is None else o
    ctx = Context.get(q2.device)
    call("fvsr_lcsa_attention_mask", ctx.handle, _dtype_code(q2), _ptr(q2), q2.shape[0], _ptr(k2), _ptr(v2),
         k2.shape[0], heads, _ptr(bm), mode, _ptr(o), _stream(stream))
    return o.reshape(shape)


def _qkv_operands(q, k, v, heads):
    """(q, k, v) token operands of an attention call: 2-D, heads * 128 wide, one dtype, K and V of one shape."""
    q2, k2, v2 = _tokens(q, "q"), _tokens(k, "k"), _tokens(v, "v")
    for t, n in ((q2, "q"), (k2, "k"), (v2, "v")):
        _heads_width(t, n, heads)
    if not (q2.dtype == k2.dtype == v2.dtype):
        raise FVSRError(_abi.ERR_INVALID_ARG, "attention", "q, k, v dtypes differ")
    if k2.shape != v2.shape:
        raise FVSRError(_abi.ERR_INVALID_ARG, "v", f"expected the shape of k {tuple(k2.shape)}, got {tuple(v2.shape)}")
    return q2, k2, v2


def _out_meta(out, ref: torch.Tensor, name: str = "out"):
    """A caller-supplied output (or None): the shape and dtype of `ref` (a batch-1 3-D view allowed), contiguous."""
    if out is None:
        return None
    o = out[0] if out.dim() == 3 and out.shape[0] == 1 else out
    _shaped(o, name, tuple(ref.shape), ref.dtype)
    if not o.is_contiguous():
        raise FVSRError(_abi.ERR_INVALID_ARG, name, "expected a contiguous tensor")
    return o


def _lists_meta(kidx, kcnt, heads: int, nq: int):
    """kidx (heads, nq, stride >= 1) and kcnt (heads, nq) of an integer type (int32 is what the library reads)."""
    if kidx.dim() != 3 or tuple(kidx.shape[:2]) != (heads, nq) or kidx.shape[2] < 1:
        raise FVSRError(_abi.ERR_INVALID_ARG, "kidx", f"expected ({heads}, {nq}, stride) lists, got {tuple(kidx.shape)}")
    _shaped(kcnt, "kcnt", (heads, nq))
    for t, n in ((kidx, "kidx"), (kcnt, "kcnt")):
        if t.dtype.is_floating_point or t.dtype.is_complex or t.dtype == torch.bool:
            raise FVSRError(_abi.ERR_INVALID_ARG, n, f"expected an integer tensor, got {t.dtype}")


def kernel_block_attention(q, k, v, block_mask, heads: int, stream=None, out=None) -> torch.Tensor:
    """Block-sparse kernel: visits only the selected key blocks. SparseAttention.swift:169-187."""
    return _attn_mask(q, k, v, block_mask, heads, ATTN_KERNEL, stream, out)


def block_masked_attention(q, k, v, block_mask, heads: int, stream=None, out=None) -> torch.Tensor:
    """Dense fallback: the same kernel walks every key block, unselected ones masked. DiT.swift:279-313."""
    return _attn_mask(q, k, v, block_mask, heads, ATTN_DENSE, stream, out)


def block_sparse_attention(q, k, v, kidx, kcnt, heads: int, stream=None, out=None) -> torch.Tensor:
    """Attention from (kidx, kcnt) lists: the Metal launch ABI of SparseAttention.swift:180-185."""
    shape = q.shape
    q2, k2, v2 = _qkv_operands(q, k, v, heads)
    nq = -(-q2.shape[0] // 128)
    _lists_meta(kidx, kcnt, heads, nq)
    o = _out_meta(out, q2)
    _devices((q2, "q"), (k2, "k"), (v2, "v"), (kidx, "kidx"), (kcnt, "kcnt"), (o, "out"))
    kidx, kcnt = kidx.to(torch.int32).contiguous(), kcnt.to(torch.int32).contiguous()
    o = torch.empty_like(q2) if o is None else o
    ctx = Context.get(q2.device)
    call("fvsr_lcsa_attention", ctx.handle, _dtype_code(q2), _ptr(q2), q2.shape[0], _ptr(k2), _ptr(v2), k2.shape[0],
         heads, _ptr(kidx), _ptr(kcnt), kidx.shape[-1], _ptr(o), _stream(stream))
    return o.reshape(shape)


class FlashVSRAttentionOps:
    """Public probe entry points (SparseAttention.swift:190-202). `gathered` is not built (study-only upstream)."""

    @staticmethod
    def dense(q, k, v, block_mask, heads: int, stream=None):
        return block_masked_attention(q, k, v, block_mask, heads, stream)

    @staticmethod
    def kernel(q, k, v, block_mask, heads: int, stream=None):
        return kernel_block_attention(q, k, v, block_mask, heads, stream)


# ------------------------------------------------------------------------------------------------------------------
# layout
# ------------------------------------------------------------------------------------------------------------------
def _layout(x, f, h, w, to_windows, stream):
    shape = x.shape
    x2 = _tokens(x, "x")
    _devices((x2, "x"))
    out = torch.empty_like(x2)
    name = "fvsr_window_partition" if to_windows else "fvsr_window_reverse"
    call(name, _dtype_code(x2), _ptr(x2), _ptr(out), f, h, w, x2.shape[1], _stream(stream))
    return out.reshape(shape)


def window_partition(x, f: int, h: int, w: int, stream=None):
    """(F*H*W, C) natural order -> window order (as a flat (L, C) token tensor). DiT.swift:113-118."""
    return _layout(x, f, h, w, True, stream)


def window_reverse(x, f: int, h: int, w: int, stream=None):
    """Window order -> natural (F*H*W, C) order. DiT.swift:121-126."""
    return _layout(x, f, h, w, False, stream)


# ------------------------------------------------------------------------------------------------------------------
# fused QKV epilogue
# ------------------------------------------------------------------------------------------------------------------
def rope_tables(theta: float = 10000.0) -> np.ndarray:
    """RoPE tables of RopeTables(headDim: 128, theta:) (DiT.swift:52-97), host fp32: cos_t, sin_t (1024 x 22),
    cos_h, sin_h, cos_w, sin_w (1024 x 21 each), concatenated. Computed by the library (fvsr_rope_tables)."""
    n = int(lib.fvsr_rope_tables_size())
    out = np.empty(n, dtype=np.float32)
    call("fvsr_rope_tables", float(theta), out.ctypes.data_as(C.c_void_p), n)
    return out


_rope_dev: dict[tuple, torch.Tensor] = {}


def rope_tables_device(device, theta: float = 10000.0) -> torch.Tensor:
    """Device copy of rope_tables(theta), uploaded once per (device, theta)."""
    dev = torch.device(device)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), float(theta))
    t = _rope_dev.get(key)
    if t is None:
        t = torch.from_numpy(rope_tables(theta)).to(f"cuda:{key[0]}")
        _rope_dev[key] = t
    return t


def _norm_weights(wq, wk, c: int, dtype):
    """The two WanRMSNorm weights: C elements each, in the tokens' dtype."""
    out = []
    for t, n in ((wq, "norm_q_weight"), (wk, "norm_k_weight")):
        if t is None or t.numel() != c:
            raise FVSRError(_abi.ERR_INVALID_ARG, n, f"expected {c} elements, got "
                            f"{None if t is None else tuple(t.shape)}")
        out.append(t.to(dtype).contiguous())
    return out


def qkv_epilogue(q, k, v, f: int, h: int, w: int, heads: int, t0: int, norm_q_weight, norm_k_weight,
                 eps: float = 1e-6, theta: float = 10000.0, stream=None):
    """(q', k', v) in window order from the projections q, k, v ((f*h*w, heads*128), natural token order):
    normQ/normK (WanRMSNorm over the full width) + ropeApply at temporal positions t0.. + windowPartition
    (DiT.swift:34-47,100-118,496-506). Returns (q_out, k_out, v_out)."""
    q2, k2, v2 = _tokens(q, "q"), _tokens(k, "k"), _tokens(v, "v")
    c = heads * HEAD_DIM
    for t, n in ((q2, "q"), (k2, "k"), (v2, "v")):
        _shaped(t, n, (f * h * w, c), q2.dtype)
    wq, wk = _norm_weights(norm_q_weight, norm_k_weight, c, q2.dtype)
    _devices((q2, "q"), (k2, "k"), (v2, "v"), (wq, "norm_q_weight"), (wk, "norm_k_weight"))
    ctx = Context.get(q2.device)
    tab = rope_tables_device(q2.device, theta)
    qo, ko, vo = torch.empty_like(q2), torch.empty_like(k2), torch.empty_like(v2)
    call("fvsr_qkv_epilogue", ctx.handle, _dtype_code(q2), _ptr(q2), _ptr(k2), _ptr(v2), f, h, w, heads, t0,
         _ptr(wq), _ptr(wk), float(eps), _ptr(tab), _ptr(qo), _ptr(ko), _ptr(vo), _stream(stream))
    return qo, ko, vo


# ------------------------------------------------------------------------------------------------------------------
# KV ring
# ------------------------------------------------------------------------------------------------------------------
class KVRing:
    """Streaming window K/V cache for `layers` DiT blocks (DiT.swift:507-511,532-538; Pipeline.swift:87-91)."""

    def __init__(self, layers: int, heads: int, bh: int, bw: int, capacity: int = 4, kv_len: int = 3,
                 dtype: torch.dtype = torch.bfloat16, device: int | None = None):
        self.ctx = Context.get(device)
        self.layers, self.heads, self.bh, self.bw = layers, heads, bh, bw
        self.s = bh * bw
        self.capacity, self.kv_len = capacity, kv_len
        self.dtype = dtype
        self.channels = heads * HEAD_DIM
        self.code = DTYPE_BF16 if dtype == torch.bfloat16 else DTYPE_F32
        h = C.c_void_p()
        call("fvsr_kv_ring_create", self.ctx.handle, self.code, layers, heads, bh, bw, capacity, kv_len, C.byref(h))
        self.handle = h

    def close(self):
        if self.handle:
            lib.fvsr_kv_ring_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        call("fvsr_kv_ring_reset", self.handle)

    def _chunk(self, x, name: str, n_slices: int) -> torch.Tensor:
        """A chunk's token operand: (n_slices * s * 128, C) in the ring's dtype (metadata only)."""
        x2 = _tokens(x, name)
        return _shaped(x2, name, (n_slices * self.s * BLOCK, self.channels), self.dtype)

    def _queries(self, x, name: str) -> torch.Tensor:
        """Queries against this ring: (L, C) in the ring's dtype (the library checks L against the slices)."""
        x2 = _tokens(x, name)
        if x2.shape[1] != self.channels or x2.dtype != self.dtype:
            raise FVSRError(_abi.ERR_INVALID_ARG, name, f"expected (L, {self.channels}) {self.dtype} tokens, got "
                            f"{tuple(x2.shape)} {x2.dtype}")
        return x2

    def append(self, layer: int, k_new, v_new, n_slices: int, layout: int = LAYOUT_WINDOWS, stream=None):
        k2, v2 = self._chunk(k_new, "k_new", n_slices), self._chunk(v_new, "v_new", n_slices)
        _devices((k2, "k_new"), (v2, "v_new"))
        call("fvsr_kv_ring_append", self.handle, layer, _ptr(k2), _ptr(v2), n_slices, layout, _stream(stream))

    def append_qkv(self, layer: int, q, k, v, n_slices: int, t0: int, norm_q_weight, norm_k_weight,
                   eps: float = 1e-6, theta: float = 10000.0, stream=None, q_out=None):
        """The projection epilogue straight into the ring (DiT.swift:496-511): appends k' = rope(normK(k)) and v of
        the chunk (natural token order, f = 2 * n_slices) and returns q' = rope(normQ(q)) in window order."""
        q2, k2, v2 = (self._chunk(t, n, n_slices) for t, n in ((q, "q"), (k, "k"), (v, "v")))
        wq, wk = _norm_weights(norm_q_weight, norm_k_weight, self.channels, self.dtype)
        qo = _out_meta(q_out, q2, "q_out")
        _devices((q2, "q"), (k2, "k"), (v2, "v"), (wq, "norm_q_weight"), (wk, "norm_k_weight"), (qo, "q_out"))
        qo = torch.empty_like(q2) if qo is None else qo
        tab = rope_tables_device(q2.device, theta)
        call("fvsr_kv_ring_append_qkv", self.handle, layer, _ptr(q2), _ptr(k2), _ptr(v2), n_slices, t0, _ptr(wq),
             _ptr(wk), float(eps), _ptr(tab), _ptr(qo), _stream(stream))
        return qo

    def layer_call_qkv(self, layer: int, q, k, v, n_new_slices: int, t0: int, norm_q_weight, norm_k_weight, local,
                       topk: int, mode: int = ATTN_AUTO, eps: float = 1e-6, theta: float = 10000.0, stream=None,
                       out=None, q_work=None, want_mask=False, want_probs=False):
        """The LCSA layer call from the projections (DiT.swift:496-539): epilogue into the ring, select, attend,
        evict; returns (o in natural token order, mask, probs)."""
        q2, k2, v2 = (self._chunk(t, n, n_new_slices) for t, n in ((q, "q"), (k, "k"), (v, "v")))
        wq, wk = _norm_weights(norm_q_weight, norm_k_weight, self.channels, self.dtype)
        qw, o = _out_meta(q_work, q2, "q_work"), _out_meta(out, q2)
        _devices((q2, "q"), (k2, "k"), (v2, "v"), (wq, "norm_q_weight"), (wk, "norm_k_weight"), (qw, "q_work"),
                 (o, "out"))
        qw = torch.empty_like(q2) if qw is None else qw
        o = torch.empty_like(q2) if o is None else o
        tab = rope_tables_device(q2.device, theta)
        nq = n_new_slices * self.s
        nk = (self.slices(layer) + n_new_slices) * self.s
        dev = q2.device
        mask = torch.empty((self.heads, nq, nk), dtype=torch.float32, device=dev) if want_mask else None
        probs = torch.empty((self.heads, nq, nk), dtype=torch.float32, device=dev) if want_probs else None
        call("fvsr_lcsa_layer_qkv", self.ctx.handle, self.handle, layer, _ptr(q2), _ptr(k2), _ptr(v2), n_new_slices,
             t0, _ptr(wq), _ptr(wk), float(eps), _ptr(tab), _ptr(self.ctx.local_device(local, self.s)), topk, mode,
             _ptr(qw), _ptr(o), _ptr(mask), _ptr(probs), _stream(stream))
        return o, mask, probs

    def evict(self, layer: int):
        call("fvsr_kv_ring_evict", self.handle, layer)

    def slices(self, layer: int) -> int:
        n = C.c_int()
        call("fvsr_kv_ring_slices", self.handle, layer, C.byref(n))
        return n.value

    def read(self, layer: int, stream=None):
        n = self.slices(layer) * self.s * BLOCK
        ch = self.heads * HEAD_DIM
        dev = f"cuda:{self.ctx.device}"
        k = torch.empty((n, ch), dtype=self.dtype, device=dev)
        v = torch.empty((n, ch), dtype=self.dtype, device=dev)
        call("fvsr_kv_ring_read", self.handle, layer, _ptr(k), _ptr(v), _stream(stream))
        return k, v

    def select(self, layer: int, qW, q_slices: int, local, topk: int, stream=None, want_mask=True, want_probs=True):
        q = self._queries(qW, "qW")
        _devices((q, "qW"))
        nq = -(-q.shape[0] // BLOCK)
        nk = self.slices(layer) * self.s
        dev = q.device
        mask = torch.empty((self.heads, nq, nk), dtype=torch.float32, device=dev) if want_mask else None
        probs = torch.empty((self.heads, nq, nk), dtype=torch.float32, device=dev) if want_probs else None
        kidx = torch.empty((self.heads, nq, nk), dtype=torch.int32, device=dev)
        kcnt = torch.empty((self.heads, nq), dtype=torch.int32, device=dev)
        call("fvsr_lcsa_select_ring", self.ctx.handle, self.handle, layer, _ptr(q), q.shape[0], q_slices,
             _ptr(self.ctx.local_device(local, self.s)), topk, _ptr(mask), _ptr(probs), _ptr(kidx), _ptr(kcnt),
             _stream(stream))
        return mask, probs, kidx, kcnt

    def attention(self, layer: int, q, kidx, kcnt, mode: int = ATTN_KERNEL, stream=None, out=None):
        q2 = self._queries(q, "q")
        _lists_meta(kidx, kcnt, self.heads, -(-q2.shape[0] // BLOCK))
        o = _out_meta(out, q2)
        _devices((q2, "q"), (kidx, "kidx"), (kcnt, "kcnt"), (o, "out"))
        kidx, kcnt = kidx.to(torch.int32).contiguous(), kcnt.to(torch.int32).contiguous()
        o = torch.empty_like(q2) if o is None else o
        call("fvsr_lcsa_attention_ring", self.ctx.handle, self.handle, layer, _ptr(q2), q2.shape[0], _ptr(kidx),
             _ptr(kcnt), kidx.shape[-1], mode, _ptr(o), _stream(stream))
        return o

    def layer_call(self, layer: int, qW, k_new, v_new, n_new_slices: int, q_slices: int, local, topk: int,
                   mode: int = ATTN_AUTO, layout: int = LAYOUT_WINDOWS, stream=None, out=None, want_mask=False,
                   want_probs=False):
        """append -> select -> attention -> evict: the LCSA core of blockForward (DiT.swift:504-538)."""
        q2 = self._queries(qW, "qW")
        k2, v2 = self._chunk(k_new, "k_new", n_new_slices), self._chunk(v_new, "v_new", n_new_slices)
        o = _out_meta(out, q2)
        _devices((q2, "qW"), (k2, "k_new"), (v2, "v_new"), (o, "out"))
        o = torch.empty_like(q2) if o is None else o
        nq = -(-q2.shape[0] // BLOCK)
        nk = (self.slices(layer) + n_new_slices) * self.s
        dev = q2.device
        mask = torch.empty((self.heads, nq, nk), dtype=torch.float32, device=dev) if want_mask else None
        probs = torch.empty((self.heads, nq, nk), dtype=torch.float32, device=dev) if want_probs else None
        call("fvsr_lcsa_layer", self.ctx.handle, self.handle, layer, _ptr(q2), q2.shape[0], _ptr(k2), _ptr(v2),
             n_new_slices, layout, q_slices, _ptr(self.ctx.local_device(local, self.s)), topk, mode, _ptr(o), _ptr(mask),
             _ptr(probs), _stream(stream))
        return o, mask, probs


# ---------------------------------------------------------------------------------------------------------------
# (f3) the dense parts of the DiT block
# ---------------------------------------------------------------------------------------------------------------
def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, gelu: bool = False,
           stream=None, out=None) -> torch.Tensor:
    """`Linear` (y = x W^T + b, W (out, in)) on hipBLASLt in bf16 with fp32 accumulation; gelu applies the tanh-form
    GELU of the FFN (DiT.swift:371) to the fp32 result. x: (rows, in) bf16 on the device."""
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise FVSRError(_abi.ERR_UNSUPPORTED, "linear", "bf16 operands only")
    if x.dim() != 2 or not x.is_contiguous() or not weight.is_contiguous():
        raise FVSRError(_abi.ERR_INVALID_ARG, "linear", "expected contiguous (rows, in) x and (out, in) weight")
    n_out, n_in = weight.shape
    if x.shape[1] != n_in:
        raise FVSRError(_abi.ERR_INVALID_ARG, "linear", f"x has {x.shape[1]} features, weight expects {n_in}")
    _on_device(x, "x", x.device)
    _on_device(weight, "weight", x.device)
    y = torch.empty((x.shape[0], n_out), dtype=x.dtype, device=x.device) if out is None else out
    _on_device(y, "out", x.device, x.shape[0] * n_out)
    b = None if bias is None else _on_device(bias.to(torch.bfloat16).contiguous(), "bias", x.device, n_out)
    ctx = Context.get(x.device)
    call("fvsr_linear", ctx.handle, _ptr(x), x.shape[0], n_in, _ptr(weight), n_out, _ptr(b), 1 if gelu else 0,
         _ptr(y), _stream(stream))
    return y


class DiTBlock:
    """One `DiTBlock` (DiT.swift:363-375) with its weights on the device (bf16), run by `forward` as the streaming
    `blockForward` (DiT.swift:491-551) over a KVRing layer. `weights` maps the field names of
    fvsr_dit_block_weights (q_weight, q_bias, ..., ffn2_bias; see DIT_WEIGHT_FIELDS) to tensors; the cross
    K/V come from `set_context` (CrossAttention.initCache, DiT.swift:346-350)."""

    def __init__(self, weights: dict, heads: int, eps: float = 1e-6):
        self.heads = heads
        self.eps = eps
        self.t = {k: v.to(torch.bfloat16).contiguous() for k, v in weights.items() if v is not None}
        for need in ("q_weight", "ffn1_weight"):
            if need not in self.t:
                raise FVSRError(_abi.ERR_INVALID_ARG, "DiTBlock", f"{need} missing")
        self.ffn_dim = int(self.t["ffn1_weight"].shape[0])
        self.ctx_len = 0
        # every field's extent follows from C and the FFN width: check them here, the kernels only see pointers
        c, f = int(self.t["q_weight"].shape[0]), self.ffn_dim
        sizes = {"modulation": 6 * c, "ffn1_weight": f * c, "ffn1_bias": f, "ffn2_weight": c * f}
        for name in self.t:
            if name.endswith("_weight") and name not in sizes and "norm" not in name:
                sizes[name] = c * c
        dev = self.t["q_weight"].device
        for name, t in self.t.items():   # cross_k / cross_v are (ctx_len, C), normally from set_context
            _on_device(t, name, dev, None if name in ("cross_k", "cross_v") else sizes.get(name, c))
        self.device, self.dim = dev, c

    def _struct(self) -> _abi.DiTBlockWeights:
        w = _abi.DiTBlockWeights()
        for name, _ in _abi.DiTBlockWeights._fields_:
            if name in ("ctx_len", "ffn_dim"):
                continue
            setattr(w, name, self.t[name].data_ptr() if name in self.t else None)
        w.ctx_len = self.ctx_len
        w.ffn_dim = self.ffn_dim
        return w

    def set_context(self, context: torch.Tensor, stream=None):
        """context: (ctx_len, C) bf16 text-embedded prompt -> cached cross K/V."""
        ctxt = _tokens(context.to(torch.bfloat16).contiguous(), "context")
        _shaped(ctxt, "context", (ctxt.shape[0], self.dim))
        _devices((ctxt, "context"))
        _on_device(ctxt, "context", self.device)
        n = ctxt.shape[0]
        self.t["cross_k"] = torch.empty_like(ctxt)
        self.t["cross_v"] = torch.empty_like(ctxt)
        self.ctx_len = 0
        w = self._struct()
        ctx = Context.get(ctxt.device)
        call("fvsr_dit_cross_kv", ctx.handle, C.byref(w), self.heads, _ptr(ctxt), n, float(self.eps),
             _ptr(self.t["cross_k"]), _ptr(self.t["cross_v"]), _stream(stream))
        self.ctx_len = n

    def forward(self, ring: "KVRing", layer: int, x: torch.Tensor, t_mod: torch.Tensor, n_new_slices: int, t0: int,
                local, topk: int, mode: int = ATTN_AUTO, theta: float = 10000.0, stream=None) -> torch.Tensor:
        """x: (L, C) bf16 tokens in natural (f, h, w) order, updated in place and returned; t_mod: (6, C)."""
        if ring.dtype != torch.bfloat16 or ring.channels != self.dim:
            raise FVSRError(_abi.ERR_INVALID_ARG, "ring", f"expected a bf16 ring of {self.dim} channels, got "
                            f"{ring.dtype} with {ring.channels}")
        x2 = _tokens(x, "x")
        if x2.dtype != torch.bfloat16:
            raise FVSRError(_abi.ERR_UNSUPPORTED, "DiTBlock.forward", "bf16 tokens only")
        _shaped(x2, "x", (n_new_slices * ring.s * BLOCK, self.dim))
        if t_mod.numel() != 6 * self.dim:
            raise FVSRError(_abi.ERR_INVALID_ARG, "t_mod", f"expected (6, {self.dim}), got {tuple(t_mod.shape)}")
        tm = t_mod.to(torch.bfloat16).reshape(6, -1).contiguous()
        _devices((x2, "x"), (tm, "t_mod"))
        _on_device(x2, "x", self.device)
        tab = rope_tables_device(x2.device, theta)
        w = self._struct()
        call("fvsr_dit_block", ring.ctx.handle, ring.handle, layer, C.byref(w), _ptr(tm), _ptr(x2), n_new_slices, t0,
             float(self.eps), _ptr(tab), _ptr(ring.ctx.local_device(local, ring.s)), topk, mode, _stream(stream))
        return x
