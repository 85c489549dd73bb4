"""CPU checks of the C ABI: the library loads, exports every function include/fvsr_lcsa.h declares, its host-only
functions agree with the oracle, and invalid arguments are rejected before any device work."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import fvsr_lcsa
from fvsr_lcsa import _abi
from oracle import lcsa as O

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "fvsr_lcsa.h")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\*?\s+\*?(fvsr_\w+)\(", text, flags=re.M)))


def test_header_declares_the_expected_surface():
    names = header_functions()
    assert len(names) >= 24
    assert set(names) == set(_abi.SIGNATURES), set(names) ^ set(_abi.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(_abi.LIB_PATH)
    for name in header_functions():
        assert hasattr(lib, name), name


def test_abi_version():
    assert _abi.lib.fvsr_abi_version() == 1


@pytest.mark.parametrize("bh,bw,r", [(3, 4, 11), (6, 10, 3), (5, 5, 4), (9, 15, 11), (4, 4, 3)])
def test_local_block_mask_host_matches_oracle(bh, bw, r):
    np.testing.assert_array_equal(fvsr_lcsa.local_block_mask(bh, bw, r), O.local_block_mask(bh, bw, r))


def test_attention_mode_auto_rule():
    # DiT.swift:517-522: expected = min(1, (topk+1)/(s*nk)); kernel iff <= 0.45
    e, m = fvsr_lcsa.attention_mode_auto(16199, 135, 540)
    assert e == pytest.approx(16200 / (135 * 540)) and m == fvsr_lcsa.ATTN_KERNEL       # 1920x1152: 22 %
    topk_720p = O.step_topk(60, O.default_topk_ratio(768, 1280))                       # ratio 2.0 -> 7199
    e, m = fvsr_lcsa.attention_mode_auto(topk_720p, 60, 180)
    assert e == pytest.approx(0.6667, abs=1e-4) and m == fvsr_lcsa.ATTN_DENSE           # 1280x768 chunk 0: 67 %
    e, m = fvsr_lcsa.attention_mode_auto(topk_720p, 60, 240)
    assert e == pytest.approx(0.5) and m == fvsr_lcsa.ATTN_DENSE                         # later chunks: 50 %
    e, m = fvsr_lcsa.attention_mode_auto(10**9, 10, 10)
    assert e == 1.0 and m == fvsr_lcsa.ATTN_DENSE


def test_workspace_size_grows_with_geometry():
    a = fvsr_lcsa.workspace_size(12, 17280, 43200, 1536)
    b = fvsr_lcsa.workspace_size(12, 17280, 69120, 1536)
    assert 0 < a < b
    assert fvsr_lcsa.workspace_size(0, 1, 1, 1) == 0


def _status(name, *args):
    return getattr(_abi.lib, name)(*args)


def test_null_context_is_rejected_with_message():
    p = C.c_void_p(0)
    rc = _status("fvsr_lcsa_attention", p, 1, p, 128, p, p, 128, 12, p, p, 1, p, p)
    assert rc == _abi.ERR_INVALID_ARG
    assert b"ctx" in _abi.lib.fvsr_last_error()


def test_window_layout_rejects_untileable_grid_before_device_work():
    p = C.c_void_p(8)   # never dereferenced: validation fails first
    assert _status("fvsr_window_partition", 1, p, p, 3, 16, 16, 1536, None) == _abi.ERR_INVALID_ARG
    assert _status("fvsr_window_reverse", 1, p, p, 2, 12, 16, 1536, None) == _abi.ERR_INVALID_ARG
    assert _status("fvsr_window_partition", 7, p, p, 2, 16, 16, 1536, None) == _abi.ERR_INVALID_ARG
    assert b"dtype" in _abi.lib.fvsr_last_error()


def test_ring_calls_reject_null_ring():
    assert _status("fvsr_kv_ring_evict", None, 0) == _abi.ERR_INVALID_ARG
    n = C.c_int()
    assert _status("fvsr_kv_ring_slices", None, 0, C.byref(n)) == _abi.ERR_INVALID_ARG
    assert _status("fvsr_kv_ring_reset", None) == _abi.ERR_INVALID_ARG


def test_local_mask_rejects_bad_geometry():
    buf = np.zeros(16, dtype=np.uint8)
    assert _status("fvsr_local_block_mask", 0, 4, 3, buf.ctypes.data_as(C.c_void_p)) == _abi.ERR_INVALID_ARG
    assert _status("fvsr_local_block_mask", 2, 2, 3, None) == _abi.ERR_INVALID_ARG


def test_python_binding_raises_fvsr_error():
    with pytest.raises(fvsr_lcsa.FVSRError) as ei:
        _abi.call("fvsr_local_block_mask", -1, 4, 3, None)
    assert ei.value.status == _abi.ERR_INVALID_ARG


def test_rope_tables_host_matches_oracle():
    """fvsr_rope_tables (host, no device work) against the oracle's float64 -> float32 tables: equal up to one
    float32 ulp (the two libm's float64 cos/sin may differ in the last bit before the float32 rounding)."""
    got = fvsr_lcsa.rope_tables()
    ref = O.rope_tables_flat()
    assert got.shape == ref.shape
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert (d <= np.spacing(np.abs(ref)).astype(np.float64) + 1e-45).all()
    assert (got == ref).mean() > 0.999


def test_rope_tables_rejects_short_buffer():
    out = np.empty(10, dtype=np.float32)
    rc = _abi.lib.fvsr_rope_tables(10000.0, out.ctypes.data_as(C.c_void_p), 10)
    assert rc == _abi.ERR_INVALID_ARG


def test_binding_rejects_host_operands_before_any_device_call():
    """The binding checks where each operand lives before a pointer reaches the library: host tensors are refused
    (no context is created, so this runs without a GPU)."""
    import torch
    x = torch.zeros((4, 16), dtype=torch.bfloat16)
    w = torch.zeros((16, 16), dtype=torch.bfloat16)
    with pytest.raises(fvsr_lcsa.FVSRError, match="expected a tensor on") as ei:
        fvsr_lcsa.linear(x, w)
    assert ei.value.status == _abi.ERR_INVALID_ARG
    t = torch.zeros((4, 128), dtype=torch.bfloat16)
    with pytest.raises(fvsr_lcsa.FVSRError, match="HIP device"):
        fvsr_lcsa.block_sparse_attention(t, t, t, torch.zeros((1, 1, 1), dtype=torch.int32),
                                         torch.zeros((1, 1), dtype=torch.int32), 1)


def _host_ring(heads=2, bh=2, bw=3, dtype=None):
    """A KVRing shell with the geometry of a real one but no library handle: enough for the binding's argument
    checks, which all run before any library call (so no GPU is needed)."""
    import torch
    r = object.__new__(fvsr_lcsa.KVRing)
    r.ctx, r.handle = None, None
    r.layers, r.heads, r.bh, r.bw, r.s = 1, heads, bh, bw, bh * bw
    r.capacity, r.kv_len = 4, 3
    r.dtype = torch.bfloat16 if dtype is None else dtype
    r.channels = heads * 128
    r.code = _abi.DTYPE_BF16
    return r


def test_binding_rejects_wrong_extents_before_any_device_call():
    """Every operand whose extent the library derives from other arguments is checked for shape and dtype before
    its device, so a short list, a narrow token buffer, a wrong-sized output or an int64 list is named on the host
    (the C ABI sees only pointers and would read or write past the buffer)."""
    import torch
    E = fvsr_lcsa.FVSRError
    bf = torch.bfloat16
    q = torch.zeros((256, 256), dtype=bf)
    k = torch.zeros((384, 256), dtype=bf)
    kidx = torch.zeros((2, 2, 3), dtype=torch.int32)
    kcnt = torch.zeros((2, 2), dtype=torch.int32)
    # attention from lists
    with pytest.raises(E, match="expected \\(L, 384\\)"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx, kcnt, 3)              # width is not heads * 128
    with pytest.raises(E, match="kidx"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx[:, :1], kcnt, 2)       # lists of one query block, two needed
    with pytest.raises(E, match="kcnt"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx, kcnt[:1], 2)
    with pytest.raises(E, match="integer"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx.float(), kcnt, 2)
    with pytest.raises(E, match="shape of k"):
        fvsr_lcsa.block_sparse_attention(q, k, k[:128], kidx, kcnt, 2)
    with pytest.raises(E, match="out"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx, kcnt, 2, out=torch.zeros((128, 256), dtype=bf))
    with pytest.raises(E, match="out"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx, kcnt, 2, out=torch.zeros((256, 256)))   # fp32 out
    with pytest.raises(E, match="HIP device"):
        fvsr_lcsa.block_sparse_attention(q, k, k, kidx.long(), kcnt, 2)       # right shapes: only the device is wrong
    # attention under a mask
    with pytest.raises(E, match="block_mask"):
        fvsr_lcsa.kernel_block_attention(q, k, k, torch.ones((2, 2, 2)), 2)   # 3 key blocks
    with pytest.raises(E, match="out"):
        fvsr_lcsa.block_masked_attention(q, k, k, torch.ones((2, 2, 3)), 2, out=torch.zeros((256, 128), dtype=bf))
    # selection
    with pytest.raises(E, match="qW"):
        fvsr_lcsa.draft_block_mask_and_probs(q, k, 1, 1, 2, np.ones((2, 2), bool), 1)
    with pytest.raises(E, match="kW"):
        fvsr_lcsa.draft_block_mask_and_probs(q, k.float(), 2, 1, 2, np.ones((2, 2), bool), 1)
    # epilogue
    w = torch.ones(256, dtype=bf)
    with pytest.raises(E, match="norm_k_weight"):
        fvsr_lcsa.qkv_epilogue(q[:128], q[:128], q[:128], 2, 8, 8, 2, 0, w, w[:128])
    with pytest.raises(E, match="'k'|k:|expected shape"):
        fvsr_lcsa.qkv_epilogue(q[:128], q[:64], q[:128], 2, 8, 8, 2, 0, w, w)


def test_ring_binding_rejects_wrong_extents_before_any_device_call():
    import torch
    E = fvsr_lcsa.FVSRError
    bf = torch.bfloat16
    ring = _host_ring(heads=2, bh=2, bw=3)        # s = 6 blocks per slice, C = 256
    tok = torch.zeros((6 * 128, 256), dtype=bf)   # one slice
    w = torch.ones(256, dtype=bf)
    local = np.ones((6, 6), bool)
    with pytest.raises(E, match="k_new"):
        ring.append(0, tok[:640], tok, 1)
    with pytest.raises(E, match="v_new"):
        ring.append(0, tok, tok.float(), 1)                                   # dtype differs from the ring's
    with pytest.raises(E, match="expected shape"):
        ring.append(0, tok, tok, 2)                                           # two slices announced, one given
    with pytest.raises(E, match="norm_q_weight"):
        ring.append_qkv(0, tok, tok, tok, 1, 0, w[:255], w)
    with pytest.raises(E, match="q_out"):
        ring.append_qkv(0, tok, tok, tok, 1, 0, w, w, q_out=tok[:128])
    with pytest.raises(E, match="q_work"):
        ring.layer_call_qkv(0, tok, tok, tok, 1, 0, w, w, local, 10, q_work=tok[:, :128])
    with pytest.raises(E, match="out"):
        ring.layer_call_qkv(0, tok, tok, tok, 1, 0, w, w, local, 10, out=tok.float())
    with pytest.raises(E, match="kidx"):
        ring.attention(0, tok, torch.zeros((2, 5, 4), dtype=torch.int32), torch.zeros((2, 6), dtype=torch.int32))
    with pytest.raises(E, match="kcnt"):
        ring.attention(0, tok, torch.zeros((2, 6, 4), dtype=torch.int32), torch.zeros((2, 5), dtype=torch.int32))
    with pytest.raises(E, match="qW"):
        ring.select(0, torch.zeros((768, 384), dtype=bf), 1, local, 10)
    with pytest.raises(E, match="k_new"):
        ring.layer_call(0, tok, tok[:128], tok, 1, 1, local, 10)
    with pytest.raises(E, match="HIP device"):
        ring.layer_call(0, tok, tok, tok, 1, 1, local, 10)                    # right shapes, host tensors


def test_dit_block_forward_checks_ring_and_tokens():
    import torch
    E = fvsr_lcsa.FVSRError
    blk = object.__new__(fvsr_lcsa.DiTBlock)
    blk.dim, blk.heads, blk.device = 256, 2, torch.device("cuda:0")
    ring = _host_ring(heads=2, bh=2, bw=3)
    x = torch.zeros((6 * 128, 256), dtype=torch.bfloat16)
    tm = torch.zeros((6, 256), dtype=torch.bfloat16)
    with pytest.raises(E, match="expected shape"):
        blk.forward(ring, 0, x[:512], tm, 1, 0, np.ones((6, 6), bool), 10)     # rows are not one slice
    with pytest.raises(E, match="ring"):
        blk.forward(_host_ring(heads=3, bh=2, bw=3), 0, x, tm, 1, 0, np.ones((6, 6), bool), 10)
    with pytest.raises(E, match="t_mod"):
        blk.forward(ring, 0, x, tm[:5], 1, 0, np.ones((6, 6), bool), 10)
    with pytest.raises(E, match="HIP device"):
        blk.forward(ring, 0, x, tm, 1, 0, np.ones((6, 6), bool), 10)
