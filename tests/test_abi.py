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
    with pytest.raises(fvsr_lcsa.FVSRError, match="device tensor"):
        fvsr_lcsa.block_sparse_attention(x, x, x, torch.zeros((1, 1, 1), dtype=torch.int32),
                                         torch.zeros((1, 1), dtype=torch.int32), 1)
