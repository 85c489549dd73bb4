"""ctypes view of include/fvsr_lcsa.h (libfvsr_lcsa.so). No fallback: importing fails if the library is absent."""
from __future__ import annotations

import ctypes as C
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# FVSR_LCSA_LIB selects another build of the same library (e.g. one compiled with different launch parameters)
LIB_PATH = os.environ.get("FVSR_LCSA_LIB") or os.path.join(_PKG, "lib", "libfvsr_lcsa.so")

OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_HIP, ERR_OUT_OF_MEMORY, ERR_CAPACITY, ERR_STATE = range(7)
DTYPE_F32, DTYPE_BF16 = 0, 1
ATTN_AUTO, ATTN_DENSE, ATTN_KERNEL = 0, 1, 3
LAYOUT_WINDOWS, LAYOUT_GRID = 0, 1

_vp = C.c_void_p
_i = C.c_int
_i64 = C.c_int64
_sz = C.c_size_t

# name -> (restype, argtypes), in header order
SIGNATURES = {
    "fvsr_abi_version": (_i, []),
    "fvsr_last_error": (C.c_char_p, []),
    "fvsr_device_props": (_i, [_i, C.POINTER(_i), C.POINTER(_i), C.POINTER(_sz), C.c_char_p, _sz]),
    "fvsr_ctx_create": (_i, [_i, C.POINTER(_vp)]),
    "fvsr_ctx_destroy": (_i, [_vp]),
    "fvsr_ctx_reserve": (_i, [_vp, _sz]),
    "fvsr_ctx_workspace_bytes": (_sz, [_vp]),
    "fvsr_workspace_size": (_sz, [_i, _i64, _i64, _i]),
    "fvsr_local_block_mask": (_i, [_i, _i, _i, _vp]),
    "fvsr_attention_mode_auto": (_i, [_i, _i, _i, C.c_double, C.POINTER(C.c_double), C.POINTER(_i)]),
    "fvsr_lcsa_select": (_i, [_vp, _i, _vp, _i64, _vp, _i64, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "fvsr_lcsa_attention": (_i, [_vp, _i, _vp, _i64, _vp, _vp, _i64, _i, _vp, _vp, _i, _vp, _vp]),
    "fvsr_lcsa_attention_noalloc": (_i, [_vp, _i, _vp, _i64, _vp, _vp, _i64, _i, _vp, _vp, _i, _vp, _vp]),
    "fvsr_lcsa_attention_mask": (_i, [_vp, _i, _vp, _i64, _vp, _vp, _i64, _i, _vp, _i, _vp, _vp]),
    "fvsr_kv_ring_create": (_i, [_vp, _i, _i, _i, _i, _i, _i, _i, C.POINTER(_vp)]),
    "fvsr_kv_ring_destroy": (_i, [_vp]),
    "fvsr_kv_ring_reset": (_i, [_vp]),
    "fvsr_kv_ring_append": (_i, [_vp, _i, _vp, _vp, _i, _i, _vp]),
    "fvsr_kv_ring_evict": (_i, [_vp, _i]),
    "fvsr_kv_ring_slices": (_i, [_vp, _i, C.POINTER(_i)]),
    "fvsr_kv_ring_read": (_i, [_vp, _i, _vp, _vp, _vp]),
    "fvsr_lcsa_select_ring": (_i, [_vp, _vp, _i, _vp, _i64, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "fvsr_lcsa_attention_ring": (_i, [_vp, _vp, _i, _vp, _i64, _vp, _vp, _i, _i, _vp, _vp]),
    "fvsr_lcsa_layer": (_i, [_vp, _vp, _i, _vp, _i64, _vp, _vp, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp, _vp]),
    "fvsr_rope_tables_size": (_sz, []),
    "fvsr_rope_tables": (_i, [C.c_double, _vp, _sz]),
    "fvsr_qkv_epilogue": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp, C.c_float, _vp, _vp, _vp, _vp,
                               _vp]),
    "fvsr_kv_ring_append_qkv": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, C.c_float, _vp, _vp, _vp]),
    "fvsr_lcsa_layer_qkv": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, C.c_float, _vp, _vp, _i, _i, _vp,
                                 _vp, _vp, _vp, _vp]),
    "fvsr_ctx_reserve_block": (_i, [_vp, _i, _i64, _i, _i, _i64]),
    "fvsr_ctx_block_workspace_bytes": (_sz, [_vp]),
    "fvsr_linear": (_i, [_vp, _vp, _i64, _i, _vp, _i, _vp, _i, _vp, _vp]),
    "fvsr_dit_cross_kv": (_i, [_vp, _vp, _i, _vp, _i, C.c_float, _vp, _vp, _vp]),
    "fvsr_dit_block": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, C.c_float, _vp, _vp, _i, _i, _vp]),
    "fvsr_window_partition": (_i, [_i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "fvsr_window_reverse": (_i, [_i, _vp, _vp, _i, _i, _i, _i, _vp]),
}


# struct fvsr_dit_block_weights, field for field
DIT_WEIGHT_FIELDS = ["modulation", "q_weight", "q_bias", "k_weight", "k_bias", "v_weight", "v_bias", "o_weight",
                     "o_bias", "norm_q_weight", "norm_k_weight", "cross_q_weight", "cross_q_bias", "cross_k_weight",
                     "cross_k_bias", "cross_v_weight", "cross_v_bias", "cross_o_weight", "cross_o_bias",
                     "cross_norm_q_weight", "cross_norm_k_weight", "cross_k", "cross_v"]


class DiTBlockWeights(C.Structure):
    _fields_ = ([(n, _vp) for n in DIT_WEIGHT_FIELDS] + [("ctx_len", _i)] +
                [(n, _vp) for n in ["norm3_weight", "norm3_bias", "ffn1_weight", "ffn1_bias", "ffn2_weight",
                                    "ffn2_bias"]] + [("ffn_dim", _i)])


class FVSRError(RuntimeError):
    """A non-zero fvsr_status; `.status` holds the code."""

    def __init__(self, status: int, fn: str, msg: str):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status


def load(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(f"libfvsr_lcsa is not built ({path} missing): build it first with python mlx-flashvsr-swift_amd/build_lib.py")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()


def call(name: str, *args) -> int:
    """Call an int-returning entry point and raise FVSRError on a non-zero status."""
    rc = getattr(lib, name)(*args)
    if rc != OK:
        raise FVSRError(rc, name, lib.fvsr_last_error().decode(errors="replace"))
    return rc
