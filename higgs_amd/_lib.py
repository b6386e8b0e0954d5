"""Loader for libhiggs_hip.so and ctypes prototypes of its C ABI.

The prototypes mirror include/higgs_hip.h one for one. Loading fails loudly
(HgkError) when the library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libhiggs_hip.so")

F32, BF16, F16, U32, I32 = 0, 1, 2, 3, 4
ACT_SILU, ACT_GELU_TANH = 0, 1
OK, ERR_ARG, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3

_vp, _i64, _int, _f32, _i32 = C.c_void_p, C.c_int64, C.c_int, C.c_float, C.c_int32
_i64p = C.POINTER(C.c_int64)
_f32p = C.POINTER(C.c_float)

class HgkOp(C.Structure):
    """hgk_op of include/higgs_hip.h (one op of a decode step's op sequence)."""
    _fields_ = [("kind", C.c_int), ("rows", C.c_int), ("n", C.c_int), ("eps", C.c_float),
                ("x", C.c_void_p), ("x_tok", C.c_int64), ("x_row", C.c_int64),
                ("r", C.c_void_p), ("r_tok", C.c_int64), ("r_row", C.c_int64),
                ("z_group_rows", C.c_int64), ("z_group_stride", C.c_int64),
                ("w", C.c_void_p), ("w2", C.c_void_p),
                ("y", C.c_void_p), ("y_tok", C.c_int64), ("y_row", C.c_int64),
                ("h", C.c_void_p), ("h_tok", C.c_int64), ("h_row", C.c_int64),
                ("act", C.c_int), ("k_heads", C.c_int), ("dims", C.c_int), ("base", C.c_float),
                ("freqs", C.POINTER(C.c_float)), ("scale", C.c_float),
                ("offsets", C.c_void_p), ("offset", C.c_int32)]


OP_RMS_NORM, OP_ADD_RMS_NORM, OP_GATED_RMS_NORM, OP_QK_NORM_ROPE, OP_GLU = 0, 1, 2, 3, 4

# name -> (restype, argtypes); kept in the order of include/higgs_hip.h
PROTOTYPES = {
    "hgk_last_error": (C.c_char_p, []),
    "hgk_abi_version": (_int, []),
    "hgk_sync": (_int, [_vp]),
    "hgk_rms_norm": (_int, [_vp, _int, _i64, _vp, _int, _int, _f32, _vp, _int, _i64,
                            _i64, _i64, _vp]),
    "hgk_rope_inv_freq": (_int, [_f32, _int, _f32p, _f32p]),
    "hgk_llama3_rope_freqs": (_int, [_f32, _int, _f32, _f32, _f32, _f32, _f32p]),
    "hgk_rope": (_int, [_int, _vp, _i64p, _vp, _i64p, _i64, _i64, _i64, _i64, _int, _int,
                        _f32, _f32, _f32p, _i32, _vp, _vp]),
    "hgk_qk_norm_rope": (_int, [_int, _vp, _i64p, _vp, _i64p, _i64, _vp,
                                _vp, _i64p, _vp, _i64p, _i64, _vp,
                                _int, _f32, _i64, _i64, _i64, _int, _f32, _f32, _f32p,
                                _i32, _vp, _vp]),
    "hgk_glu": (_int, [_int, _int, _vp, _i64, _vp, _i64, _vp, _int, _i64, _i64, _i64, _vp]),
    "hgk_gated_rms_norm": (_int, [_int, _vp, _i64, _vp, _i64, _i64, _i64, _vp, _int, _f32,
                                  _vp, _int, _i64, _i64, _i64, _vp]),
    "hgk_quantized_embedding": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _int, _i64, _i64,
                                       _int, _int, _f32, _vp, _i64, _vp]),
    "hgk_add_rms_norm": (_int, [_int, _vp, _i64, _vp, _i64, _vp, _int, _int, _f32, _vp, _i64,
                                _vp, _int, _i64, _i64, _i64, _vp]),
    "hgk_quantized_embedding_rms_norm": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _int, _i64,
                                                _i64, _int, _int, _f32, _vp, _i64, _vp, _int,
                                                _int, _f32, _vp, _int, _i64, _vp]),
    "hgk_gather_qmm": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _int, _i64, _i64,
                              _i64, _int, _int, _vp, _int, _i64, _vp, _i64, _vp]),
    "hgk_gather_qmm_swiglu": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _int, _i64, _i64, _i64, _int, _int, _vp, _int, _i64,
                                     _vp, _i64, _vp]),
    "hgk_quantized_matmul": (_int, [_int, _vp, _i64, _i64, _vp, _vp, _vp, _int, _i64, _i64, _int,
                                    _int, _vp, _i64, _vp]),
    "hgk_gated_delta": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _int, _vp, _vp, _vp, _f32,
                               _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "hgk_gated_delta_gated_norm": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _int, _vp,
                                          _vp, _vp, _f32, _i64, _i64, _i64, _i64, _i64, _vp,
                                          _vp, _vp, _i64, _i64, _i64, _vp, _int, _f32, _vp,
                                          _vp]),
    "hgk_op_list_bytes": (_i64, [_int]),
    "hgk_op_list_upload": (_int, [_int, C.POINTER(HgkOp), _int, _vp, _i64, _vp]),
    "hgk_op_list_run": (_int, [_int, _vp, _int, _i64, _vp]),
    "hgk_st_open": (_int, [C.c_char_p, C.POINTER(_vp)]),
    "hgk_st_close": (None, [_vp]),
    "hgk_st_count": (_i64, [_vp]),
    "hgk_st_find": (_int, [_vp, C.c_char_p, C.POINTER(_i64)]),
    "hgk_st_tensor": (_int, [_vp, _i64, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p),
                             C.POINTER(_int), C.POINTER(_int), C.POINTER(_i64),
                             C.POINTER(_i64)]),
    "hgk_st_copy_to_host": (_int, [_vp, _i64, _vp, _i64]),
    "hgk_st_upload": (_int, [_vp, _i64, _vp, _i64, _vp]),
    "hgk_st_collect_files": (_int, [C.c_char_p, C.c_char_p, _i64, C.POINTER(_i64)]),
    "hgk_remap_quantized_key": (_int, [C.c_char_p, C.c_char_p, _i64]),
    "hgk_last_launch_grid": (_int, [_i64p, C.POINTER(_int)]),
    "hgk_floor_empty": (_int, [_i64, _int, _vp]),
    "hgk_floor_stream": (_int, [_vp, _i64, _vp, _i64, _int, _vp]),
}


class HgkError(RuntimeError):
    """A non-zero status from the C ABI (the mlx Exception::custom analogue)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[status {status}] {message}")
        self.status = status


_lib = None


def lib():
    """The loaded library (built beforehand by higgs_amd.build)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HgkError(ERR_UNSUPPORTED,
                           f"{LIB_PATH} is missing: build it with `python -m higgs_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = lib().hgk_last_error().decode(errors="replace")
        raise HgkError(status, msg)


def i64_array(vals):
    arr = (C.c_int64 * len(vals))(*[int(v) for v in vals])
    return arr


def f32_array(vals):
    return (C.c_float * len(vals))(*[float(v) for v in vals])
