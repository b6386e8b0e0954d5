"""ctypes/numpy wrapper over liboracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle restates MLX's CPU-device arithmetic for the per-layer ops that
higgs-models calls through mlx-rs (see oracle.h for the reference call sites).
Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.

Arrays cross this boundary as numpy arrays in their storage dtype: bf16 and f16
are carried as ``np.uint16`` bit patterns, f32 as ``np.float32``.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

F32, BF16, F16, U32, I32 = 0, 1, 2, 3, 4
ACT_SILU, ACT_GELU_TANH = 0, 1

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_vp = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int
_f32 = C.c_float
_u64 = C.c_uint64


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    cmd = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        sig = {
            "or_f32_to_bf16": (C.c_uint16, [_f32]),
            "or_bf16_to_f32": (_f32, [C.c_uint16]),
            "or_f32_to_f16": (C.c_uint16, [_f32]),
            "or_f16_to_f32": (_f32, [C.c_uint16]),
            "or_mlx_exp": (_f32, [_f32]),
            "or_mlx_sigmoid": (_f32, [_f32]),
            "or_promote": (_i32, [_i32, _i32]),
            "or_fill_normal": (None, [_u64, _f32, _f32, _vp, _i64]),
            "or_fill_uniform": (None, [_u64, _f32, _f32, _vp, _i64]),
            "or_fill_u32": (None, [_u64, _vp, _i64]),
            "or_fill_ids": (None, [_u64, C.c_uint32, _vp, _i64]),
            "or_fill_offsets": (None, [_u64, C.c_int32, C.c_int32, _vp, _i64]),
            "or_convert_from_f32": (None, [_i32, _vp, _vp, _i64]),
            "or_convert_to_f32": (None, [_i32, _vp, _vp, _i64]),
            "or_rms_norm": (_i32, [_vp, _i32, _i64, _vp, _i32, _i32, _f32,
                                   _vp, _i32, _i64, _i64, _i64]),
            "or_add": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64]),
            "or_gather_qmm": (_i32, [_i32, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i32,
                                     _i64, _i64, _i64, _i32, _vp, _i64, _vp, _i64]),
            "or_gated_delta": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp,
                                      _f32, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
            "or_rope_inv_freq": (None, [_f32, _i32, _vp, _vp]),
            "or_llama3_freqs": (None, [_f32, _i32, _f32, _f32, _f32, _f32, _vp]),
            "or_norm_rope": (_i32, [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                    _i64, _vp, _i32, _f32, _i32, _vp, _f32,
                                    C.c_int32, _vp]),
            "or_norm_rope_trig": (_i32, [_i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                         _i64, _vp, _i32, _f32, _i32, _vp, _f32,
                                         C.c_int32, _vp, _i32]),
            "or_glu": (_i32, [_i32, _i32, _vp, _i64, _vp, _i64, _vp, _i32, _i64,
                              _i64, _i64]),
            "or_gated_rms_norm": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _i32,
                                         _f32, _vp, _i32, _i64, _i64, _i64]),
            "or_qembed": (_i32, [_vp, _i32, _i64, _vp, _vp, _vp, _i32, _i64,
                                 _i64, _i32, _i32, _f32, _vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(_vp)


def storage_dtype(dt: int):
    return {F32: np.float32, BF16: np.uint16, F16: np.uint16, U32: np.uint32,
            I32: np.int32}[dt]


# ---------------------------------------------------------------- inputs
def normal(key: int, shape, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), np.float32)
    lib().or_fill_normal(key, mean, std, _p(out), out.size)
    return out.reshape(shape)


def uniform(key: int, shape, lo, hi) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), np.float32)
    lib().or_fill_uniform(key, lo, hi, _p(out), out.size)
    return out.reshape(shape)


def u32(key: int, shape) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), np.uint32)
    lib().or_fill_u32(key, _p(out), out.size)
    return out.reshape(shape)


def ids(key: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().or_fill_ids(key, vocab, _p(out), n)
    return out


def offsets(key: int, n: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().or_fill_offsets(key, lo, hi, _p(out), n)
    return out


def from_f32(a: np.ndarray, dt: int) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    if dt == F32:
        return a.copy()
    out = np.empty(a.shape, np.uint16)
    lib().or_convert_from_f32(dt, _p(a), _p(out), a.size)
    return out


def to_f32(a: np.ndarray, dt: int) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if dt == F32:
        return a.astype(np.float32, copy=True)
    out = np.empty(a.shape, np.float32)
    lib().or_convert_to_f32(dt, _p(a), _p(out), a.size)
    return out


def promote(a: int, b: int) -> int:
    return lib().or_promote(a, b)


# ---------------------------------------------------------------- ops
def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (status {rc})")


def rms_norm(x, x_dt, w, w_dt, eps, *, plus_one=False, out_dt=None):
    """x: [rows, n] storage array (rows may be a strided view of a 2-D buffer)."""
    rows, n = x.shape
    assert x.strides[1] == x.itemsize
    w_eff = (F32 if plus_one else w_dt) if w is not None else x_dt
    t_out = promote(x_dt, w_eff)
    out_dt = t_out if out_dt is None else out_dt
    y = np.empty((rows, n), storage_dtype(out_dt))
    _check(lib().or_rms_norm(_p(x), x_dt, x.strides[0] // x.itemsize, _p(w),
                             w_dt, int(plus_one), eps, _p(y), out_dt, n, rows, n),
           "rms_norm")
    return y


def add(a, b, dt):
    """MLX add of two [rows, n] storage arrays (rows may be strided views)."""
    rows, n = a.shape
    assert b.shape == a.shape and a.strides[1] == a.itemsize and b.strides[1] == b.itemsize
    out = np.empty((rows, n), storage_dtype(dt))
    _check(lib().or_add(dt, C.c_void_p(a.__array_interface__["data"][0]), a.strides[0] // a.itemsize,
                        C.c_void_p(b.__array_interface__["data"][0]), b.strides[0] // b.itemsize,
                        _p(out), n, rows, n), "add")
    return out


def add_rms_norm(x, r, dt, w, w_dt, eps, *, plus_one=False, out_dt=None):
    """The block boundary `h = x.add(residual); norm(h)` (transformer.rs:413-415;
    qwen3_next.rs:1539-1540): returns (h, y) with h = MLX add on dt and
    y = rms_norm(h)."""
    h = add(x, r, dt)
    return h, rms_norm(h, dt, w, w_dt, eps, plus_one=plus_one, out_dt=out_dt)


def qembed_rms_norm(ids_arr, wq, scales, biases, s_dt, w, w_dt, eps, *, group=64, bits=4,
                    out_scale=0.0, plus_one=False, out_dt=None):
    """`embed_tokens.forward(ids)` then the first block's
    `input_layernorm.forward(&h)` (transformer.rs:494, 407; gemma2.rs:587-600,
    491): returns (h, y) for ids flattened to [T]."""
    h = qembed(np.ascontiguousarray(ids_arr).reshape(-1), wq, scales, biases, s_dt,
               group=group, bits=bits, out_scale=out_scale)
    return h, rms_norm(h, s_dt, w, w_dt, eps, plus_one=plus_one, out_dt=out_dt)


def gather_qmm(x, x_dt, w, scales, biases, s_dt, experts, *, group=64, x_div=1, lhs=None):
    """SwitchMlpWeights::forward_gather's gather_qmm (qwen3_next.rs:844-904):
    x [R, K] storage array, w [E, N, K/8] u32, scales/biases [E, N, K/group],
    experts int32 [P]; pair p uses x row lhs[p] (or p // x_div). Returns
    y [P, N] in x's dtype: the exact contraction rounded once."""
    x = np.ascontiguousarray(x)
    R, K = x.shape
    E, N, _ = w.shape
    experts = np.ascontiguousarray(experts, np.int32)
    P = experts.size
    y = np.empty((P, N), storage_dtype(x_dt))
    lhs_arr = None if lhs is None else np.ascontiguousarray(lhs, np.int32)
    _check(lib().or_gather_qmm(x_dt, _p(x), R, K, x_div, _p(lhs_arr),
                               _p(np.ascontiguousarray(w, np.uint32)), _p(np.ascontiguousarray(scales)),
                               _p(np.ascontiguousarray(biases)), s_dt, E, N, K, group,
                               _p(experts), P, _p(y), N), "gather_qmm")
    return y


def quantized_matmul(x, x_dt, w, scales, biases, s_dt, *, group=64):
    """QLinear::forward's quantized_matmul (qwen3_next.rs:174-183): x [M, K],
    w [N, K/8] u32, scales/biases [N, K/group]; y [M, N] in x's dtype, the
    exact contraction rounded once (gather_qmm with one expert)."""
    M = np.asarray(x).shape[0]
    return gather_qmm(x, x_dt, np.asarray(w)[None], np.asarray(scales)[None],
                      np.asarray(biases)[None], s_dt, np.zeros(M, np.int32), group=group)


def gated_delta(q, k, v, a_log, a, dt_bias, b, dt, *, p_dt=F32, state=None, qw=None, kw=None,
                eps=1e-6):
    """GatedDeltaNet recurrence (qwen3_next.rs:376-451): q, k [B,T,Hk,Dk],
    v [B,T,Hv,Dv], a, b [B,T,Hv] in dt; a_log, dt_bias [Hv] in p_dt; state
    [B,Hv,Dv,Dk] in dt or None. qw/kw: the constant q/k norm weights [Dk] in
    dt (1172-1173), or None. Returns (y [B,T,Hv,Dv], state_out) in dt."""
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    y = np.empty((B, T, Hv, Dv), storage_dtype(dt))
    so = np.empty((B, Hv, Dv, Dk), storage_dtype(dt))
    c = lambda arr: None if arr is None else np.ascontiguousarray(arr)
    q, k, v, a, b, a_log, dt_bias, state, qw, kw = map(c, (q, k, v, a, b, a_log, dt_bias, state, qw, kw))
    _check(lib().or_gated_delta(dt, _p(q), _p(k), _p(v), _p(a_log), _p(a), _p(dt_bias), _p(b), p_dt,
                                _p(state), _p(qw), _p(kw), eps, B, T, Hk, Dk, Hv, Dv, _p(y), _p(so)),
           "gated_delta")
    return y, so


def gdn_qk_norm_weights(Dk: int, dt: int):
    """The constant q/k norm weights of GatedDeltaNet (qwen3_next.rs:1075-1094):
    s = 1/sqrt(Dk) in f32; q's weight is s*s, k's is s, each cast to dt."""
    s = np.float32(1.0) / np.sqrt(np.float32(Dk))
    return (from_f32(np.full(Dk, s * s, np.float32), dt), from_f32(np.full(Dk, s, np.float32), dt))


def rope_inv_freq(base, dims, freqs=None) -> np.ndarray:
    inv = np.empty(dims // 2, np.float32)
    f = None if freqs is None else np.ascontiguousarray(freqs, np.float32)
    lib().or_rope_inv_freq(base, dims, _p(f), _p(inv))
    return inv


def llama3_freqs(base, dims, factor, low, high, original_max_pos) -> np.ndarray:
    f = np.empty(dims // 2, np.float32)
    lib().or_llama3_freqs(base, dims, factor, low, high, original_max_pos, _p(f))
    return f


TRIG_LIBM, TRIG_F64 = 0, 1


def norm_rope(x, x_dt, *, dims, inv_freq, scale=1.0, offset=0, offsets=None,
              norm_w=None, w_dt=None, eps=1e-6, out=None, out_strides=None, trig=TRIG_LIBM):
    """x: 4-D storage array viewed as [B, L, H, D] (any element strides with a
    unit stride on D). Returns y, by default a contiguous [B, L, H, D] array;
    pass ``out``/``out_strides`` (elements, for b/l/h) for other layouts.
    trig: TRIG_LIBM takes cos/sin from libm's f32 cosf/sinf (MLX's CPU rope),
    TRIG_F64 the f32 rounding of f64 cos/sin of the same angle (the device's
    evaluation)."""
    B, L, H, D = x.shape
    assert x.strides[3] == x.itemsize
    t = promote(x_dt, w_dt) if norm_w is not None else x_dt
    xs = np.array([s // x.itemsize for s in x.strides[:3]], np.int64)
    if out is None:
        out = np.zeros((B, L, H, D), storage_dtype(t))
        ys = np.array([L * H * D, H * D, D], np.int64)
    else:
        ys = np.array(out_strides, np.int64)
    inv = np.ascontiguousarray(inv_freq, np.float32)
    offs = None if offsets is None else np.ascontiguousarray(offsets, np.int32)
    base_ptr = x.__array_interface__["data"][0]
    _check(lib().or_norm_rope_trig(x_dt, C.c_void_p(base_ptr), _p(xs), _p(out), _p(ys),
                                   B, L, H, D, _p(norm_w), 0 if w_dt is None else w_dt,
                                   eps, dims, _p(inv), scale, offset, _p(offs), trig),
           "norm_rope")
    return out


def glu(act, gate, up, x_dt, *, out_dt=None):
    rows, n = gate.shape
    out_dt = x_dt if out_dt is None else out_dt
    o = np.empty((rows, n), storage_dtype(out_dt))
    g_ptr = gate.__array_interface__["data"][0]
    u_ptr = up.__array_interface__["data"][0]
    _check(lib().or_glu(act, x_dt, C.c_void_p(g_ptr), gate.strides[0] // gate.itemsize,
                        C.c_void_p(u_ptr), up.strides[0] // up.itemsize, _p(o), out_dt,
                        n, rows, n), "glu")
    return o


def gated_rms_norm(y, z, x_dt, w, w_dt, eps, *, out_dt=None):
    rows, n = y.shape
    t_n = promote(x_dt, w_dt)
    out_dt = promote(x_dt, t_n) if out_dt is None else out_dt
    o = np.empty((rows, n), storage_dtype(out_dt))
    z_ptr = z.__array_interface__["data"][0]
    _check(lib().or_gated_rms_norm(x_dt, _p(y), y.strides[0] // y.itemsize,
                                   C.c_void_p(z_ptr), z.strides[0] // z.itemsize,
                                   _p(w), w_dt, eps, _p(o), out_dt, n, rows, n),
           "gated_rms_norm")
    return o


def qembed(ids_arr, wq, scales, biases, s_dt, *, group=64, bits=4, out_scale=0.0):
    ids_arr = np.ascontiguousarray(ids_arr)
    id_dt = I32 if ids_arr.dtype == np.int32 else U32
    V, wpr = wq.shape
    H = wpr * 8
    out = np.empty((ids_arr.size, H), storage_dtype(s_dt))
    _check(lib().or_qembed(_p(ids_arr), id_dt, ids_arr.size, _p(wq), _p(scales),
                           _p(biases), s_dt, V, H, group, bits, out_scale, _p(out)),
           "qembed")
    return out.reshape(ids_arr.shape + (H,))
