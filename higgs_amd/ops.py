"""Host-side mirror of the mlx-rs calls higgs-models makes on this path, over
the C ABI of libhiggs_hip.so. torch supplies device memory and the stream only.

Each function keeps the reference call's name and argument meaning:

    rms_norm(x, weight, eps)                 mlx_rs::fast::rms_norm / nn::RmsNorm
    rope(x, dims, traditional, base, scale, offset, freqs)
                                             mlx_rs::fast::rope (utils.rs:16-26)
    qk_norm_rope(...)                        q_norm/k_norm + transpose + apply_rope
                                             (transformer.rs:264-287)
    swiglu(gate, x)                          qwen3_next.rs:275-277
    silu_mul(gate, up)                       nn::silu(gate) * up (transformer.rs:349-353)
    gelu_approximate_mul(gate, up)           nn::gelu_approximate(gate) * up (gemma2.rs:422-427)
    gated_rms_norm(x, z, weight, eps)        swiglu(z, norm(x)) (qwen3_next.rs:1204-1205)
    add_rms_norm(x, r, weight, eps)          h = x.add(r); norm(h) (transformer.rs:413-415)
    QuantizedEmbedding(...).forward(ids)     nn::QuantizedEmbedding / QEmbedding::forward
    gather_qmm(x, w, scales, biases, rhs_indices)   qwen3_next.rs:294-363, 844-904
    gated_delta(q, k, v, a_log, a, dt_bias, b, state)
                                             qwen3_next.rs:376-451, 1152-1201
    QuantizedEmbedding(...).forward_rms_norm(ids, w, eps)
                                             embed_tokens + the first input_layernorm
                                             (transformer.rs:494, 407)
    OpSequence                               a decode step's per-layer ops in one launch
                                             (the layer loop, qwen3_next.rs:1508-1547)

Errors surface as HgkError (the reference returns Err(Exception::custom(..))).
Every op enqueues on torch's current CUDA/HIP stream and never synchronises.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Sequence

import torch

from ._lib import (ACT_GELU_TANH, ACT_SILU, BF16, F16, F32, I32, OP_ADD_RMS_NORM, OP_GATED_RMS_NORM,
                   OP_GLU, OP_QK_NORM_ROPE, OP_RMS_NORM, U32, HgkError, HgkOp, check, f32_array,
                   i64_array, lib)

_DT = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16, torch.int32: I32}
if hasattr(torch, "uint32"):
    _DT[torch.uint32] = U32
_TORCH = {F32: torch.float32, BF16: torch.bfloat16, F16: torch.float16}


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DT[t]
    except KeyError:
        raise HgkError(1, f"unsupported dtype {t}") from None


def _promote(a: int, b: int) -> int:
    return a if a == b else F32


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else C.c_void_p(t.data_ptr())


def _stream(device: torch.device):
    return C.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _rows2d(x: torch.Tensor):
    """View x as [rows, n] with unit stride on n; returns (rows, n, row_stride)."""
    if x.dim() == 0:
        raise HgkError(1, "expected at least 1 dimension")
    n = x.shape[-1]
    if n > 1 and x.stride(-1) != 1:
        raise HgkError(1, "last axis must be unit-stride")
    if x.dim() == 1:
        return 1, n, n
    try:
        x2 = x.view(-1, n)
    except RuntimeError:
        raise HgkError(1, "leading axes must collapse to a single row stride") from None
    return x2.shape[0], n, x2.stride(0)


# ---------------------------------------------------------------- RMSNorm
def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float, *,
             plus_one: bool = False, out_dtype: Optional[torch.dtype] = None,
             out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fast::rms_norm(x, weight, eps) over the last axis. ``plus_one`` applies
    Gemma's (1 + weight) in f32 (the reference bakes it into the weight at load
    time, gemma2.rs:799-826). The default output dtype is MLX's promotion of x
    and the effective weight."""
    xd = dtype_code(x.dtype)
    wd = dtype_code(weight.dtype) if weight is not None else xd
    w_eff = (F32 if plus_one else wd) if weight is not None else xd
    od = dtype_code(out_dtype) if out_dtype is not None else _promote(xd, w_eff)
    rows, n, xs = _rows2d(x)
    if weight is not None and (weight.dim() != 1 or weight.shape[0] != n):
        raise HgkError(1, f"weight shape {tuple(weight.shape)} does not match ({n},)")
    if out is None:
        out = torch.empty(x.shape, dtype=_TORCH[od], device=x.device)
    _, _, ys = _rows2d(out)
    check(lib().hgk_rms_norm(_ptr(x), xd, xs, _ptr(weight), wd, int(plus_one), eps,
                             _ptr(out), od, ys, rows, n, _stream(x.device)))
    return out


def add_rms_norm(x: torch.Tensor, r: torch.Tensor, weight: Optional[torch.Tensor], eps: float,
                 *, plus_one: bool = False, out_dtype: Optional[torch.dtype] = None,
                 h_out: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                 write_h: bool = True):
    """The block boundary `h = x.add(residual); norm.forward(&h)`
    (transformer.rs:413-415; qwen3_next.rs:1539-1540) in one pass: returns
    (h, y). Pass ``h_out=x`` to update the residual stream in place;
    ``write_h=False`` skips h (returns None for it)."""
    xd = dtype_code(x.dtype)
    if r.dtype != x.dtype or r.shape != x.shape:
        raise HgkError(1, "x and r must match in shape and dtype")
    wd = dtype_code(weight.dtype) if weight is not None else xd
    w_eff = (F32 if plus_one else wd) if weight is not None else xd
    od = dtype_code(out_dtype) if out_dtype is not None else _promote(xd, w_eff)
    rows, n, xs = _rows2d(x)
    _, _, rs = _rows2d(r)
    if weight is not None and (weight.dim() != 1 or weight.shape[0] != n):
        raise HgkError(1, f"weight shape {tuple(weight.shape)} does not match ({n},)")
    if write_h and h_out is None:
        h_out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    hs = _rows2d(h_out)[2] if h_out is not None else 0
    if out is None:
        out = torch.empty(x.shape, dtype=_TORCH[od], device=x.device)
    _, _, ys = _rows2d(out)
    check(lib().hgk_add_rms_norm(xd, _ptr(x), xs, _ptr(r), rs, _ptr(weight), wd, int(plus_one),
                                 eps, _ptr(h_out), hs, _ptr(out), od, ys, rows, n,
                                 _stream(x.device)))
    return h_out, out


def _z_layout(z: torch.Tensor, rows: int, n: int):
    """(row_stride, group_rows, group_stride) addressing z's rows in place."""
    try:
        zr, zn, zs = _rows2d(z)
        if (zr, zn) == (rows, n):
            return zs, 0, 0
    except HgkError:
        pass
    if z.dim() >= 3 and z.shape[-1] == n and z.stride(-1) == 1:
        try:
            z3 = z.view(-1, z.shape[-2], n)
        except RuntimeError:
            raise HgkError(1, "z layout is not expressible as (groups, rows, n)") from None
        if z3.shape[0] * z3.shape[1] == rows:
            return z3.stride(1), z3.shape[1], z3.stride(0)
    raise HgkError(1, f"z shape {tuple(z.shape)} does not match {rows} rows of {n}")


def gated_rms_norm(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float, *,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """swiglu(z, rms_norm(x, weight, eps)) = z * sigmoid(z) * norm(x).

    z may be a strided view such as the z slice of Qwen3-Next's in_proj_qkvz
    output viewed as [..., v_per_k, head_v_dim]; it is read in place."""
    xd = dtype_code(x.dtype)
    wd = dtype_code(weight.dtype)
    od = _promote(xd, _promote(xd, wd))
    rows, n, xs = _rows2d(x)
    if z.dtype != x.dtype:
        raise HgkError(1, "z must have x's dtype")
    zs, zg, zgs = _z_layout(z, rows, n)
    if out is None:
        out = torch.empty(x.shape, dtype=_TORCH[od], device=x.device)
    _, _, os_ = _rows2d(out)
    check(lib().hgk_gated_rms_norm(xd, _ptr(x), xs, _ptr(z), zs, zg, zgs, _ptr(weight), wd,
                                   eps, _ptr(out), od, os_, rows, n, _stream(x.device)))
    return out


# ---------------------------------------------------------------- RoPE
def rope_inv_freq(base: float, dims: int, freqs: Optional[Sequence[float]] = None):
    inv = (C.c_float * (dims // 2))()
    fr = None if freqs is None else f32_array(list(freqs))
    check(lib().hgk_rope_inv_freq(base, dims, fr, inv))
    return list(inv)


def llama3_rope_freqs(base: float, dims: int, factor: float, low_freq_factor: float,
                      high_freq_factor: float, original_max_position: float):
    """mlx-lm Llama3RoPE frequency table (pass as ``freqs`` to rope)."""
    f = (C.c_float * (dims // 2))()
    check(lib().hgk_llama3_rope_freqs(base, dims, factor, low_freq_factor, high_freq_factor,
                                      original_max_position, f))
    return list(f)


def _freqs_arg(freqs):
    if freqs is None:
        return None
    if isinstance(freqs, torch.Tensor):
        freqs = freqs.detach().to("cpu", torch.float32).tolist()
    return f32_array(list(freqs))


def _offsets_arg(offsets, batch, device):
    if offsets is None:
        return None, None
    if not isinstance(offsets, torch.Tensor):
        offsets = torch.tensor(list(offsets), dtype=torch.int32, device=device)
    if offsets.dtype != torch.int32 or offsets.device != device or offsets.numel() != batch:
        raise HgkError(1, f"offsets must be int32[{batch}] on {device}")
    offsets = offsets.contiguous()
    return offsets, _ptr(offsets)


def rope(x: torch.Tensor, dims: int, traditional: bool = False, base: Optional[float] = 10000.0,
         scale: float = 1.0, offset: int = 0, freqs=None, *, offsets=None,
         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fast::rope(x, dims, traditional, base, scale, offset, freqs).

    x is [..., L, D] with positions along axis -2, as MLX's rope; leading axes
    are flattened to [N, ...]. For 4-D x [B, H, L, D] (the reference's
    post-transpose layout), ``offsets`` (int32[B]) gives each sequence its own
    offset, replacing forward_batched's per-request loop."""
    if (freqs is None) == (base is None):
        raise HgkError(1, "exactly one of base and freqs must be given")
    if x.dim() < 3:
        raise HgkError(1, "rope expects at least 3 dimensions")
    D, L = x.shape[-1], x.shape[-2]
    if x.dim() == 3:
        B, H = x.shape[0], 1
        xs = (x.stride(0), x.stride(1), 0)
    else:
        xv = x.reshape(-1, x.shape[-3], L, D) if x.dim() > 4 else x
        B, H = xv.shape[0], xv.shape[1]
        xs = (xv.stride(0), xv.stride(2), xv.stride(1))
        x = xv
    if out is None:
        out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if out.dim() == 3:
        ys = (out.stride(0), out.stride(1), 0)
    else:
        ys = (out.stride(0), out.stride(2), out.stride(1))
    offs, offs_p = _offsets_arg(offsets, B, x.device)
    check(lib().hgk_rope(dtype_code(x.dtype), _ptr(x), i64_array(xs), _ptr(out), i64_array(ys),
                         B, L, H, D, dims, int(traditional), float(base or 0.0), scale,
                         _freqs_arg(freqs), offset, offs_p, _stream(x.device)))
    return out


def qk_norm_rope(q: torch.Tensor, k: Optional[torch.Tensor], q_norm_w: Optional[torch.Tensor],
                 k_norm_w: Optional[torch.Tensor], eps: float, dims: int, base: float = 10000.0,
                 scale: float = 1.0, offset: int = 0, freqs=None, *, offsets=None,
                 q_out: Optional[torch.Tensor] = None,
                 k_out: Optional[torch.Tensor] = None):
    """Per-head RMSNorm + RoPE for q [B, L, Hq, D] and k [B, L, Hk, D] (the
    projection layout, any strides with unit D stride). Outputs default to the
    reference's post-transpose [B, H, L, D] contiguous layout."""
    B, L, Hq, D = q.shape
    wd = dtype_code(q_norm_w.dtype if q_norm_w is not None else
                    (k_norm_w.dtype if k_norm_w is not None else q.dtype))
    if q_out is None:
        q_out = torch.empty((B, Hq, L, D), dtype=q.dtype, device=q.device)
    qos = (q_out.stride(0), q_out.stride(2), q_out.stride(1))
    Hk = 0
    ks = kos = (0, 0, 0)
    if k is not None:
        Hk = k.shape[2]
        if k_out is None:
            k_out = torch.empty((B, Hk, L, D), dtype=k.dtype, device=k.device)
        ks = (k.stride(0), k.stride(1), k.stride(2))
        kos = (k_out.stride(0), k_out.stride(2), k_out.stride(1))
    offs, offs_p = _offsets_arg(offsets, B, q.device)
    qs = (q.stride(0), q.stride(1), q.stride(2))
    check(lib().hgk_qk_norm_rope(
        dtype_code(q.dtype), _ptr(q), i64_array(qs), _ptr(q_out), i64_array(qos), Hq,
        _ptr(q_norm_w), _ptr(k), i64_array(ks), _ptr(k_out), i64_array(kos), Hk,
        _ptr(k_norm_w), wd, eps, B, L, D, dims, float(base or 0.0), scale,
        _freqs_arg(freqs), offset, offs_p, _stream(q.device)))
    return q_out, k_out


# ---------------------------------------------------------------- GLU
def _glu(act: int, gate: torch.Tensor, up: torch.Tensor, out_dtype, out):
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise HgkError(1, "gate and up must match in shape and dtype")
    xd = dtype_code(gate.dtype)
    od = dtype_code(out_dtype) if out_dtype is not None else xd
    rows, n, gs = _rows2d(gate)
    _, _, us = _rows2d(up)
    if out is None:
        out = torch.empty(gate.shape, dtype=_TORCH[od], device=gate.device)
    _, _, os_ = _rows2d(out)
    check(lib().hgk_glu(act, xd, _ptr(gate), gs, _ptr(up), us, _ptr(out), od, os_, rows, n,
                        _stream(gate.device)))
    return out


def silu_mul(gate, up, *, out_dtype=None, out=None):
    """nn::silu(gate) * up (transformer.rs:349-353)."""
    return _glu(ACT_SILU, gate, up, out_dtype, out)


def swiglu(gate, x, *, out=None):
    """swiglu(gate, x) = gate * sigmoid(gate) * x (qwen3_next.rs:275-277)."""
    return _glu(ACT_SILU, gate, x, None, out)


def gelu_approximate_mul(gate, up, *, out_dtype=None, out=None):
    """nn::gelu_approximate(gate) * up (gemma2.rs:422-427)."""
    return _glu(ACT_GELU_TANH, gate, up, out_dtype, out)


def fused_gate_up_swiglu(gate_up: torch.Tensor, *, out=None):
    """phi3-style fused projection [.., 2I]: silu(first half) * second half
    (phi3.rs:261-265), read in place through row strides."""
    I2 = gate_up.shape[-1]
    return _glu(ACT_SILU, gate_up[..., : I2 // 2], gate_up[..., I2 // 2:], None, out)


# ---------------------------------------------------------------- gather_qmm
def gather_qmm(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               rhs_indices: torch.Tensor, transpose: bool = True, group_size: int = 64,
               bits: int = 4, *, x_row_div: int = 1, lhs_indices: Optional[torch.Tensor] = None,
               out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gather_qmm(x, w, scales, biases, rhs_indices, transpose, group_size, bits)
    as SwitchMlpWeights::forward_gather uses it (qwen3_next.rs:844-904): one
    row of x per (token, expert) pair. x is [R, K]; w [E, N, K*bits/32] packed
    32-bit words; rhs_indices [P] expert per pair; pair p reads x row
    lhs_indices[p], or p // x_row_div (x_row_div = top_k broadcasts a token
    over its experts). Returns y [P, N] in x's dtype."""
    if not transpose:
        raise HgkError(2, "gather_qmm: only transpose=True (weights stored [N, K]) is implemented")
    if x.dim() != 2 or x.stride(-1) != 1:
        raise HgkError(1, "x must be [rows, K] with a unit-stride last axis")
    if w.dim() != 3 or scales.dim() != 3 or scales.shape != biases.shape:
        raise HgkError(1, "w must be [E, N, K/8]; scales and biases [E, N, K/group]")
    if scales.dtype != biases.dtype:
        raise HgkError(1, "scales and biases must share a dtype")
    E, N = w.shape[0], w.shape[1]
    K = x.shape[1]
    P = rhs_indices.numel()
    idx = rhs_indices.reshape(-1).contiguous()
    lhs = None if lhs_indices is None else lhs_indices.reshape(-1).contiguous()
    if out is None:
        out = torch.empty((P, N), dtype=x.dtype, device=x.device)
    check(lib().hgk_gather_qmm(dtype_code(x.dtype), _ptr(x), x.shape[0], x.stride(0), x_row_div,
                               _ptr(lhs), _ptr(w.contiguous()), _ptr(scales.contiguous()),
                               _ptr(biases.contiguous()), dtype_code(scales.dtype), E, N, K,
                               group_size, bits, _ptr(idx), dtype_code(idx.dtype), P, _ptr(out),
                               out.stride(0), _stream(x.device)))
    return out


def gather_qmm_swiglu(x: torch.Tensor, w_gate: torch.Tensor, scales_gate: torch.Tensor,
                      biases_gate: torch.Tensor, w_up: torch.Tensor, scales_up: torch.Tensor,
                      biases_up: torch.Tensor, rhs_indices: torch.Tensor, group_size: int = 64,
                      bits: int = 4, *, x_row_div: int = 1,
                      lhs_indices: Optional[torch.Tensor] = None,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """swiglu(gather_qmm(x, gate...), gather_qmm(x, up...)) -- the gate/up half of
    SwitchMlpWeights::forward_gather (qwen3_next.rs:862-886) -- in one launch
    where a fused kernel applies (the per-pair decode kernel, or the grouped
    matrix-core kernel's fused form at 16 or more pairs per expert), else as
    the three calls. Returns [P, N] in x's dtype."""
    E, N = w_gate.shape[0], w_gate.shape[1]
    K = x.shape[1]
    idx = rhs_indices.reshape(-1).contiguous()
    P = idx.numel()
    lhs = None if lhs_indices is None else lhs_indices.reshape(-1).contiguous()
    if out is None:
        out = torch.empty((P, N), dtype=x.dtype, device=x.device)
    if w_up.shape != w_gate.shape or scales_up.shape != scales_gate.shape:
        raise HgkError(1, "gate and up weights must have the same shapes")
    for name, t in (("biases_gate", biases_gate), ("scales_up", scales_up), ("biases_up", biases_up)):
        # one scales dtype reaches the kernel for both projections
        if t.dtype != scales_gate.dtype:
            raise HgkError(1, f"{name} dtype {t.dtype} differs from scales_gate's {scales_gate.dtype}")
    st = lib().hgk_gather_qmm_swiglu(
        dtype_code(x.dtype), _ptr(x), x.shape[0], x.stride(0), x_row_div, _ptr(lhs),
        _ptr(w_gate.contiguous()), _ptr(scales_gate.contiguous()), _ptr(biases_gate.contiguous()),
        _ptr(w_up.contiguous()), _ptr(scales_up.contiguous()), _ptr(biases_up.contiguous()),
        dtype_code(scales_gate.dtype), E, N, K, group_size, bits, _ptr(idx),
        dtype_code(idx.dtype), P, _ptr(out), out.stride(0), _stream(x.device))
    if st == 2:  # not the fused kernel's regime: the reference's three calls
        g = gather_qmm(x, w_gate, scales_gate, biases_gate, idx, True, group_size, bits,
                       x_row_div=x_row_div, lhs_indices=lhs)
        u = gather_qmm(x, w_up, scales_up, biases_up, idx, True, group_size, bits,
                       x_row_div=x_row_div, lhs_indices=lhs)
        return swiglu(g, u, out=out)
    check(st)
    return out


def quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                     biases: torch.Tensor, transpose: bool = True, group_size: int = 64,
                     bits: int = 4, *, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """quantized_matmul(x, w, scales, biases, transpose, group_size, bits) as
    QLinear::forward calls it (qwen3_next.rs:174-221): x [..., K], w [N,
    K*bits/32] packed 32-bit words, scales/biases [N, K/group_size]. Returns
    y [..., N] in x's dtype. M >= 16 rows in bf16 with group 64 run on the
    matrix cores; fewer rows, f16 or other groups run one GEMV per row."""
    if not transpose:
        raise HgkError(2, "quantized_matmul: only transpose=True (weights stored [N, K]) is implemented")
    if w.dim() != 2 or scales.dim() != 2 or scales.shape != biases.shape:
        raise HgkError(1, "w must be [N, K/8]; scales and biases [N, K/group]")
    if scales.dtype != biases.dtype:
        raise HgkError(1, "scales and biases must share a dtype")
    K = x.shape[-1]
    N = w.shape[0]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    M = x2.shape[0]
    if out is None:
        out = torch.empty((*lead, N), dtype=x.dtype, device=x.device)
    o2 = out.view(-1, N)
    check(lib().hgk_quantized_matmul(dtype_code(x.dtype), _ptr(x2), M, x2.stride(0) if M else K,
                                     _ptr(w.contiguous()), _ptr(scales.contiguous()),
                                     _ptr(biases.contiguous()), dtype_code(scales.dtype), N, K,
                                     group_size, bits, _ptr(o2), o2.stride(0) if M else N,
                                     _stream(x.device)))
    return out


# ---------------------------------------------------------------- GatedDeltaNet
def gdn_qk_norm_weights(head_k_dim: int, dtype: torch.dtype, device):
    """GatedDeltaNet's constant q/k norm weights (qwen3_next.rs:1075-1094, cast to the input dtype at 1165-1169):
    s = 1/sqrt(Dk) in f32; q's weight is s*s, k's is s, cast to `dtype`."""
    s = torch.tensor(1.0, dtype=torch.float32) / torch.sqrt(torch.tensor(float(head_k_dim)))
    wq = torch.full((head_k_dim,), float(s * s), dtype=torch.float32).to(dtype)
    wk = torch.full((head_k_dim,), float(s), dtype=torch.float32).to(dtype)
    return wq.to(device), wk.to(device)


def gated_delta(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, a_log: torch.Tensor,
                a: torch.Tensor, dt_bias: torch.Tensor, b: torch.Tensor,
                state: Optional[torch.Tensor] = None, *, q_norm_w: Optional[torch.Tensor] = None,
                k_norm_w: Optional[torch.Tensor] = None, eps: float = 1e-6,
                state_out: Optional[torch.Tensor] = None):
    """The gated-delta recurrence (gated_delta_kernel_ffi, qwen3_next.rs:376-451)
    with the optional constant-weight q/k RMSNorm fused in: q, k [B, T, Hk, Dk],
    v [B, T, Hv, Dv], a, b [B, T, Hv], a_log, dt_bias [Hv], state [B, Hv, Dv, Dk]
    or None (zeros). Returns (y [B, T, Hv, Dv], new_state)."""
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    for t in (q, k, v, a, b):
        if not t.is_contiguous() or t.dtype != q.dtype:
            raise HgkError(1, "q, k, v, a, b must be contiguous and share a dtype")
    if a_log.dtype != dt_bias.dtype:
        raise HgkError(1, "a_log and dt_bias must share a dtype")
    y = torch.empty((B, T, Hv, Dv), dtype=q.dtype, device=q.device)
    if state_out is None:
        state_out = torch.empty((B, Hv, Dv, Dk), dtype=q.dtype, device=q.device)
    check(lib().hgk_gated_delta(dtype_code(q.dtype), _ptr(q), _ptr(k), _ptr(v),
                                _ptr(a_log.contiguous()), _ptr(a), _ptr(dt_bias.contiguous()),
                                _ptr(b), dtype_code(a_log.dtype),
                                None if state is None else _ptr(state.contiguous()),
                                _ptr(q_norm_w), _ptr(k_norm_w), eps, B, T, Hk, Dk, Hv, Dv,
                                _ptr(y), _ptr(state_out), _stream(q.device)))
    return y, state_out


def gated_delta_gated_norm(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           a_log: torch.Tensor, a: torch.Tensor, dt_bias: torch.Tensor,
                           b: torch.Tensor, state: Optional[torch.Tensor], z: torch.Tensor,
                           norm_weight: torch.Tensor, norm_eps: float, *,
                           q_norm_w: Optional[torch.Tensor] = None,
                           k_norm_w: Optional[torch.Tensor] = None, eps: float = 1e-6,
                           state_out: Optional[torch.Tensor] = None,
                           out: Optional[torch.Tensor] = None):
    """One decode token of GatedDeltaNet from the recurrence through its gated
    output norm (qwen3_next.rs:1185-1205): swiglu(z, norm(gated_delta(...).y))
    in one launch where it applies, else as the two calls. q, k [B, 1, Hk, Dk],
    v [B, 1, Hv, Dv], a, b [B, 1, Hv]; z [B, 1, Hv, Dv] (may be a strided view
    of in_proj_qkvz). Returns (out [B, 1, Hv, Dv], new_state)."""
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    if T != 1:
        raise HgkError(1, "gated_delta_gated_norm is the one-token (decode) form")
    for t in (q, k, v, a, b):
        if not t.is_contiguous() or t.dtype != q.dtype:
            raise HgkError(1, "q, k, v, a, b must be contiguous and share a dtype")
    if a_log.dtype != dt_bias.dtype:
        raise HgkError(1, "a_log and dt_bias must share a dtype")
    if state_out is None:
        state_out = torch.empty((B, Hv, Dv, Dk), dtype=q.dtype, device=q.device)
    if out is None:
        out = torch.empty((B, T, Hv, Dv), dtype=q.dtype, device=q.device)
    zs, zg, zgs = _z_layout(z, B * Hv, Dv)
    st = lib().hgk_gated_delta_gated_norm(
        dtype_code(q.dtype), _ptr(q), _ptr(k), _ptr(v), _ptr(a_log.contiguous()), _ptr(a),
        _ptr(dt_bias.contiguous()), _ptr(b), dtype_code(a_log.dtype),
        None if state is None else _ptr(state.contiguous()), _ptr(q_norm_w), _ptr(k_norm_w), eps,
        B, Hk, Dk, Hv, Dv, _ptr(state_out), None, _ptr(z), zs, zg, zgs, _ptr(norm_weight),
        dtype_code(norm_weight.dtype), norm_eps, _ptr(out), _stream(q.device))
    if st == 2:  # outside the fused form: the reference's two calls
        y, state_out = gated_delta(q, k, v, a_log, a, dt_bias, b, state, q_norm_w=q_norm_w,
                                   k_norm_w=k_norm_w, eps=eps, state_out=state_out)
        gated_rms_norm(y, z, norm_weight, norm_eps, out=out)
        return out, state_out
    check(st)
    return out, state_out


# ---------------------------------------------------------------- embedding
class QuantizedEmbedding:
    """nn::QuantizedEmbedding: 4-bit affine table (weight u32 [V, H/8], scales
    and biases [V, H/group] in bf16/f16). forward(ids) gathers and
    dequantizes only the requested rows; out_scale applies Gemma's
    bf16(sqrt(H)) embedding scale in the same pass (gemma2.rs:587-600)."""

    def __init__(self, weight: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
                 group_size: int = 64, bits: int = 4):
        if weight.dtype not in (torch.int32, getattr(torch, "uint32", torch.int32)):
            raise HgkError(1, "weight must hold packed 32-bit words")
        self.weight, self.scales, self.biases = weight, scales, biases
        self.group_size, self.bits = group_size, bits
        self.vocab = weight.shape[0]
        self.hidden = weight.shape[1] * 32 // bits

    def forward(self, ids: torch.Tensor, *, out_scale: float = 0.0,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
        idd = dtype_code(ids.dtype)
        sd = dtype_code(self.scales.dtype)
        flat = ids.reshape(-1).contiguous()
        if out is None:
            out = torch.empty((flat.numel(), self.hidden), dtype=_TORCH[sd], device=ids.device)
        check(lib().hgk_quantized_embedding(
            _ptr(flat), idd, flat.numel(), _ptr(self.weight), _ptr(self.scales),
            _ptr(self.biases), sd, self.vocab, self.hidden, self.group_size, self.bits,
            out_scale, _ptr(out), out.stride(0), _stream(ids.device)))
        return out.reshape(*ids.shape, self.hidden)

    __call__ = forward

    def forward_rms_norm(self, ids: torch.Tensor, weight: torch.Tensor, eps: float, *,
                         plus_one: bool = False, out_scale: float = 0.0,
                         out_dtype: Optional[torch.dtype] = None, write_h: bool = True):
        """forward(ids) followed by the first block's input RMSNorm, in one
        pass: returns (h, y), both [*ids.shape, hidden]; h is None when
        ``write_h`` is False."""
        idd = dtype_code(ids.dtype)
        sd = dtype_code(self.scales.dtype)
        wd = dtype_code(weight.dtype)
        w_eff = F32 if plus_one else wd
        od = dtype_code(out_dtype) if out_dtype is not None else _promote(sd, w_eff)
        flat = ids.reshape(-1).contiguous()
        T = flat.numel()
        h = (torch.empty((T, self.hidden), dtype=_TORCH[sd], device=ids.device)
             if write_h else None)
        y = torch.empty((T, self.hidden), dtype=_TORCH[od], device=ids.device)
        check(lib().hgk_quantized_embedding_rms_norm(
            _ptr(flat), idd, T, _ptr(self.weight), _ptr(self.scales), _ptr(self.biases), sd,
            self.vocab, self.hidden, self.group_size, self.bits, out_scale, _ptr(h),
            self.hidden, _ptr(weight), wd, int(plus_one), eps, _ptr(y), od, self.hidden,
            _stream(ids.device)))
        shape = (*ids.shape, self.hidden)
        return (None if h is None else h.reshape(shape)), y.reshape(shape)


def gemma_embed_scale(hidden: int) -> float:
    """sqrt(hidden) as the reference computes it (f32), before the cast to the
    activation dtype that the kernel applies."""
    return float(math.sqrt(float(hidden)))


# ---------------------------------------------------------------- op sequence
def _tok_rows(t: torch.Tensor, what: str):
    """(rows, n, token stride, row stride) of a [T, n] or [T, rows, n] view
    with a unit-stride last axis."""
    if t.stride(-1) != 1 and t.shape[-1] > 1:
        raise HgkError(1, f"{what}: the last axis must have unit stride")
    if t.dim() == 2:
        return 1, t.shape[1], t.stride(0), t.shape[1]
    if t.dim() == 3:
        return t.shape[1], t.shape[2], t.stride(0), t.stride(1)
    raise HgkError(1, f"{what}: expected [tokens, n] or [tokens, rows, n]")


class OpSequence:
    """A decode step's per-layer ops -- input_layernorm (residual add +
    RMSNorm), the gated RMSNorm or q/k RMSNorm + RoPE, post_attention_layernorm,
    the experts' SwiGLU, layer after layer as the loop of qwen3_next.rs:1508-1547
    calls them -- recorded once, uploaded once, then run over a batch of tokens
    in one launch (hgk_op_list_upload / hgk_op_list_run). Every operand is a
    view whose first axis is the token; the recorded addresses are used at
    every run, so the tensors must stay alive and in place (this object keeps
    references to them). Results are the same bits as the separate calls."""

    def __init__(self, dtype: torch.dtype, device):
        if dtype not in (torch.bfloat16, torch.float16):
            raise HgkError(2, "OpSequence: bf16 or f16 only")
        self.dtype, self.device = dtype, torch.device(device)
        self._ops, self._keep, self._list, self._uploaded = [], [], None, 0

    def _check(self, *ts):
        for t in ts:
            if t is not None and t.dtype != self.dtype:
                raise HgkError(1, f"OpSequence: operand dtype {t.dtype}, list dtype {self.dtype}")
        self._keep.extend(t for t in ts if t is not None)

    def __len__(self):
        return len(self._ops)

    def rms_norm(self, x, weight, eps, y):
        """y = rms_norm(x, weight, eps) (weight may be None)."""
        self._check(x, weight, y)
        rows, n, xt, xr = _tok_rows(x, "x")
        _, _, yt, yr = _tok_rows(y, "y")
        self._ops.append(HgkOp(kind=OP_RMS_NORM, rows=rows, n=n, eps=eps, x=x.data_ptr(), x_tok=xt,
                               x_row=xr, w=None if weight is None else weight.data_ptr(),
                               y=y.data_ptr(), y_tok=yt, y_row=yr))
        return self

    def add_rms_norm(self, x, r, weight, eps, y, h=None):
        """h = x + r (written when h is given); y = rms_norm(h, weight, eps)."""
        self._check(x, r, weight, y, h)
        rows, n, xt, xr = _tok_rows(x, "x")
        _, _, rt, rr = _tok_rows(r, "r")
        _, _, yt, yr = _tok_rows(y, "y")
        ht, hr = (0, 0) if h is None else _tok_rows(h, "h")[2:]
        self._ops.append(HgkOp(kind=OP_ADD_RMS_NORM, rows=rows, n=n, eps=eps, x=x.data_ptr(),
                               x_tok=xt, x_row=xr, r=r.data_ptr(), r_tok=rt, r_row=rr,
                               w=None if weight is None else weight.data_ptr(), y=y.data_ptr(),
                               y_tok=yt, y_row=yr, h=None if h is None else h.data_ptr(),
                               h_tok=ht, h_row=hr))
        return self

    def gated_rms_norm(self, x, z, weight, eps, y):
        """y = swiglu(z, rms_norm(x, weight, eps)). x, y: [T, rows, n]; z:
        [T, rows, n] or [T, groups, rows_per_group, n] (e.g. the z slice of
        in_proj_qkvz, read in place)."""
        self._check(x, z, weight, y)
        rows, n, xt, xr = _tok_rows(x, "x")
        _, _, yt, yr = _tok_rows(y, "y")
        if z.dim() == 4:
            if z.shape[1] * z.shape[2] != rows or z.shape[3] != n or z.stride(3) != 1:
                raise HgkError(1, "z must be [T, groups, rows_per_group, n] covering x's rows")
            zt, zr, zg, zgs = z.stride(0), z.stride(2), z.shape[2], z.stride(1)
        else:
            _, _, zt, zr = _tok_rows(z, "z")
            zg, zgs = 0, 0
        self._ops.append(HgkOp(kind=OP_GATED_RMS_NORM, rows=rows, n=n, eps=eps, x=x.data_ptr(),
                               x_tok=xt, x_row=xr, r=z.data_ptr(), r_tok=zt, r_row=zr,
                               z_group_rows=zg, z_group_stride=zgs, w=weight.data_ptr(),
                               y=y.data_ptr(), y_tok=yt, y_row=yr))
        return self

    def qk_norm_rope(self, q, k, q_weight, k_weight, eps, dims, base, q_out, k_out, *,
                     scale=1.0, offset=0, offsets=None, freqs=None):
        """q/k RMSNorm (weights may be None) and RoPE of one new token per
        sequence at position offsets[t] (or offset) times scale: q [T, Hq, D]
        (a head may sit in a wider block, as Qwen3-Next's q), k [T, Hk, D];
        outputs q_out [T, Hq, D], k_out [T, Hk, D] (any token/head strides)."""
        self._check(q, k, q_weight, k_weight, q_out, k_out)
        hq, D, qt, qr = _tok_rows(q, "q")
        hk, _, kt, kr = _tok_rows(k, "k")
        _, _, yt, yr = _tok_rows(q_out, "q_out")
        _, _, ht, hr = _tok_rows(k_out, "k_out")
        if offsets is not None:
            if offsets.dtype != torch.int32 or offsets.device != q.device:
                raise HgkError(1, "offsets must be int32 on q's device")
            self._keep.append(offsets)
        fr = _freqs_arg(freqs)
        if fr is not None:
            self._keep.append(fr)
        self._ops.append(HgkOp(kind=OP_QK_NORM_ROPE, rows=hq, n=D, eps=eps, x=q.data_ptr(),
                               x_tok=qt, x_row=qr, r=k.data_ptr(), r_tok=kt, r_row=kr,
                               w=None if q_weight is None else q_weight.data_ptr(),
                               w2=None if k_weight is None else k_weight.data_ptr(),
                               y=q_out.data_ptr(), y_tok=yt, y_row=yr, h=k_out.data_ptr(),
                               h_tok=ht, h_row=hr, k_heads=hk, dims=dims,
                               base=0.0 if base is None else base, freqs=fr, scale=scale,
                               offsets=None if offsets is None else offsets.data_ptr(),
                               offset=offset))
        return self

    def glu(self, act, gate, up, y):
        """y = act(gate) * up (ACT_SILU: swiglu; ACT_GELU_TANH: GeGLU)."""
        self._check(gate, up, y)
        rows, n, gt, gr = _tok_rows(gate, "gate")
        _, _, ut, ur = _tok_rows(up, "up")
        _, _, yt, yr = _tok_rows(y, "y")
        self._ops.append(HgkOp(kind=OP_GLU, rows=rows, n=n, act=act, x=gate.data_ptr(), x_tok=gt,
                               x_row=gr, r=up.data_ptr(), r_tok=ut, r_row=ur, y=y.data_ptr(),
                               y_tok=yt, y_row=yr))
        return self

    def upload(self):
        """Writes the recorded ops into a device list (done by run() when
        ops were added since the last upload)."""
        n = len(self._ops)
        if n == 0:
            raise HgkError(1, "OpSequence: no ops")
        nbytes = lib().hgk_op_list_bytes(n)
        if nbytes < 0:
            raise HgkError(1, f"OpSequence: {n} ops is too many")
        self._list = torch.empty(((nbytes + 15) // 16 * 16,), dtype=torch.uint8, device=self.device)
        arr = (HgkOp * n)(*self._ops)
        check(lib().hgk_op_list_upload(dtype_code(self.dtype), arr, n, _ptr(self._list),
                                       self._list.numel(), _stream(self.device)))
        self._uploaded = n
        return self

    def run(self, tokens: int):
        """Every op over tokens 0..tokens-1, in one launch on the current stream."""
        if self._uploaded != len(self._ops):
            self.upload()
        check(lib().hgk_op_list_run(dtype_code(self.dtype), _ptr(self._list), self._uploaded,
                                    tokens, _stream(self.device)))
