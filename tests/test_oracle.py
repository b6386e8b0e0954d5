"""Pins for the CPU oracle (no GPU). Each check compares the oracle with
something it does not compute itself: the reference's own known answers,
numpy/torch float64 mathematics, IEEE conversions done by numpy/torch, closed
forms and invariants. Sizes keep the whole file to a few seconds."""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

import oracle as O
from bits import assert_close, exact_frac, ulp_dist

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bf16_bits_torch(a_f32: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(a_f32, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def from_bf16_bits(b: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(b, np.uint16).view(np.int16)).view(torch.bfloat16)


# ------------------------------------------------------------------ conversions
def test_bf16_rounding_matches_torch():
    x = O.normal(11, (200_000,)) * np.float32(3.0)
    edge = np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.0078125, 3.3895314e38,
                     3.4e38, -3.4e38, 1e-39, -1e-40, 1e-45, np.inf, -np.inf], np.float32)
    # exact halfway cases between neighbouring bf16 values
    halves = (np.arange(1, 2000, dtype=np.uint32) << 16) | 0x8000
    x = np.concatenate([x, edge, halves.view(np.float32)])
    assert np.array_equal(O.from_f32(x, O.BF16), bf16_bits_torch(x))


def test_f16_rounding_matches_numpy():
    x = O.normal(12, (200_000,)) * np.float32(300.0)
    edge = np.array([65504.0, 65519.9, 65520.0, 70000.0, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8,
                     1e-9, -0.0, np.inf], np.float32)
    x = np.concatenate([x, edge, O.normal(13, (10_000,)) * np.float32(1e-5)])
    assert np.array_equal(O.from_f32(x, O.F16), x.astype(np.float16).view(np.uint16))
    back = O.to_f32(x.astype(np.float16).view(np.uint16), O.F16)
    assert np.array_equal(back, x.astype(np.float16).astype(np.float32))


# ------------------------------------------------------------------ MLX math
def test_mlx_exp_accuracy_and_specials():
    L = O.lib()
    xs = np.concatenate([np.linspace(-87.0, 87.9, 40_001), np.linspace(-2, 2, 4001)])
    got = np.array([L.or_mlx_exp(float(v)) for v in xs.astype(np.float32)], np.float64)
    ref = np.exp(xs.astype(np.float32).astype(np.float64))
    rel = np.abs(got - ref) / ref
    # MLX's polynomial exp: the f32 product x*1.442695f carries an absolute
    # error up to ulp(x*log2 e)/2, i.e. ~|x| * 2^-24 * 1.44 relative; near 0 it
    # is within a few f32 ulps. A wrong polynomial coefficient breaks both.
    small = np.abs(xs) <= 2
    assert rel[small].max() < 4 * 2.0 ** -23, rel[small].max()
    bound = 3e-7 + np.abs(xs.astype(np.float32).astype(np.float64)) * 1.5 * 2.0 ** -23
    assert np.all(rel <= bound), (rel / bound).max()
    assert L.or_mlx_exp(0.0) == 1.0
    # 2^int is built in the exponent field, so once int(x*log2 e + 0.5) reaches
    # -127 the result is 0 instead of a subnormal
    assert L.or_mlx_exp(-87.9) == 0.0 and L.or_mlx_exp(-87.5) > 0.0
    assert L.or_mlx_exp(89.0) == math.inf
    assert L.or_mlx_exp(-89.0) == 0.0
    assert math.isnan(L.or_mlx_exp(float("nan")))


def test_mlx_sigmoid_matches_float64():
    L = O.lib()
    xs = np.linspace(-30, 30, 60_001).astype(np.float32)
    got = np.array([L.or_mlx_sigmoid(float(v)) for v in xs], np.float64)
    ref = 1.0 / (1.0 + np.exp(-xs.astype(np.float64)))
    assert np.abs(got - ref).max() < 2e-7
    # relative error in the left tail is exp's (|x| * 1.5 * 2^-23 at most)
    bound = (3e-7 + np.abs(xs.astype(np.float64)) * 1.5 * 2.0 ** -23) * ref + 2.0 ** -25
    assert np.all(np.abs(got - ref) <= bound)
    assert L.or_mlx_sigmoid(0.0) == 0.5


# ------------------------------------------------------------------ SwiGLU
def _glu_f32(act, g, u):
    g = np.ascontiguousarray(g, np.float32).reshape(1, -1)
    u = np.ascontiguousarray(u, np.float32).reshape(1, -1)
    return O.glu(act, g, u, O.F32)[0]


def test_swiglu_reference_known_answers():
    ka = json.load(open(os.path.join(GOLDEN, "reference_known_answers.json")))
    for c in ka["swiglu_numeric_correctness"]["cases"]:
        got = _glu_f32(O.ACT_SILU, [c["gate"]], [c["x"]])[0]
        assert abs(got - c["expected"]) < c["tol"], (c, got)
    s = ka["swiglu_shape"]
    got = _glu_f32(O.ACT_SILU, s["gate"][0], s["x"][0])
    assert got.shape == (3,) and got[0] > s["first_greater_than"]


def test_silu_f32_matches_torch_float64():
    g = O.normal(21, (64, 512)) * np.float32(4)
    u = O.normal(22, (64, 512))
    got = O.glu(O.ACT_SILU, g, u, O.F32)
    ref = (torch.nn.functional.silu(torch.from_numpy(g).double()) * torch.from_numpy(u).double()).numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-7)


def test_gelu_tanh_f32_matches_torch_float64():
    g = O.normal(23, (64, 512)) * np.float32(3)
    u = O.normal(24, (64, 512))
    got = O.glu(O.ACT_GELU_TANH, g, u, O.F32)
    ref = (torch.nn.functional.gelu(torch.from_numpy(g).double(), approximate="tanh") *
           torch.from_numpy(u).double()).numpy()
    # the reference formula 0.5*g*(1+tanh(.)) cancels in f32 for g << 0
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=2e-6)


def test_silu_bf16_rounding_sequence_matches_torch_ops():
    """MLX's composition sig=bf16(sigmoid(g)); s=bf16(g*sig); out=bf16(s*u)
    restated with torch's bf16 ops (each computes in f32 and rounds)."""
    g = O.from_f32(O.normal(25, (256, 512)) * np.float32(3), O.BF16)
    u = O.from_f32(O.normal(26, (256, 512)), O.BF16)
    got = O.glu(O.ACT_SILU, g, u, O.BF16)
    tg, tu = from_bf16_bits(g), from_bf16_bits(u)
    ref = (tg * torch.sigmoid(tg)) * tu
    ref_bits = ref.view(torch.int16).numpy().view(np.uint16)
    # torch's sigmoid uses a different exp: rare one-ulp flips only
    assert exact_frac(got, ref_bits, O.BF16) > 0.999
    assert ulp_dist(got, ref_bits, O.BF16).max() <= 1
    # dropping the intermediate roundings is a different function
    fused = bf16_bits_torch((tg.float() * torch.sigmoid(tg.float()) * tu.float()).numpy())
    assert exact_frac(got, fused, O.BF16) < 0.99


# ------------------------------------------------------------------ RMSNorm
def test_rms_norm_f32_matches_float64():
    x = O.normal(31, (64, 2048))
    w = O.normal(32, (2048,), 1.0, 0.02)
    got = O.rms_norm(x, O.F32, w, O.F32, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * w.astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-5)


def test_rms_norm_constant_row_closed_form():
    for c in (0.5, -3.0, 1e-3):
        x = np.full((3, 512), c, np.float32)
        w = O.normal(33, (512,), 1.0, 0.02)
        got = O.rms_norm(x, O.F32, w, O.F32, 1e-6)
        ref = w.astype(np.float64) * c / math.sqrt(c * c + 1e-6)
        np.testing.assert_allclose(got, np.broadcast_to(ref, got.shape), rtol=4e-7)
    z = O.rms_norm(np.zeros((2, 64), np.float32), O.F32, None, O.F32, 1e-5)
    assert not z.any()


def test_rms_norm_bf16_rounding_sequence_matches_torch_ops():
    """astype(f32) -> x*rsqrt(mean(x^2)+eps) -> astype(bf16) -> * w (bf16)."""
    x = O.from_f32(O.normal(34, (512, 2048)), O.BF16)
    w = O.from_f32(O.normal(35, (2048,), 1.0, 0.02), O.BF16)
    got = O.rms_norm(x, O.BF16, w, O.BF16, 1e-5)
    tx, tw = from_bf16_bits(x), from_bf16_bits(w)
    xf = tx.float()
    r = torch.rsqrt((xf * xf).mean(-1, keepdim=True) + 1e-5)
    ref = ((xf * r).to(torch.bfloat16) * tw).view(torch.int16).numpy().view(np.uint16)
    # torch sums in f32 pairwise: a one-bit change in r can flip the bf16 cast
    # of x*r, which the second rounding (after * w) can widen to 2 ulp
    assert exact_frac(got, ref, O.BF16) > 0.998
    assert ulp_dist(got, ref, O.BF16).max() <= 2
    single = bf16_bits_torch((xf * r * tw.float()).numpy())
    assert exact_frac(got, single, O.BF16) < 0.99  # the cast before * w matters


def test_gemma_plus_one_is_f32_weight_shift():
    x = O.from_f32(O.normal(36, (64, 3584)), O.BF16)
    w = O.from_f32(O.normal(37, (3584,), 0.0, 0.02), O.BF16)
    got = O.rms_norm(x, O.BF16, w, O.BF16, 1e-6, plus_one=True)
    assert got.dtype == np.float32  # promoted by the f32 shift (gemma2.rs:802)
    w1 = O.to_f32(w, O.BF16) + np.float32(1.0)
    same = O.rms_norm(x, O.BF16, w1, O.F32, 1e-6)
    assert np.array_equal(got, same)
    xd = O.to_f32(x, O.BF16).astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-6) * w1.astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-5)


# ------------------------------------------------------------------ RoPE
def _rope_ref64(x, inv, pos):
    """float64 NeoX rotation of x[..., D] at positions pos (broadcast)."""
    half = inv.size
    th = pos[..., None].astype(np.float64) * inv.astype(np.float64)
    c, s = np.cos(th), np.sin(th)
    x1, x2 = x[..., :half].astype(np.float64), x[..., half:2 * half].astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c, x[..., 2 * half:]], -1)


def test_default_inv_freq_matches_closed_form():
    for base, dims in ((500000.0, 64), (1e6, 128), (1e4, 256), (1e7, 64)):
        inv = O.rope_inv_freq(base, dims)
        ref = base ** (-np.arange(dims // 2) / (dims / 2))
        # MLX's polynomial exp of arguments down to -ln(base) (~-16)
        np.testing.assert_allclose(inv, ref, rtol=4e-6)
        assert inv[0] == 1.0


def test_llama3_freq_bands():
    f = O.llama3_freqs(500000.0, 64, 32.0, 1.0, 4.0, 8192.0)
    e = np.arange(0, 64, 2, dtype=np.float32) / np.float32(64)
    plain = np.array([np.float32(500000.0) ** v for v in e], np.float32)
    wl = 2 * np.pi * plain.astype(np.float64)
    hi = wl < 2048            # high-frequency band: unchanged
    lo = wl > 8192            # low-frequency band: exactly x factor
    mid = ~hi & ~lo
    assert hi[:15].all() and lo[18:].all() and mid[15:18].all()
    np.testing.assert_allclose(f[hi], plain[hi], rtol=2e-7)
    np.testing.assert_allclose(f[lo], plain[lo] * 32.0, rtol=2e-7)
    sm = (8192.0 / wl[mid] - 1.0) / 3.0
    np.testing.assert_allclose(f[mid], plain[mid] / ((1 - sm) / 32.0 + sm), rtol=1e-5)


def test_rope_f32_matches_float64_and_invariants():
    B, L, H, D = 2, 33, 3, 128
    x = O.normal(41, (B, L, H, D))
    inv = O.rope_inv_freq(1e6, D)
    y = O.norm_rope(x, O.F32, dims=D, inv_freq=inv, offset=5)
    pos = (np.arange(L) + 5.0)[None, :, None]
    ref = _rope_ref64(x, inv, np.broadcast_to(pos, (B, L, H)))
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=2e-5)
    # the rotation preserves each (x1_i, x2_i) pair's norm
    h = D // 2
    n0 = x[..., :h].astype(np.float64) ** 2 + x[..., h:].astype(np.float64) ** 2
    n1 = y[..., :h].astype(np.float64) ** 2 + y[..., h:].astype(np.float64) ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)


ROPE_TRIG_CASES = [
    # base (None: llama3 freqs), dims, positions (range or sampled offsets)
    (None, 64, np.arange(0, 1024)),                          # Llama-3.2-1B, llama3 scaling
    (1e6, 128, np.arange(0, 2048)),                          # Qwen3-8B
    (1e4, 256, np.arange(0, 4096)),                          # Gemma-2-9B
    (1e7, 64, np.arange(1, 32769)),                          # Qwen3-Next offsets
]


@pytest.mark.parametrize("case", ROPE_TRIG_CASES, ids=lambda c: f"dims{c[1]}-n{len(c[2])}")
def test_rope_trig_modes_pinned_to_float64(case):
    """The oracle's two cos/sin evaluations, read back exactly through an f32
    rotation of x = (1, 0) pairs (y1 = c, y2 = s), at the configurations'
    positions: the f64 mode is bit for bit the f32 rounding of torch's float64
    cos/sin of the f32 angle (f32(position) times the f32 inverse frequency),
    and the libm mode lies within one f32 ulp of it."""
    base, dims, pos = case
    if base is None:
        inv = O.rope_inv_freq(0.0, dims, O.llama3_freqs(500000.0, dims, 32.0, 1.0, 4.0, 8192.0))
    else:
        inv = O.rope_inv_freq(base, dims)
    half = dims // 2
    n = len(pos)
    x = np.zeros((n, 1, 1, dims), np.float32)  # one sequence per position
    x[..., :half] = 1.0
    offs = pos.astype(np.int32)
    th = torch.from_numpy(pos.astype(np.float32))[:, None] * torch.from_numpy(inv)[None, :]
    want_c = torch.cos(th.double()).float().numpy()
    want_s = torch.sin(th.double()).float().numpy()
    y64 = O.norm_rope(x, O.F32, dims=dims, inv_freq=inv, offsets=offs, trig=O.TRIG_F64)
    assert np.array_equal(y64[:, 0, 0, :half], want_c)
    assert np.array_equal(y64[:, 0, 0, half:], want_s)
    ylm = O.norm_rope(x, O.F32, dims=dims, inv_freq=inv, offsets=offs, trig=O.TRIG_LIBM)
    assert ulp_dist(ylm, y64, O.F32).max() <= 1


def test_rope_position_zero_is_identity_bitexact():
    for dt in (O.BF16, O.F32):
        x = O.from_f32(O.normal(42, (1, 1, 8, 64)), dt)
        y = O.norm_rope(x, dt, dims=64, inv_freq=O.rope_inv_freq(1e4, 64))
        assert np.array_equal(y, x)


def test_rope_offset_shift_invariance_and_per_sequence_offsets():
    D, p = 64, 37
    inv = O.rope_inv_freq(500000.0, D)
    x = O.from_f32(O.normal(43, (1, p + 1, 4, D)), O.BF16)
    full = O.norm_rope(x, O.BF16, dims=D, inv_freq=inv)
    last = O.norm_rope(np.ascontiguousarray(x[:, p:]), O.BF16, dims=D, inv_freq=inv, offset=p)
    assert np.array_equal(full[:, p:], last)
    # per-sequence offsets equal separate scalar-offset calls (forward_batched loop)
    xb = O.from_f32(O.normal(44, (5, 1, 4, D)), O.BF16)
    offs = np.array([0, 7, 1000, 32768, 12345], np.int32)
    batched = O.norm_rope(xb, O.BF16, dims=D, inv_freq=inv, offsets=offs)
    for b in range(5):
        one = O.norm_rope(np.ascontiguousarray(xb[b:b + 1]), O.BF16, dims=D, inv_freq=inv,
                          offset=int(offs[b]))
        assert np.array_equal(batched[b:b + 1], one)


def test_rope_inverse_rotation_recovers_input():
    x = O.normal(45, (1, 50, 2, 128))
    inv = O.rope_inv_freq(1e4, 128)
    y = O.norm_rope(x, O.F32, dims=128, inv_freq=inv, offset=3)
    back = O.norm_rope(y, O.F32, dims=128, inv_freq=inv, offset=3, scale=-1.0)
    np.testing.assert_allclose(back, x, rtol=1e-5, atol=1e-5)


def test_partial_rope_passes_tail_through_bitexact():
    x = O.from_f32(O.normal(46, (4, 1, 16, 256)), O.BF16)
    offs = O.offsets(47, 4, 1, 32768)
    y = O.norm_rope(x, O.BF16, dims=64, inv_freq=O.rope_inv_freq(1e7, 64), offsets=offs)
    assert np.array_equal(y[..., 64:], x[..., 64:])
    assert not np.array_equal(y[..., :64], x[..., :64])


def test_rope_bf16_rounding_sequence_matches_torch_ops():
    B, L, H, D = 1, 300, 4, 128
    x = O.from_f32(O.normal(48, (B, L, H, D)), O.BF16)
    inv = O.rope_inv_freq(1e6, D)
    got = O.norm_rope(x, O.BF16, dims=D, inv_freq=inv, offset=100)
    tx = from_bf16_bits(x)
    th = ((torch.arange(L, dtype=torch.float32) + 100.0)[:, None] * torch.from_numpy(inv)[None, :])
    c = torch.cos(th).to(torch.bfloat16)[None, :, None, :]
    s = torch.sin(th).to(torch.bfloat16)[None, :, None, :]
    x1, x2 = tx[..., :64], tx[..., 64:]
    ref = torch.cat([x1 * c - x2 * s, x1 * s + x2 * c], -1)
    rb = ref.view(torch.int16).numpy().view(np.uint16)
    assert exact_frac(got, rb, O.BF16) > 0.999


def test_norm_rope_equals_norm_then_rope():
    B, L, H, D = 2, 16, 5, 128
    x = O.from_f32(O.normal(49, (B, L, H, D)), O.BF16)
    w = O.from_f32(O.normal(50, (D,), 1.0, 0.02), O.BF16)
    inv = O.rope_inv_freq(1e6, D)
    fused = O.norm_rope(x, O.BF16, dims=D, inv_freq=inv, norm_w=w, w_dt=O.BF16, eps=1e-6)
    n = O.rms_norm(x.reshape(-1, D), O.BF16, w, O.BF16, 1e-6).reshape(B, L, H, D)
    two = O.norm_rope(n, O.BF16, dims=D, inv_freq=inv)
    assert np.array_equal(fused, two)


# ------------------------------------------------------------------ gated norm
def test_gated_norm_is_swiglu_of_norm():
    y = O.from_f32(O.normal(51, (128, 128)), O.BF16)
    z = O.from_f32(O.normal(52, (128, 128)), O.BF16)
    w = O.from_f32(O.normal(53, (128,), 1.0, 0.02), O.BF16)
    got = O.gated_rms_norm(y, z, O.BF16, w, O.BF16, 1e-6)
    n = O.rms_norm(y, O.BF16, w, O.BF16, 1e-6)
    ref = O.glu(O.ACT_SILU, z, n, O.BF16)
    assert np.array_equal(got, ref)
    yf, zf, wf = (O.to_f32(a, O.BF16).astype(np.float64) for a in (y, z, w))
    exact = zf / (1 + np.exp(-zf)) * yf / np.sqrt((yf ** 2).mean(-1, keepdims=True) + 1e-6) * wf
    # four bf16 roundings in the composition: within a few ulp of exact math
    assert_close(got, O.from_f32(exact.astype(np.float32), O.BF16), O.BF16, max_ulp=4,
                 rtol=3e-2, what="gated vs float64")


# ------------------------------------------------------------------ embedding
def _unpack_nibbles(words: np.ndarray) -> np.ndarray:
    shifts = (4 * np.arange(8, dtype=np.uint32))
    return ((words[..., None] >> shifts) & 0xF).reshape(*words.shape[:-1], -1)


def test_qembed_unit_scale_returns_codes_bitexact():
    V, H = 97, 256
    wq = O.u32(61, (V, H // 8))
    one = O.from_f32(np.ones((V, H // 64), np.float32), O.BF16)
    zero = O.from_f32(np.zeros((V, H // 64), np.float32), O.BF16)
    ids = O.ids(62, 300, V)
    got = O.to_f32(O.qembed(ids, wq, one, zero, O.BF16), O.BF16)
    assert np.array_equal(got, _unpack_nibbles(wq)[ids].astype(np.float32))


def test_qembed_matches_torch_composition_and_table_rows():
    V, H, g = 211, 512, 64
    wq = O.u32(63, (V, H // 8))
    s = O.from_f32(O.uniform(64, (V, H // g), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(65, (V, H // g), -0.1, 0.1), O.BF16)
    ids = O.ids(66, 500, V)
    got = O.qembed(ids, wq, s, b, O.BF16)
    q = torch.from_numpy(_unpack_nibbles(wq).astype(np.float32))
    ts = from_bf16_bits(s).float().repeat_interleave(g, 1)
    tb = from_bf16_bits(b).repeat_interleave(g, 1)
    table = (q * ts).to(torch.bfloat16) + tb  # bf16 add rounds once more
    ref = table[torch.from_numpy(ids.astype(np.int64))].view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)
    full = O.qembed(np.arange(V, dtype=np.uint32), wq, s, b, O.BF16)
    assert np.array_equal(got, full[ids])  # gather-then-dequant == dequant-then-take


def test_qembed_zero_code_gives_bias_and_ids_edge_cases():
    V, H = 16, 64
    wq = np.zeros((V, H // 8), np.uint32)
    s = O.from_f32(O.uniform(67, (V, 1), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(68, (V, 1), -0.1, 0.1), O.BF16)
    ids = np.array([3, -1, -16, 16, -17, 0], np.int32)
    got = O.qembed(ids, wq, s, b, O.BF16)
    assert np.array_equal(got[0], np.repeat(b[3], H))
    assert np.array_equal(got[1], np.repeat(b[15], H))   # -1 -> last row
    assert np.array_equal(got[2], np.repeat(b[0], H))
    assert not got[3].any() and not got[4].any()         # out of range -> zeros
    assert np.array_equal(got[5], np.repeat(b[0], H))


def test_gemma_embedding_scale():
    assert O.to_f32(O.from_f32(np.array([math.sqrt(3584.0)], np.float32), O.BF16), O.BF16)[0] == 59.75
    V, H = 31, 3584
    wq = O.u32(69, (V, H // 8))
    s = O.from_f32(O.uniform(70, (V, H // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(71, (V, H // 64), -0.1, 0.1), O.BF16)
    ids = O.ids(72, 40, V)
    plain = O.qembed(ids, wq, s, b, O.BF16)
    scaled = O.qembed(ids, wq, s, b, O.BF16, out_scale=math.sqrt(3584.0))
    ref = (from_bf16_bits(plain) * torch.tensor(59.75, dtype=torch.bfloat16))
    assert np.array_equal(scaled, ref.view(torch.int16).numpy().view(np.uint16))


# ------------------------------------------------------------------ inputs
def test_rng_is_deterministic_and_well_formed():
    a = O.normal(1001, (1_000_001,))
    assert np.array_equal(a, O.normal(1001, (1_000_001,)))
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1) < 5e-3
    c = O.u32(1002, (100_000,))
    nib = _unpack_nibbles(c).ravel()
    counts = np.bincount(nib, minlength=16) / nib.size
    assert np.abs(counts - 1 / 16).max() < 2e-3
    i = O.ids(1003, 100_000, 128256)
    assert i.max() < 128256 and i.min() >= 0
    o = O.offsets(1004, 10_000, 1, 32768)
    assert o.min() >= 1 and o.max() <= 32768


# ------------------------------------------------------------------ residual add (+ norm)
def test_add_matches_torch_bf16_numpy_f16_and_f32():
    """MLX's add on bf16/f16 widens to f32, adds once and rounds once. torch's
    bf16 add and numpy's float16 add are independent implementations of the
    same IEEE operation; f32 is plain IEEE addition."""
    a = O.normal(2101, (64, 256)) * np.float32(40.0)
    b = O.normal(2102, (64, 256)) * np.float32(40.0)
    # exact bf16 ties: a + b lands halfway between two bf16 values
    a[0, :8] = np.float32(1.0)
    b[0, :8] = np.float32(2.0 ** -8) * np.arange(1, 9, dtype=np.float32)
    a[1, :4] = [60000.0, -60000.0, 1.0, -3.0]
    b[1, :4] = [60000.0, -60000.0, -1.0, 3.0]
    xa, xb = O.from_f32(a, O.BF16), O.from_f32(b, O.BF16)
    ref = (from_bf16_bits(xa) + from_bf16_bits(xb)).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.add(xa, xb, O.BF16), ref)
    ha, hb = O.from_f32(a, O.F16), O.from_f32(b, O.F16)
    with np.errstate(over="ignore"):
        ref16 = (ha.view(np.float16) + hb.view(np.float16)).view(np.uint16)
    assert np.array_equal(O.add(ha, hb, O.F16), ref16)  # incl. 60000+60000 -> inf
    assert np.array_equal(O.add(a, b, O.F32), a + b)
    # strided rows and an in-place form
    wide = O.from_f32(O.normal(2103, (16, 96)), O.BF16)
    got = O.add(wide[:, :48], wide[:, 48:], O.BF16)
    ref = (from_bf16_bits(wide[:, :48]) + from_bf16_bits(wide[:, 48:])).view(torch.int16)
    assert np.array_equal(got, ref.numpy().view(np.uint16))


def test_add_rms_norm_closed_forms():
    """r = 0 leaves h = x and y = rms_norm(x); r = -x gives h = +0 and y = 0
    (the zero row's scale is 1/sqrt(eps), times 0)."""
    x = O.from_f32(O.normal(2111, (32, 512)), O.BF16)
    w = O.from_f32(O.normal(2112, (512,), 1.0, 0.02), O.BF16)
    zero = O.from_f32(np.zeros((32, 512), np.float32), O.BF16)
    h, y = O.add_rms_norm(x, zero, O.BF16, w, O.BF16, 1e-5)
    assert np.array_equal(h, x)
    assert np.array_equal(y, O.rms_norm(x, O.BF16, w, O.BF16, 1e-5))
    neg = x ^ np.uint16(0x8000)
    h, y = O.add_rms_norm(x, neg, O.BF16, w, O.BF16, 1e-5)
    assert not h.any() and not (y & np.uint16(0x7FFF)).any()


def test_add_rms_norm_matches_torch_composition():
    """h from torch's bf16 add; y against a float64 RMSNorm of that h within
    the bf16 bar (the f64 path rounds differently only in the last place)."""
    x = O.from_f32(O.normal(2121, (48, 2048)), O.BF16)
    r = O.from_f32(O.normal(2122, (48, 2048)), O.BF16)
    w = O.from_f32(O.normal(2123, (2048,), 1.0, 0.02), O.BF16)
    h, y = O.add_rms_norm(x, r, O.BF16, w, O.BF16, 1e-5)
    th = from_bf16_bits(x) + from_bf16_bits(r)
    assert np.array_equal(h, th.view(torch.int16).numpy().view(np.uint16))
    hd = th.double()
    ref = hd * torch.rsqrt((hd * hd).mean(-1, keepdim=True) + 1e-5) * from_bf16_bits(w).double()
    assert_close(y, bf16_bits_torch(ref.float().numpy()), O.BF16, max_ulp=2,
                 what="add_rms_norm vs f64")


def test_qembed_rms_norm_constant_row_closed_form():
    """Codes all 3 with scale 1 and bias 0 give h = 3 exactly; the norm of a
    constant row c is c / sqrt(c^2 + eps), which rounds to 1.0 in bf16 at
    eps = 1e-5, so y is exactly the weight row."""
    V, Hd = 16, 256
    wq = np.full((V, Hd // 8), 0x33333333, np.uint32)
    one = O.from_f32(np.ones((V, Hd // 64), np.float32), O.BF16)
    zero = O.from_f32(np.zeros((V, Hd // 64), np.float32), O.BF16)
    w = O.from_f32(O.normal(2131, (Hd,), 1.0, 0.02), O.BF16)
    ids = np.array([0, 5, 15], np.uint32)
    h, y = O.qembed_rms_norm(ids, wq, one, zero, O.BF16, w, O.BF16, 1e-5)
    assert np.array_equal(O.to_f32(h, O.BF16), np.full((3, Hd), 3.0, np.float32))
    assert np.array_equal(y, np.broadcast_to(w, (3, Hd)))
    # and in general it is the gather followed by the norm, invalid ids -> zero rows
    wq = O.u32(2132, (V, Hd // 8))
    s = O.from_f32(O.uniform(2133, (V, Hd // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(2134, (V, Hd // 64), -0.1, 0.1), O.BF16)
    ids = np.array([1, -1, 20, 3], np.int32)
    h, y = O.qembed_rms_norm(ids, wq, s, b, O.BF16, w, O.BF16, 1e-6, out_scale=16.0)
    hq = O.qembed(ids, wq, s, b, O.BF16, out_scale=16.0)
    assert np.array_equal(h, hq)
    assert np.array_equal(y, O.rms_norm(hq, O.BF16, w, O.BF16, 1e-6))
    assert not y[2].any()


# ------------------------------------------------------------------ gather_qmm
def _qmm_case(key, P, R, E, N, K, group=64, dt=O.BF16):
    x = O.from_f32(O.normal(key, (R, K)), dt)
    w = O.u32(key + 1, (E, N, K // 8))
    s = O.from_f32(O.uniform(key + 2, (E, N, K // group), 0.005, 0.02), dt)
    b = O.from_f32(O.uniform(key + 3, (E, N, K // group), -0.1, 0.1), dt)
    ex = (O.u32(key + 4, (P,)) % np.uint32(E)).astype(np.int32)
    return x, w, s, b, ex


def _dequant_f64(w, s, b, dt, group):
    E, N, W = w.shape
    q = ((w[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(E, N, W * 8)
    sf = np.repeat(O.to_f32(s, dt).astype(np.float64), group, axis=-1)
    bf = np.repeat(O.to_f32(b, dt).astype(np.float64), group, axis=-1)
    return q.astype(np.float64) * sf + bf


def test_gather_qmm_matches_torch_f64_dequant_matmul():
    """torch f64: dequantize the table, gather each pair's expert, matmul,
    round once to bf16 -- an independent route to the same number."""
    P, R, E, N, K, top_k = 40, 4, 6, 96, 512, 10
    x, w, s, b, ex = _qmm_case(2201, P, R, E, N, K)
    y = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=top_k)
    wd = torch.from_numpy(_dequant_f64(w, s, b, O.BF16, 64))
    xd = torch.from_numpy(O.to_f32(x, O.BF16).astype(np.float64))
    rows = torch.arange(P) // top_k
    ref = torch.einsum("pk,pnk->pn", xd[rows], wd[torch.from_numpy(ex).long()])
    ref_bits = ref.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert_close(y, ref_bits, O.BF16, max_ulp=1, what="gather_qmm vs torch f64")
    assert exact_frac(y, ref_bits, O.BF16) >= 0.999


def test_quantized_matmul_matches_torch_f64_and_groups():
    """quantized_matmul (QLinear::forward): torch f64 dequantize-then-matmul
    rounded once to bf16 agrees; groups 32 and 128 dequantize with their own
    scale spans; f16 activations too."""
    for dt, group, M, N, K in ((O.BF16, 64, 9, 80, 512), (O.BF16, 32, 5, 48, 256),
                               (O.BF16, 128, 5, 48, 512), (O.F16, 64, 7, 40, 256)):
        x = O.from_f32(O.normal(2250 + group, (M, K)), dt)
        w = O.u32(2251 + group, (N, K // 8))
        s = O.from_f32(O.uniform(2252 + group, (N, K // group), 0.005, 0.02), dt)
        b = O.from_f32(O.uniform(2253 + group, (N, K // group), -0.1, 0.1), dt)
        y = O.quantized_matmul(x, dt, w, s, b, dt, group=group)
        wd = torch.from_numpy(_dequant_f64(w[None], s[None], b[None], dt, group)[0])
        xd = torch.from_numpy(O.to_f32(x, dt).astype(np.float64))
        ref = (xd @ wd.T).to(torch.bfloat16 if dt == O.BF16 else torch.float16)
        ref_bits = ref.view(torch.int16).numpy().view(np.uint16)
        assert_close(y, ref_bits, dt, max_ulp=1, what=f"quantized_matmul g{group}")
        assert exact_frac(y, ref_bits, dt) >= 0.99


def test_gather_qmm_closed_forms():
    """Unit scales, zero biases and one-hot x return the raw codes; all-zero
    codes return sum_g b_g * sum_{k in g} x_k."""
    E, N, K = 3, 16, 128
    w = O.u32(2211, (E, N, K // 8))
    one = O.from_f32(np.ones((E, N, K // 64), np.float32), O.BF16)
    zero = O.from_f32(np.zeros((E, N, K // 64), np.float32), O.BF16)
    x = np.zeros((K, K), np.float32)
    x[np.arange(K), np.arange(K)] = 1.0
    xb = O.from_f32(x, O.BF16)
    ex = np.full(K, 2, np.int32)
    y = O.to_f32(O.gather_qmm(xb, O.BF16, w, one, zero, O.BF16, ex), O.BF16)
    q = ((w[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(E, N, K)
    assert np.array_equal(y, q[2].T.astype(np.float32))  # row k of y = codes at k
    xs = O.from_f32(O.normal(2212, (4, K)), O.BF16)
    bias = O.from_f32(O.uniform(2213, (E, N, K // 64), -0.1, 0.1), O.BF16)
    y0 = O.gather_qmm(xs, O.BF16, np.zeros_like(w), one, bias, O.BF16, np.array([0, 1, 2, 0], np.int32))
    xg = O.to_f32(xs, O.BF16).astype(np.float64).reshape(4, K // 64, 64).sum(-1)
    bt = O.to_f32(bias, O.BF16).astype(np.float64)
    ref = np.einsum("pg,png->pn", xg, bt[[0, 1, 2, 0]])
    assert_close(y0, O.from_f32(ref.astype(np.float32), O.BF16), O.BF16, max_ulp=1,
                 what="zero codes")


def test_gather_qmm_routing_and_out_of_range():
    """p // x_div routing equals explicit lhs rows; experts and rows out of
    range give zero rows (negative expert ids wrap once, as int32 indices)."""
    P, R, E, N, K = 12, 3, 4, 32, 256
    x, w, s, b, ex = _qmm_case(2221, P, R, E, N, K)
    y1 = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, x_div=4)
    y2 = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, lhs=np.arange(P) // 4)
    assert np.array_equal(y1, y2)
    bad = ex.copy()
    bad[[0, 5]] = [E, -1]
    y3 = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, bad, x_div=4)
    assert not y3[0].any()
    wrapped = ex.copy()
    wrapped[5] = E - 1
    y4 = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, wrapped, x_div=4)
    assert np.array_equal(y3[5], y4[5])
    lhs = np.arange(P) // 4
    lhs[3] = R
    y5 = O.gather_qmm(x, O.BF16, w, s, b, O.BF16, ex, lhs=lhs)
    assert not y5[3].any()


# ------------------------------------------------------------------ GatedDeltaNet
def _gdn_inputs(key, B, T, Hk, Dk, Hv, Dv, dt=O.F32):
    """The reference tests' distributions (qwen3_next.rs:2577-2595)."""
    u = lambda k, shape, lo, hi: O.from_f32(O.uniform(key + k, shape, lo, hi), dt)
    return dict(q=u(0, (B, T, Hk, Dk), -1, 1), k=u(1, (B, T, Hk, Dk), -1, 1),
                v=u(2, (B, T, Hv, Dv), -1, 1), a_log=O.uniform(key + 3, (Hv,), -1, 0),
                a=u(4, (B, T, Hv), -1, 1), dt_bias=O.uniform(key + 5, (Hv,), -0.5, 0.5),
                b=u(6, (B, T, Hv), -1, 1), state=u(7, (B, Hv, Dv, Dk), -0.1, 0.1))


def _gdn_torch_f64(inp, dt):
    """An independent torch f64 restatement of the step loop (the shape of the
    reference's gated_delta_step_ref, qwen3_next.rs:2452-2486)."""
    f = lambda x: torch.from_numpy(O.to_f32(x, dt).astype(np.float64))
    q, k, v, a, b, S = (f(inp[n]) for n in ("q", "k", "v", "a", "b", "state"))
    a_log = torch.from_numpy(inp["a_log"].astype(np.float64))
    dtb = torch.from_numpy(inp["dt_bias"].astype(np.float64))
    Hk, Hv = q.shape[2], v.shape[2]
    rep = Hv // Hk
    ys = []
    for t in range(q.shape[1]):
        g = torch.exp(-torch.exp(a_log) * torch.nn.functional.softplus(a[:, t] + dtb))
        beta = torch.sigmoid(b[:, t])
        qt = q[:, t].repeat_interleave(rep, dim=1)
        kt = k[:, t].repeat_interleave(rep, dim=1)
        S = S * g[..., None, None]
        kv = (S * kt[:, :, None, :]).sum(-1)
        delta = (v[:, t] - kv) * beta[..., None]
        S = S + kt[:, :, None, :] * delta[..., None]
        ys.append((S * qt[:, :, None, :]).sum(-1))
    return torch.stack(ys, 1), S


@pytest.mark.parametrize("shape", [(1, 3, 2, 32, 4, 32), (2, 5, 16, 128, 32, 16)])
def test_gated_delta_matches_torch_f64(shape):
    B, T, Hk, Dk, Hv, Dv = shape
    inp = _gdn_inputs(2501 + T, *shape)
    y, s = O.gated_delta(inp["q"], inp["k"], inp["v"], inp["a_log"], inp["a"], inp["dt_bias"],
                         inp["b"], O.F32, state=inp["state"])
    ty, ts = _gdn_torch_f64(inp, O.F32)
    np.testing.assert_allclose(y, ty.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s, ts.numpy(), rtol=1e-5, atol=1e-6)


def test_gated_delta_closed_forms():
    """a = dt_bias = 0 and a_log = 0 give g = 2^-1 exactly; with k = 0 the
    update leaves s = g * s0, so y = (s0 . q) / 2. With s0 = 0, a huge b
    (beta = 1) and k = e_j, one step gives s[dv] = v[dv] e_j and y = v q_j."""
    B, T, Hk, Dk, Hv, Dv = 1, 1, 1, 32, 2, 8
    inp = _gdn_inputs(2511, B, T, Hk, Dk, Hv, Dv)
    z = lambda shape: np.zeros(shape, np.float32)
    y, s = O.gated_delta(inp["q"], z((B, T, Hk, Dk)), inp["v"], z(Hv), z((B, T, Hv)), z(Hv),
                         inp["b"], O.F32, state=inp["state"])
    s0 = inp["state"].astype(np.float64)
    np.testing.assert_allclose(s, s0 * 0.5, rtol=0, atol=0)
    ref = 0.5 * np.einsum("bhvk,bk->bhv", s0, inp["q"][:, 0, 0].astype(np.float64))
    np.testing.assert_allclose(y[:, 0], ref, rtol=1e-6, atol=1e-7)
    j = 5
    k = z((B, T, Hk, Dk))
    k[..., j] = 1.0
    y, s = O.gated_delta(inp["q"], k, inp["v"], z(Hv), z((B, T, Hv)), z(Hv),
                         np.full((B, T, Hv), 60.0, np.float32), O.F32, state=None)
    np.testing.assert_allclose(s[0, :, :, j], inp["v"][0, 0], rtol=1e-6)
    assert not np.delete(s, j, axis=-1).any()
    np.testing.assert_allclose(y[0, 0], inp["v"][0, 0] * inp["q"][0, 0, 0, j], rtol=1e-6)


def test_gated_delta_norm_weights_and_rounding():
    """The fused q/k norm is rms_norm with the constant weights s*s and s
    (s = 1/sqrt(Dk) in f32, cast to the dtype): bf16(1/128) and
    bf16(0.0883883) at Dk = 128; a bf16 run equals the run on pre-normalised
    inputs, and the state and y come back rounded to bf16."""
    wq, wk = O.gdn_qk_norm_weights(128, O.BF16)
    assert O.to_f32(wq, O.BF16)[0] == np.float32(1 / 128)
    assert O.to_f32(wk, O.BF16)[0] == np.float32(0.08837890625)
    shape = (1, 2, 2, 128, 4, 8)
    inp = _gdn_inputs(2521, *shape, dt=O.BF16)
    args = (inp["v"], inp["a_log"], inp["a"], inp["dt_bias"], inp["b"], O.BF16)
    y1, s1 = O.gated_delta(inp["q"], inp["k"], *args, state=inp["state"], qw=wq, kw=wk)
    B, T, Hk, Dk = inp["q"].shape
    qn = O.rms_norm(inp["q"].reshape(-1, Dk), O.BF16, wq, O.BF16, 1e-6).reshape(inp["q"].shape)
    kn = O.rms_norm(inp["k"].reshape(-1, Dk), O.BF16, wk, O.BF16, 1e-6).reshape(inp["k"].shape)
    y2, s2 = O.gated_delta(qn, kn, *args, state=inp["state"])
    assert np.array_equal(y1, y2) and np.array_equal(s1, s2)
    assert y1.dtype == np.uint16 and s1.dtype == np.uint16


def test_geglu_f32_bar_admits_an_accurate_evaluation_and_rejects_a_slip():
    """The f32 GeGLU bar (tests/bits.py) holds for an accurate evaluation that
    does not cancel, g / (1 + e^(-2x)) in float64 rounded once to f32, against
    the oracle's MLX composition, over gates from -9 to 9; and it rejects the
    same evaluation with a dropped cubic term."""
    from bits import check_geglu_f32

    g = np.linspace(-9.0, 9.0, 200001).astype(np.float32)
    u = O.normal(77, (g.size,)) * np.float32(3.0)
    ref = O.glu(O.ACT_GELU_TANH, g[None, :], u[None, :], O.F32)[0]
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    k0, k1 = math.sqrt(2.0 / math.pi), 0.044715

    def dev_like(cubic):
        x = k0 * (g64 + cubic * k1 * g64 ** 3)
        return (g64 / (1.0 + np.exp(-2.0 * x)) * u64).astype(np.float32)

    check_geglu_f32(dev_like(1.0), ref, g, u, "accurate")
    with pytest.raises(AssertionError):
        check_geglu_f32(dev_like(0.0), ref, g, u, "no cubic term")


def test_rope_parity_check_ties_libm_differences_to_the_tables():
    """tests/bits.check_rope_parity: the device-trig oracle itself passes, its
    libm differences are all at elements where the tables differ; a 2-ulp
    slip on one element fails."""
    from bits import check_rope_parity

    x = O.from_f32(O.normal(81, (2, 512, 4, 128)), O.BF16)
    inv = O.rope_inv_freq(1e6, 128)
    offs = np.array([7, 30000], np.int32)
    rl = O.norm_rope(x, O.BF16, dims=128, inv_freq=inv, offsets=offs, trig=O.TRIG_LIBM)
    rd = O.norm_rope(x, O.BF16, dims=128, inv_freq=inv, offsets=offs, trig=O.TRIG_F64)
    check_rope_parity(rd, rl, rd, O.BF16, "device-trig oracle")
    bad = rd.copy()
    i = np.unravel_index(np.argmax(np.abs(O.to_f32(rd, O.BF16))), rd.shape)
    bad[i] = np.uint16(int(bad[i]) + 2)
    with pytest.raises(AssertionError):
        check_rope_parity(bad, rl, rd, O.BF16, "slip")
