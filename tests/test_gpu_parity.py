"""GPU parity: every kernel, through the C ABI (via the higgs_amd mirror),
against the CPU oracle on the same seeded inputs.

Bars (stated per test): SwiGLU, the gated norm's gate, dequantized embeddings
and unpacked codes are bit-exact; RMSNorm-family outputs are bit-exact (both
sides round an f64 sum of squares once); RoPE is within 1 bf16 ulp (rtol 1e-2,
atol 1e-3) - the device's f64 sin/cos and libm's f32 sin/cos can differ in the
last f32 bit - and f32 outputs within rtol 1e-5 (plus a small atol where a
difference of two rounded products cancels).
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np
import pytest
import torch

import higgs_amd as H
import oracle as O
from bits import assert_close, check_geglu_f32, check_rope_parity, exact_frac, ulp_dist
from gpu_util import tdtype, to_dev, to_host, words_dev

pytestmark = pytest.mark.gpu


def _report(what, got, ref, dt):
    print(f"[parity] {what}: exact={exact_frac(got, ref, dt):.6f} "
          f"max_ulp={int(ulp_dist(got, ref, dt).max()) if got.size else 0}", flush=True)


# ------------------------------------------------------------------ RMSNorm
RMS_CASES = [
    # rows, n, x_dt, w_dt (None = no weight), plus_one, y_dt, eps
    (512, 2048, O.BF16, O.BF16, False, O.BF16, 1e-5),     # RMSNorm alone [512, 2048]
    (96, 4096, O.BF16, O.BF16, False, O.BF16, 1e-6),      # Qwen3-8B hidden
    (64, 3584, O.BF16, O.BF16, True, O.F32, 1e-6),        # Gemma (1+w), promoted f32 out
    (64, 3584, O.BF16, O.BF16, True, O.BF16, 1e-6),       # Gemma (1+w), bf16 out
    (40, 4608, O.BF16, O.BF16, True, O.F32, 1e-6),        # Gemma-2-27B (1+w): 16-byte units
    (40, 5376, O.BF16, O.BF16, True, O.F32, 1e-6),        # Gemma-3-27B (1+w): 16-byte units
    (24, 8192, O.F16, O.F32, False, O.F32, 1e-5),         # f32 weight, f32 out, 16 units/lane
    (64, 2048, O.F32, O.F32, False, O.F32, 1e-5),
    (64, 2048, O.F16, O.F16, False, O.F16, 1e-5),
    (64, 2048, O.BF16, O.F32, False, O.F32, 1e-5),        # f32 weight promotes
    (2048, 128, O.BF16, O.BF16, False, O.BF16, 1e-6),     # q/k-norm rows
    (333, 256, O.BF16, O.BF16, False, O.BF16, 1e-6),
    (64, 2048, O.BF16, None, False, O.BF16, 1e-5),        # no weight
    (33, 100, O.BF16, O.BF16, False, O.BF16, 1e-5),       # generic path (n % 8 != 0)
    (17, 8192, O.BF16, O.BF16, False, O.BF16, 1e-5),      # 16 chunks per lane
    (5, 12288, O.BF16, O.BF16, False, O.BF16, 1e-5),      # beyond registers: generic
    (1, 2048, O.BF16, O.BF16, False, O.BF16, 1e-5),
]


@pytest.mark.parametrize("case", RMS_CASES, ids=lambda c: f"{c[0]}x{c[1]}-x{c[2]}w{c[3]}p{int(c[4])}y{c[5]}")
def test_rms_norm(dev, case):
    rows, n, xdt, wdt, p1, ydt, eps = case
    key = rows * 7 + n
    x = O.from_f32(O.normal(key, (rows, n)), xdt)
    w = None
    if wdt is not None:
        w = O.from_f32(O.normal(key + 1, (n,), 0.0 if p1 else 1.0, 0.02), wdt)
    ref = O.rms_norm(x, xdt, w, wdt if wdt is not None else xdt, eps, plus_one=p1, out_dt=ydt)
    got = H.rms_norm(to_dev(x, xdt, dev), None if w is None else to_dev(w, wdt, dev), eps,
                     plus_one=p1, out_dtype=tdtype(ydt))
    got = to_host(got)
    _report(f"rms_norm {case}", got, ref, ydt)
    assert ulp_dist(got, ref, ydt).max() <= 1
    assert exact_frac(got, ref, ydt) >= 0.9999


def test_rms_norm_strided_rows_and_views(dev):
    rows, n, pad = 300, 2048, 64
    buf = O.from_f32(O.normal(901, (rows, n + pad)), O.BF16)
    w = O.from_f32(O.normal(902, (n,), 1.0, 0.02), O.BF16)
    ref = O.rms_norm(buf[:, :n], O.BF16, w, O.BF16, 1e-5)
    tb = to_dev(buf, O.BF16, dev)
    out = torch.zeros((rows, n + pad), dtype=torch.bfloat16, device=dev)
    H.rms_norm(tb[:, :n], to_dev(w, O.BF16, dev), 1e-5, out=out[:, :n])
    got = to_host(out)
    assert np.array_equal(got[:, :n], ref)
    assert not got[:, n:].any()  # the pad columns are untouched


# ------------------------------------------------------------------ RoPE
def _rope_case(dev, *, B, L, Hq, D, dims, base=None, freqs=None, dt=O.BF16, offset=0,
               offsets=None, layout="BHLD", key=0):
    """Plain RoPE on x laid out [B,H,L,D] (post-transpose) or [B,L,H,D]."""
    shape = (B, Hq, L, D) if layout == "BHLD" else (B, L, Hq, D)
    x = O.from_f32(O.normal(key, shape), dt)
    xv = np.transpose(x, (0, 2, 1, 3)) if layout == "BHLD" else x
    inv = O.rope_inv_freq(base if base is not None else 0.0, dims, freqs)
    offs_np = None if offsets is None else np.asarray(offsets, np.int32)
    refs = [np.ascontiguousarray(O.norm_rope(xv, dt, dims=dims, inv_freq=inv, offset=offset,
                                             offsets=offs_np, trig=tr))
            for tr in (O.TRIG_LIBM, O.TRIG_F64)]
    tx = to_dev(x, dt, dev)
    offs_t = None if offs_np is None else torch.from_numpy(offs_np).to(dev)
    if layout == "BHLD":
        y = H.rope(tx, dims, False, None if freqs is not None else base, 1.0, offset,
                   freqs=freqs, offsets=offs_t)
        got = np.transpose(to_host(y), (0, 2, 1, 3))
    else:
        # [B,L,H,D] is addressed as a 4-D view whose axis -2 is L
        y = H.rope(tx.permute(0, 2, 1, 3), dims, False, None if freqs is not None else base,
                   1.0, offset, freqs=freqs, offsets=offs_t)
        got = np.transpose(to_host(y), (0, 2, 1, 3))
    return got, refs, dt


def _check_rope(got, refs, dt, what):
    """Every element within 1 ulp (16-bit) or rtol 1e-5 (f32) of the oracle
    with the device's cos/sin evaluation; against the libm oracle, every
    element outside that bar sits where the two oracles' cos/sin differ."""
    print(f"[parity] {what}: " + check_rope_parity(got, refs[0], refs[1], dt, what), flush=True)


def test_rope_llama3_chain_shape(dev):
    """Llama-3.2-1B: q [B,32,L,64], theta 5e5, llama3 scaling factor 32."""
    f = O.llama3_freqs(500000.0, 64, 32.0, 1.0, 4.0, 8192.0)
    got, ref, dt = _rope_case(dev, B=2, L=256, Hq=32, D=64, dims=64, freqs=f, key=1101)
    _check_rope(got, ref, dt, "rope llama3 q")
    got, ref, dt = _rope_case(dev, B=2, L=256, Hq=8, D=64, dims=64, freqs=f, key=1102,
                              offset=700)
    _check_rope(got, ref, dt, "rope llama3 k offset")


@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
def test_rope_default_dtypes(dev, dt):
    got, ref, dt = _rope_case(dev, B=2, L=97, Hq=4, D=128, dims=128, base=1e6, dt=dt,
                              key=1103, offset=31)
    _check_rope(got, ref, dt, f"rope dt={dt}")


def test_rope_gemma_head256_bld_layout(dev):
    got, ref, dt = _rope_case(dev, B=1, L=128, Hq=16, D=256, dims=256, base=1e4, key=1104,
                              layout="BLHD")
    _check_rope(got, ref, dt, "rope D=256 [B,L,H,D]")


def test_rope_per_sequence_offsets_large(dev):
    offs = O.offsets(1105, 64, 1, 32768)
    for dt in (O.BF16, O.F32):
        got, ref, dt = _rope_case(dev, B=64, L=1, Hq=16, D=128, dims=128, base=1e6, dt=dt,
                                  offsets=offs, key=1106)
        _check_rope(got, ref, dt, f"rope offsets to 32768 dt={dt}")


def test_rope_device_cos_sin_are_f32_of_f64(dev):
    """The device's cos/sin table itself. In f32 with x1 = 1 and x2 = 0 a
    RoPE returns its table entries: y1 = c, y2 = s. Over 4 sequences x 4096
    positions x 64 frequencies (offsets 0 .. 2^21, so angles up to ~2.1e6
    rad, through the fast evaluation below 2^20 rad and the library's beyond
    it) every entry must equal the f32 rounding of the f64 cos/sin of the
    same f32 angle, computed here by numpy (the oracle's TRIG_F64 choice)."""
    B, L, D = 4, 4096, 128
    offs = np.array([0, 5 * 4096, 2 ** 19 - 4096, 2 ** 21], np.int32)
    x = torch.zeros((B, 1, L, D), dtype=torch.float32, device=dev)
    x[..., : D // 2] = 1.0
    y = H.rope(x, D, base=10000.0, offsets=torch.tensor(offs, device=dev))
    got = to_host(y)[:, 0]
    inv = np.array(H.rope_inv_freq(10000.0, D), np.float32)
    pos = (np.arange(L, dtype=np.float32)[None, :] + offs[:, None].astype(np.float32)).astype(np.float32)
    th = (pos[:, :, None] * inv[None, None, :]).astype(np.float32)
    c = np.cos(th.astype(np.float64)).astype(np.float32)
    s = np.sin(th.astype(np.float64)).astype(np.float32)
    bad_c = got[..., : D // 2] != c
    bad_s = got[..., D // 2:] != s
    print(f"[rope] cos/sin table: {th.size} angles, max {float(np.abs(th).max()):.0f} rad, "
          f"{int(bad_c.sum())} cos and {int(bad_s.sum())} sin entries differ", flush=True)
    assert not bad_c.any() and not bad_s.any()


def test_rope_generic_path_head80(dev):
    got, ref, dt = _rope_case(dev, B=2, L=9, Hq=3, D=80, dims=80, base=1e4, key=1107)
    _check_rope(got, ref, dt, "rope D=80 generic")
    got, ref, dt = _rope_case(dev, B=2, L=9, Hq=3, D=96, dims=32, base=1e4, key=1108)
    _check_rope(got, ref, dt, "rope partial D=96 generic")


def test_rope_in_place(dev):
    x = O.from_f32(O.normal(1109, (2, 4, 33, 64)), O.BF16)
    inv = O.rope_inv_freq(1e4, 64)
    ref = O.norm_rope(np.transpose(x, (0, 2, 1, 3)), O.BF16, dims=64, inv_freq=inv, offset=5,
                      trig=O.TRIG_F64)
    tx = to_dev(x, O.BF16, dev)
    H.rope(tx, 64, False, 1e4, 1.0, 5, out=tx)
    assert np.array_equal(np.transpose(to_host(tx), (0, 2, 1, 3)), ref)


# ------------------------------------------------------------------ q/k norm + RoPE
def _qk_case(dev, *, B, L, Hq, Hk, D, dims, base, eps, dt=O.BF16, offsets=None, offset=0,
             q_block=None, key=0):
    """q from a projection [B,L,Hq,D] (or the first D of each q_block-wide head block,
    Qwen3-Next), k [B,L,Hk,D]; outputs [B,H,L,D] as after the reference's transpose."""
    qb = q_block or D
    qbuf = O.from_f32(O.normal(key, (B, L, Hq, qb)), dt)
    kbuf = O.from_f32(O.normal(key + 1, (B, L, Hk, D)), dt)
    wq = O.from_f32(O.normal(key + 2, (D,), 1.0, 0.02), dt)
    wk = O.from_f32(O.normal(key + 3, (D,), 1.0, 0.02), dt)
    inv = O.rope_inv_freq(base, dims)
    offs_np = None if offsets is None else np.asarray(offsets, np.int32)
    qv = qbuf[..., :D]
    rq = [O.norm_rope(qv, dt, dims=dims, inv_freq=inv, norm_w=wq, w_dt=dt, eps=eps,
                      offset=offset, offsets=offs_np, trig=tr) for tr in (O.TRIG_LIBM, O.TRIG_F64)]
    rk = [O.norm_rope(kbuf, dt, dims=dims, inv_freq=inv, norm_w=wk, w_dt=dt, eps=eps,
                      offset=offset, offsets=offs_np, trig=tr) for tr in (O.TRIG_LIBM, O.TRIG_F64)]
    tq = to_dev(qbuf, dt, dev)[..., :D]
    tk = to_dev(kbuf, dt, dev)
    offs_t = None if offs_np is None else torch.from_numpy(offs_np).to(dev)
    qo, ko = H.qk_norm_rope(tq, tk, to_dev(wq, dt, dev), to_dev(wk, dt, dev), eps, dims, base,
                            1.0, offset, offsets=offs_t)
    gq = np.transpose(to_host(qo), (0, 2, 1, 3))
    gk = np.transpose(to_host(ko), (0, 2, 1, 3))
    return (gq, rq), (gk, rk)


def test_qk_norm_rope_qwen3_prefill_shape(dev):
    """Qwen3-8B: q [B,L,32,128], k [B,L,8,128], theta 1e6, eps 1e-6, positions 0..L-1."""
    (gq, rq), (gk, rk) = _qk_case(dev, B=2, L=256, Hq=32, Hk=8, D=128, dims=128, base=1e6,
                                  eps=1e-6, key=1201)
    _check_rope(gq, rq, O.BF16, "qk-norm-rope q")
    _check_rope(gk, rk, O.BF16, "qk-norm-rope k")


def test_qk_norm_partial_rope_qwen3_next_decode(dev):
    """Qwen3-Next decode: q is the first 256 of each 512-wide head block, 16 q / 2 kv
    heads, 64 of 256 dims rotated, theta 1e7, offsets uniform in 1..32768."""
    offs = O.offsets(1301, 64, 1, 32768)
    (gq, rq), (gk, rk) = _qk_case(dev, B=64, L=1, Hq=16, Hk=2, D=256, dims=64, base=1e7,
                                  eps=1e-6, offsets=offs, q_block=512, key=1302)
    _check_rope(gq, rq, O.BF16, "qk-norm partial q")
    _check_rope(gk, rk, O.BF16, "qk-norm partial k")
    # dims >= 64 are only normalised: bit-exact against the oracle
    assert np.array_equal(gq[..., 64:], rq[0][..., 64:])


def test_qk_norm_rope_f32(dev):
    (gq, rq), (gk, rk) = _qk_case(dev, B=1, L=64, Hq=4, Hk=2, D=128, dims=128, base=1e6,
                                  eps=1e-6, dt=O.F32, offset=1000, key=1401)
    _check_rope(gq, rq, O.F32, "qk-norm-rope f32 q")
    _check_rope(gk, rk, O.F32, "qk-norm-rope f32 k")


# Shapes that take the one-chunk-per-lane layout (rows under 256 bytes), over
# every partner distance R = dims / (2 * chunk) it meets (1, 2, 4), each
# dtype, full and partial rotation, with and without the fused norm; ragged
# sequences (L 37) and per-sequence offsets.
LANE_CASES = [
    # D, dims, dtype, norm
    (16, 16, O.BF16, False),   # R 1, 2 lanes per row
    (32, 32, O.BF16, True),    # R 2, 4 lanes
    (64, 64, O.F16, True),     # R 4, 8 lanes
    (64, 32, O.BF16, True),    # partial: R 2 of 8 lanes
    (64, 16, O.F16, False),    # partial: R 1 of 8 lanes
    (32, 32, O.F32, False),    # f32 rows of 128 bytes: R 4
    (32, 16, O.F32, True),     # partial f32: R 2 of 8 lanes
    (8, 8, O.F32, True),       # f32: R 1, 2 lanes
]


@pytest.mark.parametrize("case", LANE_CASES, ids=lambda c: f"D{c[0]}-dims{c[1]}-dt{c[2]}-n{int(c[3])}")
def test_rope_one_chunk_per_lane_layouts(dev, case):
    D, dims, dt, norm = case
    offs = O.offsets(1450 + D + dims, 3, 0, 5000)
    if norm:
        (gq, rq), (gk, rk) = _qk_case(dev, B=3, L=37, Hq=5, Hk=3, D=D, dims=dims, base=1e4,
                                      eps=1e-6, dt=dt, offsets=offs, key=1460 + D + dims)
        _check_rope(gq, rq, dt, f"lane layout {case} q")
        _check_rope(gk, rk, dt, f"lane layout {case} k")
    else:
        got, ref, _ = _rope_case(dev, B=3, L=37, Hq=5, D=D, dims=dims, base=1e4, dt=dt,
                                 offsets=offs, layout="BLHD", key=1470 + D + dims)
        _check_rope(got, ref, dt, f"lane layout {case}")
        if dims < D:  # the pass-through dims are copied bit-exactly
            assert np.array_equal(got[..., dims:], ref[0][..., dims:])


# ------------------------------------------------------------------ GLU
@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
def test_swiglu_bitexact(dev, dt):
    """bf16/f16 at these sizes take the LDS-table kernel; f32 the direct one."""
    rows, n = {O.BF16: (4096, 8192), O.F16: (2048, 2048), O.F32: (256, 1024)}[dt]
    g = O.from_f32(O.normal(1501 + dt, (rows, n)) * np.float32(2.0), dt)
    u = O.from_f32(O.normal(1511 + dt, (rows, n)), dt)
    ref = O.glu(O.ACT_SILU, g, u, dt)
    got = to_host(H.swiglu(to_dev(g, dt, dev), to_dev(u, dt, dev)))
    _report(f"swiglu dt={dt}", got, ref, dt)
    assert np.array_equal(got, ref)


def _same_bits_nan_aware(got, ref, dt):
    from bits import nan_mask
    gn, rn = nan_mask(got, dt), nan_mask(ref, dt)
    assert np.array_equal(gn, rn), "NaN positions differ"
    bad = (got != ref) & ~gn
    assert not bad.any(), f"{int(bad.sum())} elements differ, first at {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
def test_swiglu_every_16bit_gate_value(dev, dt):
    """The 16-bit SwiGLU keeps a fast sigmoid only where it provably rounds like
    MLX's exact one; check that claim for all 65536 gate bit patterns
    (subnormals, infinities and NaNs included), through both launch shapes."""
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g = codes.reshape(256, 256)
    one = O.from_f32(np.ones((256, 256), np.float32), dt)
    ref = O.glu(O.ACT_SILU, g, one, dt)
    got = to_host(H.swiglu(to_dev(g, dt, dev), to_dev(one, dt, dev)))
    _same_bits_nan_aware(got, ref, dt)
    gt = np.ascontiguousarray(np.tile(codes, 512).reshape(4096, 8192))
    u = O.from_f32(O.normal(1901 + dt, (4096, 8192)), dt)
    ref = O.glu(O.ACT_SILU, gt, u, dt)
    got = to_host(H.swiglu(to_dev(gt, dt, dev), to_dev(u, dt, dev)))
    _same_bits_nan_aware(got, ref, dt)


def test_swiglu_reference_known_answers(dev):
    g = torch.tensor([[0.0, 1.0, -1.0]], device=dev)
    u = torch.tensor([[5.0, 1.0, 2.0]], device=dev)
    out = H.swiglu(g, u).cpu().numpy()[0]
    assert abs(out[0]) < 1e-6
    assert abs(out[1] - 0.7310586) < 1e-4
    assert abs(out[2] - (-0.5378828)) < 1e-4


def test_swiglu_layouts(dev):
    # phi3 fused gate_up [rows, 2I] split in place; expert rows [64*10, 512]; odd width
    gu = O.from_f32(O.normal(1521, (64, 1024)), O.BF16)
    ref = O.glu(O.ACT_SILU, gu[:, :512], gu[:, 512:], O.BF16)
    got = to_host(H.fused_gate_up_swiglu(to_dev(gu, O.BF16, dev)))
    assert np.array_equal(got, ref)
    g = O.from_f32(O.normal(1522, (640, 512)), O.BF16)
    u = O.from_f32(O.normal(1523, (640, 512)), O.BF16)
    assert np.array_equal(to_host(H.silu_mul(to_dev(g, O.BF16, dev), to_dev(u, O.BF16, dev))),
                          O.glu(O.ACT_SILU, g, u, O.BF16))
    g = O.from_f32(O.normal(1524, (7, 1001)), O.BF16)
    u = O.from_f32(O.normal(1525, (7, 1001)), O.BF16)
    assert np.array_equal(to_host(H.silu_mul(to_dev(g, O.BF16, dev), to_dev(u, O.BF16, dev))),
                          O.glu(O.ACT_SILU, g, u, O.BF16))
    # bf16 in, f32 out: the bf16 result widened (direct path, then table path)
    got = to_host(H.silu_mul(to_dev(g, O.BF16, dev), to_dev(u, O.BF16, dev),
                             out_dtype=torch.float32))
    assert np.array_equal(got, O.glu(O.ACT_SILU, g, u, O.BF16, out_dt=O.F32))
    g = O.from_f32(O.normal(1526, (1024, 4096)) * np.float32(3.0), O.BF16)
    u = O.from_f32(O.normal(1527, (1024, 4096)), O.BF16)
    got = to_host(H.silu_mul(to_dev(g, O.BF16, dev), to_dev(u, O.BF16, dev),
                             out_dtype=torch.float32))
    assert np.array_equal(got, O.glu(O.ACT_SILU, g, u, O.BF16, out_dt=O.F32))
    # strided rows through the table path: fused gate_up [rows, 2I]
    gu = O.from_f32(O.normal(1528, (512, 2 * 4096)), O.BF16)
    ref = O.glu(O.ACT_SILU, gu[:, :4096], gu[:, 4096:], O.BF16)
    assert np.array_equal(to_host(H.fused_gate_up_swiglu(to_dev(gu, O.BF16, dev))), ref)


@pytest.mark.parametrize("dt,odt", [(O.BF16, O.BF16), (O.BF16, O.F32), (O.F32, O.F32),
                                    (O.F16, O.F16)])
def test_geglu(dev, dt, odt):
    rows, n = (1024, 14336) if dt == O.BF16 else (128, 2048)
    g = O.from_f32(O.normal(1601 + dt, (rows, n)) * np.float32(2.0), dt)
    u = O.from_f32(O.normal(1611 + dt, (rows, n)), dt)
    ref = O.glu(O.ACT_GELU_TANH, g, u, dt, out_dt=odt)
    got = to_host(H.gelu_approximate_mul(to_dev(g, dt, dev), to_dev(u, dt, dev),
                                         out_dtype=tdtype(odt)))
    _report(f"geglu {dt}->{odt}", got, ref, odt)
    if odt == O.F32:
        print("[parity] geglu f32: " + check_geglu_f32(got, ref, O.to_f32(g, dt), O.to_f32(u, dt),
                                                       "geglu f32"), flush=True)
    else:
        assert_close(got, ref, odt, max_ulp=1, what="geglu")


# ------------------------------------------------------------------ gated norm
def test_gated_norm_qwen3_next_z_in_place(dev):
    """64 tokens x 32 value heads x 128; z read straight from in_proj_qkvz
    [tokens, 16 key heads, 768] where z is the last 256 (2 value heads) of each block."""
    T, nk, vpk, dv = 64, 16, 2, 128
    y = O.from_f32(O.normal(1701, (T * nk * vpk, dv)), O.BF16)
    qkvz = O.from_f32(O.normal(1702, (T, nk, 768)), O.BF16)
    w = O.from_f32(O.normal(1703, (dv,), 1.0, 0.02), O.BF16)
    z_np = np.ascontiguousarray(qkvz[:, :, 512:768]).reshape(T * nk * vpk, dv)
    ref = O.gated_rms_norm(y, z_np, O.BF16, w, O.BF16, 1e-6)
    tq = to_dev(qkvz, O.BF16, dev)
    zview = tq[:, :, 512:768].unflatten(-1, (vpk, dv))
    got = to_host(H.gated_rms_norm(to_dev(y, O.BF16, dev), zview, to_dev(w, O.BF16, dev), 1e-6))
    _report("gated norm", got, ref, O.BF16)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("dt", [O.BF16, O.F32])
def test_gated_norm_contiguous(dev, dt):
    y = O.from_f32(O.normal(1711, (512, 128)), dt)
    z = O.from_f32(O.normal(1712, (512, 128)), dt)
    w = O.from_f32(O.normal(1713, (128,), 1.0, 0.02), dt)
    ref = O.gated_rms_norm(y, z, dt, w, dt, 1e-6)
    got = to_host(H.gated_rms_norm(to_dev(y, dt, dev), to_dev(z, dt, dev), to_dev(w, dt, dev),
                                   1e-6))
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------ embedding
def _qemb(dev, V, Hd, n_ids, group=64, sdt=O.BF16, out_scale=0.0, ids=None, key=0):
    wq = O.u32(key, (V, Hd // 8))
    s = O.from_f32(O.uniform(key + 1, (V, Hd // group), 0.005, 0.02), sdt)
    b = O.from_f32(O.uniform(key + 2, (V, Hd // group), -0.1, 0.1), sdt)
    if ids is None:
        ids = O.ids(key + 3, n_ids, V)
    ref = O.qembed(ids, wq, s, b, sdt, group=group, out_scale=out_scale)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(s, sdt, dev), to_dev(b, sdt, dev),
                               group_size=group)
    id_dt = O.I32 if ids.dtype == np.int32 else O.U32
    got = to_host(emb.forward(to_dev(ids, id_dt, dev), out_scale=out_scale))
    return got, ref


def test_qembed_llama_vocab(dev):
    got, ref = _qemb(dev, 128256, 2048, 4096, key=1801)
    assert np.array_equal(got, ref)


def test_qembed_gemma_vocab_scaled(dev):
    got, ref = _qemb(dev, 256000, 3584, 4096, out_scale=math.sqrt(3584.0), key=1811)
    assert np.array_equal(got, ref)


def test_qembed_codes_bitexact_and_variants(dev):
    V, Hd = 1000, 512
    wq = O.u32(1821, (V, Hd // 8))
    one = O.from_f32(np.ones((V, Hd // 64), np.float32), O.BF16)
    zero = O.from_f32(np.zeros((V, Hd // 64), np.float32), O.BF16)
    ids = O.ids(1822, 777, V)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(one, O.BF16, dev),
                               to_dev(zero, O.BF16, dev))
    got = O.to_f32(to_host(emb.forward(to_dev(ids, O.U32, dev))), O.BF16)
    codes = ((wq[..., None] >> (4 * np.arange(8, dtype=np.uint32))) & 0xF).reshape(V, Hd)
    assert np.array_equal(got, codes[ids].astype(np.float32))
    for group in (32, 128):
        got, ref = _qemb(dev, 500, 1024, 300, group=group, key=1830 + group)
        assert np.array_equal(got, ref)
    got, ref = _qemb(dev, 500, 1024, 300, sdt=O.F16, key=1840)
    assert np.array_equal(got, ref)
    got, ref = _qemb(dev, 50, 96, 70, group=32, key=1850)  # generic path (hidden % 32 != 0)
    assert np.array_equal(got, ref)
    ids = np.array([3, -1, -50, 50, -51, 0, 49], np.int32)
    got, ref = _qemb(dev, 50, 256, 0, ids=ids, key=1860)
    assert np.array_equal(got, ref)
    assert not got[3].any() and not got[4].any()


@pytest.mark.parametrize("V,Hd,n,group,sdt,offset", [
    (300, 4608, 9000, 32, O.BF16, 0),   # 144 groups a row: the 256-group table, 9 of 16 steps
    (300, 448, 9000, 64, O.BF16, 0),    # 7 groups, one partial step
    (300, 3584, 9000, 64, O.F16, 0),    # 56 groups
    (300, 2048, 8193, 64, O.BF16, 1),   # scales/biases 2-byte aligned only
    (300, 8192, 8500, 128, O.BF16, 0),  # 16 steps a row, group 128
    (300, 3584, 16387, 64, O.F16, 0),   # f16, a ragged last workgroup
    (300, 2048, 20000, 32, O.BF16, 0),  # 64 groups a row
    (300, 1024, 16384, 128, O.BF16, 0), # 2 steps a row
    (300, 3584, 5000, 32, O.BF16, 0),   # 112 groups: 7 steps, the 256-group table
    (300, 4096, 5000, 32, O.F16, 1),    # 128 groups: 8 steps, two table groups per lane
    (300, 8192, 3000, 32, O.BF16, 0),   # 256 groups: the largest table
    (300, 8192, 700, 64, O.BF16, 0),    # 128 groups, fewer than 1024 ids (one wave a workgroup)
])
def test_qembed_row_load_forms(dev, V, Hd, n, group, sdt, offset):
    """The table gather at every table size (64 and 256 groups; one to four
    groups per lane), group 32, 64 and 128, partial last steps, scales and
    biases at a 2-byte offset, one and four waves per workgroup. Bit-exact
    against the oracle."""
    key = 1870 + group + Hd
    wq = O.u32(key, (V, Hd // 8))
    s = O.from_f32(O.uniform(key + 1, (V, Hd // group), 0.005, 0.02), sdt)
    b = O.from_f32(O.uniform(key + 2, (V, Hd // group), -0.1, 0.1), sdt)
    ids = O.ids(key + 3, n, V)
    ref = O.qembed(ids, wq, s, b, sdt, group=group)

    def placed(a):  # the table at an element offset inside a larger buffer
        flat = to_dev(a.reshape(-1), sdt, dev)
        buf = torch.zeros(flat.numel() + offset, dtype=flat.dtype, device=dev)
        buf[offset:] = flat
        return buf[offset:].view(a.shape)

    emb = H.QuantizedEmbedding(words_dev(wq, dev), placed(s), placed(b), group_size=group)
    got = to_host(emb.forward(to_dev(ids, O.U32, dev)))
    assert np.array_equal(got, ref)


def test_qembed_600k_ids(dev):
    """600,000 ids (150,000 workgroups, many rounds of resident waves); int32
    ids with negative (from the end) and out-of-range values. Bit-exact."""
    V, Hd, n = 1000, 256, 600000
    key = 1940
    wq = O.u32(key, (V, Hd // 8))
    s = O.from_f32(O.uniform(key + 1, (V, Hd // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(key + 2, (V, Hd // 64), -0.1, 0.1), O.BF16)
    ids = O.ids(key + 3, n, V).astype(np.int32)
    ids[::997] = -3
    ids[5::1009] = V + 2
    ref = O.qembed(ids, wq, s, b, O.BF16)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev))
    got = to_host(emb.forward(to_dev(ids, O.I32, dev)))
    assert np.array_equal(got, ref)
    assert not got[5].any() and got[0].any()


def _bits16(key, shape, sdt, exp_lo, exp_hi, zero_frac=0.0):
    """Random 16-bit float codes of `sdt` with a random sign and mantissa and an
    exponent field uniform in [exp_lo, exp_hi]; a fraction of them +-0."""
    mbits = 7 if sdt == O.BF16 else 10
    r = O.u32(key, shape)
    sign = (r >> np.uint32(31)) & np.uint32(1)
    mant = r & np.uint32((1 << mbits) - 1)
    ex = np.uint32(exp_lo) + (O.u32(key + 1, shape) % np.uint32(exp_hi - exp_lo + 1))
    out = ((sign << np.uint32(15)) | (ex << np.uint32(mbits)) | mant).astype(np.uint16)
    if zero_frac:
        z = (O.u32(key + 2, shape) % np.uint32(1000)) < np.uint32(zero_frac * 1000)
        out[z] &= np.uint16(0x8000)
    return out


@pytest.mark.parametrize("sdt", [O.BF16, O.F16])
@pytest.mark.parametrize("out_scale", [0.0, math.sqrt(3584.0), -math.sqrt(3584.0), -0.75])
def test_qembed_any_scale_and_bias_values(dev, sdt, out_scale):
    """Rows whose scales and biases span wide exponent ranges (bf16: scales
    of either sign from 2^-100 to 2^100, biases +-0 or from 2^-100 to 2^126,
    so that round(q s) + b is often inexact in f32; f16: normal scales below
    2^12, biases below 2^11), rows of arbitrary 16-bit codes (zeros,
    subnormals, huge values, inf, NaN, overflowing products) and ordinary
    rows, with and without the output scale, positive or negative (a negative
    one turns row 7's +0 elements into -0). The gather's tables hold each
    group's 16 values from the element formula, so every such row must come
    out as the oracle's: bit-exact, zero signs included (NaN positions
    compared as a mask)."""
    V, Hd, n = 1536, 2048, 3000
    G = Hd // 64
    key = 1950 + 10 * sdt + int(out_scale > 0) + 2 * int(out_scale < 0)
    wq = O.u32(key, (V, Hd // 8))
    s = O.from_f32(O.uniform(key + 1, (V, G), 0.005, 0.02), sdt)
    b = O.from_f32(O.uniform(key + 2, (V, G), -0.1, 0.1), sdt)
    bf = sdt == O.BF16
    wide_s = _bits16(key + 3, (V, G), sdt, 27 if bf else 1, 226 if bf else 26)
    wide_b = _bits16(key + 6, (V, G), sdt, 27 if bf else 0, 252 if bf else 25, zero_frac=0.05)
    any_s = (O.u32(key + 9, (V, G)) & np.uint32(0xffff)).astype(np.uint16)
    any_b = (O.u32(key + 10, (V, G)) & np.uint32(0xffff)).astype(np.uint16)
    rows = np.arange(V)
    s[rows % 3 == 1] = wide_s[rows % 3 == 1]
    b[rows % 3 == 1] = wide_b[rows % 3 == 1]
    s[rows % 3 == 2] = any_s[rows % 3 == 2]
    b[rows % 3 == 2] = any_b[rows % 3 == 2]
    # a negative scale beside a -0 bias (q = 0 must give -0), and a +0 bias
    s[4, :] = s[4, :] | np.uint16(0x8000)
    b[4, :] = np.uint16(0x8000)
    b[7, :] = np.uint16(0x0000)
    ids = O.ids(key + 11, n, V)
    ids[:4] = np.array([4, 7, 1, 2], ids.dtype)
    ref = O.qembed(ids, wq, s, b, sdt, out_scale=out_scale)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(s, sdt, dev), to_dev(b, sdt, dev))
    got = to_host(emb.forward(to_dev(ids, O.U32, dev), out_scale=out_scale))
    _same_bits_nan_aware(got, ref, sdt)


# ------------------------------------------------------------------ hgk_sync
def test_sync_waits_for_the_stream_it_names(dev):
    """hgk_sync is the only blocking entry: after it returns for a side stream,
    everything queued there has finished (the stream reports idle) and the
    result is the one the oracle gives."""
    from higgs_amd import _lib
    rows, n = 4096, 4096
    x = O.from_f32(O.normal(1901, (rows, n)), O.BF16)
    w = O.from_f32(O.normal(1902, (n,), 1.0, 0.02), O.BF16)
    xd, wd = to_dev(x, O.BF16, dev), to_dev(w, O.BF16, dev)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        outs = [H.rms_norm(xd, wd, 1e-5) for _ in range(8)]
    _lib.check(_lib.lib().hgk_sync(C.c_void_p(side.cuda_stream)))
    assert side.query()
    _lib.check(_lib.lib().hgk_sync(None))
    ref = O.rms_norm(x, O.BF16, w, O.BF16, 1e-5)
    assert np.array_equal(to_host(outs[-1]), ref) or ulp_dist(to_host(outs[-1]), ref, O.BF16).max() <= 1
