"""GPU parity at the launch geometry bench.py times: every kernel of the
prefill workloads, at the configuration's full size, called with the same
arguments (dtypes, strides, heads per launch, output layout) as the timed
launch, against the CPU oracle on seeded inputs.

Workloads covered here (the decode sequence and the single RMSNorm are at full
size in test_gpu_parity.py):
  llama3.2-1b chain  RMSNorm [4096, 2048]; q and k RoPE in one launch with
                     llama3 frequencies, [B,L,H,D] in, [B,H,L,D] out, 4 x 1024
  qwen3-8b prefill   RMSNorm [16384, 4096]; q/k-norm + RoPE in one launch,
                     8 x 2048; SwiGLU [16384, 12288]
  gemma2-9b prefill  embedding gather x 59.75 over 256000 x 3584 for 16384
                     ids; (1+w) RMSNorm to f32 [16384, 3584]; q and k RoPE at
                     head_dim 256, 4 x 4096; GeGLU to f32 [16384, 14336]

Bars: bf16 within 1 ulp (RMSNorm at least 99.99 % bit-identical); RoPE within
1 ulp on every element of the oracle with the device's cos/sin evaluation,
with every difference from the libm oracle beyond that bar where the two
oracles' cos/sin differ; the f32 norm within rtol 1e-5 (atol 1e-6); GeGLU f32
within rtol 1e-5 plus the rounding error of the reference's own 1 + tanh
(2^-23 |gate x up|); SwiGLU and the embedding bit-exact.
"""
from __future__ import annotations

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
    print(f"[bench-shape] {what}: exact={exact_frac(got, ref, dt):.6f} "
          f"max_ulp={int(ulp_dist(got, ref, dt).max()) if got.size else 0}", flush=True)


def _rms(dev, rows, n, eps, *, plus_one=False, ydt=O.BF16, key):
    x = O.from_f32(O.normal(key, (rows, n)), O.BF16)
    w = O.from_f32(O.normal(key + 1, (n,), 0.0 if plus_one else 1.0, 0.02), O.BF16)
    ref = O.rms_norm(x, O.BF16, w, O.BF16, eps, plus_one=plus_one, out_dt=ydt)
    got = to_host(H.rms_norm(to_dev(x, O.BF16, dev), to_dev(w, O.BF16, dev), eps,
                             plus_one=plus_one, out_dtype=tdtype(ydt)))
    return got, ref


def test_llama32_chain_rms_norm(dev):
    got, ref = _rms(dev, 4096, 2048, 1e-5, key=2101)
    _report("llama rms_norm [4096,2048]", got, ref, O.BF16)
    assert ulp_dist(got, ref, O.BF16).max() <= 1
    assert exact_frac(got, ref, O.BF16) >= 0.9999


def test_qwen3_prefill_rms_norm(dev):
    got, ref = _rms(dev, 16384, 4096, 1e-6, key=2102)
    _report("qwen3 rms_norm [16384,4096]", got, ref, O.BF16)
    assert ulp_dist(got, ref, O.BF16).max() <= 1
    assert exact_frac(got, ref, O.BF16) >= 0.9999


def test_gemma2_prefill_plus_one_rms_norm_f32_out(dev):
    """(1+w) with the weight promoted to f32 (gemma2.rs:799-826): computation
    and output in f32."""
    got, ref = _rms(dev, 16384, 3584, 1e-6, plus_one=True, ydt=O.F32, key=2103)
    _report("gemma (1+w) rms_norm f32 [16384,3584]", got, ref, O.F32)
    assert_close(got, ref, O.F32, rtol=1e-5, atol=1e-6, what="gemma (1+w) rms_norm f32")


def _qk_rope(dev, *, B, L, Hq, Hk, D, dims, base=None, freqs=None, norm=False, eps=1e-6,
             key):
    """One hgk_qk_norm_rope launch over q [B,L,Hq,D] and k [B,L,Hk,D]
    (contiguous projection layout) writing [B,H,L,D], as bench.py's k_qkrope."""
    q = O.from_f32(O.normal(key, (B, L, Hq, D)), O.BF16)
    k = O.from_f32(O.normal(key + 1, (B, L, Hk, D)), O.BF16)
    wq = wk = None
    if norm:
        wq = O.from_f32(O.normal(key + 2, (D,), 1.0, 0.02), O.BF16)
        wk = O.from_f32(O.normal(key + 3, (D,), 1.0, 0.02), O.BF16)
    inv = O.rope_inv_freq(0.0 if freqs is not None else base, dims, freqs)
    kw = dict(dims=dims, inv_freq=inv, eps=eps)
    trigs = (O.TRIG_LIBM, O.TRIG_F64)
    rq = [O.norm_rope(q, O.BF16, norm_w=wq, w_dt=O.BF16 if norm else None, trig=t, **kw)
          for t in trigs]
    rk = [O.norm_rope(k, O.BF16, norm_w=wk, w_dt=O.BF16 if norm else None, trig=t, **kw)
          for t in trigs]
    qo, ko = H.qk_norm_rope(to_dev(q, O.BF16, dev), to_dev(k, O.BF16, dev),
                            None if wq is None else to_dev(wq, O.BF16, dev),
                            None if wk is None else to_dev(wk, O.BF16, dev), eps, dims,
                            base if freqs is None else None, 1.0, 0, freqs=freqs)
    assert qo.shape == (B, Hq, L, D) and qo.is_contiguous()
    assert ko.shape == (B, Hk, L, D) and ko.is_contiguous()
    gq = np.transpose(to_host(qo), (0, 2, 1, 3))
    gk = np.transpose(to_host(ko), (0, 2, 1, 3))
    return (gq, rq), (gk, rk)


def _check_rope(got, refs, what):
    """Every element within 1 bf16 ulp of the oracle with the device's cos/sin
    evaluation; against the libm oracle, every element outside that bar sits
    where the two oracles' cos/sin differ."""
    print(f"[bench-shape] {what}: " + check_rope_parity(got, refs[0], refs[1], O.BF16, what),
          flush=True)


def test_llama32_chain_fused_qk_rope(dev):
    """The chain's RoPE launch: q (32 heads) and k (8 heads) together, no norm,
    llama3 frequencies (factor 32, low 1, high 4, original 8192, theta 5e5)."""
    f = O.llama3_freqs(500000.0, 64, 32.0, 1.0, 4.0, 8192.0)
    (gq, rq), (gk, rk) = _qk_rope(dev, B=4, L=1024, Hq=32, Hk=8, D=64, dims=64, freqs=f,
                                  key=2201)
    _check_rope(gq, rq, "llama3 rope q [4,1024,32,64]")
    _check_rope(gk, rk, "llama3 rope k [4,1024,8,64]")


def test_qwen3_prefill_qk_norm_rope(dev):
    (gq, rq), (gk, rk) = _qk_rope(dev, B=8, L=2048, Hq=32, Hk=8, D=128, dims=128, base=1e6,
                                  norm=True, key=2202)
    _check_rope(gq, rq, "qwen3 qk-norm+rope q [8,2048,32,128]")
    _check_rope(gk, rk, "qwen3 qk-norm+rope k [8,2048,8,128]")


def test_gemma2_prefill_rope_d256(dev):
    (gq, rq), (gk, rk) = _qk_rope(dev, B=4, L=4096, Hq=16, Hk=8, D=256, dims=256, base=1e4,
                                  key=2203)
    _check_rope(gq, rq, "gemma rope q [4,4096,16,256]")
    _check_rope(gk, rk, "gemma rope k [4,4096,8,256]")


def test_qwen3_prefill_swiglu(dev):
    g = O.from_f32(O.normal(2301, (16384, 12288)), O.BF16)
    u = O.from_f32(O.normal(2302, (16384, 12288)), O.BF16)
    ref = O.glu(O.ACT_SILU, g, u, O.BF16)
    got = to_host(H.swiglu(to_dev(g, O.BF16, dev), to_dev(u, O.BF16, dev)))
    _report("qwen3 swiglu [16384,12288]", got, ref, O.BF16)
    assert np.array_equal(got, ref)


def test_gemma2_prefill_geglu_f32_out(dev):
    """gelu_approximate(gate) * up with bf16 gate/up computes and writes f32
    (mlx-rs builds the activation from f32 scalars, gemma2.rs:422-427)."""
    g = O.from_f32(O.normal(2303, (16384, 14336)), O.BF16)
    u = O.from_f32(O.normal(2304, (16384, 14336)), O.BF16)
    ref = O.glu(O.ACT_GELU_TANH, g, u, O.BF16, out_dt=O.F32)
    got = to_host(H.gelu_approximate_mul(to_dev(g, O.BF16, dev), to_dev(u, O.BF16, dev),
                                         out_dtype=torch.float32))
    print("[bench-shape] gemma geglu f32 [16384,14336]: " +
          check_geglu_f32(got, ref, O.to_f32(g, O.BF16), O.to_f32(u, O.BF16), "gemma geglu f32"),
          flush=True)


def test_gemma2_prefill_embedding_scaled(dev):
    """16384 ids over the full 256000 x 3584 table, group 64, scaled by
    bf16(sqrt(3584)) = 59.75 (gemma2.rs:587-600)."""
    V, Hd, T = 256000, 3584, 16384
    wq = O.u32(2401, (V, Hd // 8))
    sc = O.from_f32(O.uniform(2402, (V, Hd // 64), 0.005, 0.02), O.BF16)
    bi = O.from_f32(O.uniform(2403, (V, Hd // 64), -0.1, 0.1), O.BF16)
    ids = O.ids(2404, T, V)
    scale = math.sqrt(3584.0)
    ref = O.qembed(ids, wq, sc, bi, O.BF16, out_scale=scale)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(sc, O.BF16, dev),
                               to_dev(bi, O.BF16, dev), group_size=64)
    id_dt = O.I32 if ids.dtype == np.int32 else O.U32
    got = to_host(emb.forward(to_dev(ids, id_dt, dev), out_scale=scale))
    assert got.shape == (T, Hd)
    assert np.array_equal(got, ref)
