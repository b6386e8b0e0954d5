"""quantized_matmul (QLinear::forward, qwen3_next.rs:174-221) on the GPU
against the oracle (the exact f64 contraction rounded once). A floating-point
contraction accumulated in f32, so the bar is the stated tolerance, written
here: every bf16/f16 output within 1 ulp of the oracle, or within atol 1e-3
next to zero (rtol 1e-2, atol 1e-3); at least 99 % bit-identical. M >= 16
rows in bf16 with group 64 run on the matrix cores; the rest one GEMV per
row."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import higgs_amd as H
import oracle as O
from bits import assert_close, exact_frac
from gpu_util import to_dev, to_host, words_dev

pytestmark = pytest.mark.gpu


def _case(key, M, N, K, group=64, dt=O.BF16, xs=1.0):
    x = O.from_f32(O.normal(key, (M, K)) * np.float32(xs), dt)
    w = O.u32(key + 1, (N, K // 8))
    s = O.from_f32(O.uniform(key + 2, (N, K // group), 0.005, 0.02), dt)
    b = O.from_f32(O.uniform(key + 3, (N, K // group), -0.1, 0.1), dt)
    return x, w, s, b


def _run(dev, x, w, s, b, dt, group=64):
    y = H.quantized_matmul(to_dev(x, dt, dev), words_dev(w, dev), to_dev(s, dt, dev),
                           to_dev(b, dt, dev), True, group, 4)
    return to_host(y)


def _check(got, ref, dt, what):
    ef = exact_frac(got, ref, dt)
    print(f"[qgemm] {what}: exact={ef:.5f}", flush=True)
    assert_close(got, ref, dt, max_ulp=1, what=what)
    assert ef >= 0.99, what


@pytest.mark.parametrize("M,N,K", [(16, 256, 512), (64, 2048, 2048), (33, 640, 1536),
                                   (48, 200, 576), (64, 256, 4096), (100, 384, 1024),
                                   (512, 1024, 2048), (777, 1000, 512), (1024, 512, 4096)],
                         ids=["M16", "decode64", "odd-chunks", "K576", "skinny-K4096", "ragged-M",
                              "M512", "ragged-MN", "K4096"])
def test_mfma_path_matches_oracle(dev, M, N, K):
    x, w, s, b = _case(3000 + M + N, M, N, K)
    got = _run(dev, x, w, s, b, O.BF16)
    ref = O.quantized_matmul(x, O.BF16, w, s, b, O.BF16)
    _check(got, ref, O.BF16, f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N", [(64, 12288), (40, 12288), (64, 12400)],
                         ids=["in_proj_qkvz", "rows40", "ragged-tiles"])
def test_decode_wide_projection(dev, M, N):
    """The decode step of a batch through in_proj_qkvz (2048 -> 12288), the
    launch geometry bench.py times, plus a partly filled second row half and
    a column count that leaves the last column tile ragged."""
    K = 2048
    x, w, s, b = _case(3701 + M + N, M, N, K)
    got = _run(dev, x, w, s, b, O.BF16)
    ref = O.quantized_matmul(x, O.BF16, w, s, b, O.BF16)
    _check(got, ref, O.BF16, f"decode M={M} N={N} K={K}")


def test_qwen3_next_prefill_projection(dev):
    """A 2048-token prefill through a 2048 -> 4096 projection (the attention
    q projection's shape class)."""
    M, N, K = 2048, 4096, 2048
    x, w, s, b = _case(3101, M, N, K)
    got = _run(dev, x, w, s, b, O.BF16)
    # the oracle on a sample of rows (the full f64 product takes minutes)
    rows = np.r_[0:64, 1000:1032, M - 64:M]
    ref = O.quantized_matmul(x[rows], O.BF16, w, s, b, O.BF16)
    _check(got[rows], ref, O.BF16, "prefill 2048x4096x2048 (sampled rows)")


@pytest.mark.parametrize("M", [1, 3, 15])
def test_few_rows_take_the_gemv_path(dev, M):
    x, w, s, b = _case(3200 + M, M, 512, 2048)
    got = _run(dev, x, w, s, b, O.BF16)
    ref = O.quantized_matmul(x, O.BF16, w, s, b, O.BF16)
    _check(got, ref, O.BF16, f"M={M}")


@pytest.mark.parametrize("dt,group", [(O.F16, 64), (O.BF16, 32), (O.BF16, 128)])
def test_other_dtypes_and_groups(dev, dt, group):
    x, w, s, b = _case(3300 + group, 40, 256, 1024, group=group, dt=dt)
    got = _run(dev, x, w, s, b, dt, group=group)
    ref = O.quantized_matmul(x, dt, w, s, b, dt, group=group)
    _check(got, ref, dt, f"dt={dt} group={group}")


def test_equals_gather_qmm_per_pair(dev):
    """The reference's own gather-vs-quantized_matmul check (qwen3_next.rs:
    2152-2206): gather_qmm over pairs of one expert equals quantized_matmul
    with that expert's weights, here within the same 1-ulp bar (the two run
    different kernels, with different f32 summation orders)."""
    M, E, N, K = 48, 4, 256, 1024
    x, _, _, _ = _case(3401, M, N, K)
    w = O.u32(3402, (E, N, K // 8))
    s = O.from_f32(O.uniform(3403, (E, N, K // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(3404, (E, N, K // 64), -0.1, 0.1), O.BF16)
    e = 2
    qm = _run(dev, x, w[e], s[e], b[e], O.BF16)
    ga = to_host(H.gather_qmm(to_dev(x, O.BF16, dev), words_dev(w, dev), to_dev(s, O.BF16, dev),
                              to_dev(b, O.BF16, dev),
                              torch.full((M,), e, dtype=torch.int32, device=dev)))
    _check(qm, ga, O.BF16, "quantized_matmul vs gather_qmm")


def test_strided_rows_and_leading_dims(dev):
    """x as [B, L, K] with a padded row stride; y written with the leading dims."""
    B, L, N, K = 3, 20, 256, 512
    x, w, s, b = _case(3501, B * L, N, K)
    buf = torch.zeros((B * L, K + 64), dtype=torch.bfloat16, device=dev)
    buf[:, :K] = to_dev(x, O.BF16, dev)
    xv = buf[:, :K]
    assert xv.stride(0) == K + 64
    y = H.quantized_matmul(xv, words_dev(w, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev))
    ref = O.quantized_matmul(x, O.BF16, w, s, b, O.BF16)
    _check(to_host(y), ref, O.BF16, "strided x")
    y3 = H.quantized_matmul(to_dev(x, O.BF16, dev).view(B, L, K), words_dev(w, dev),
                            to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev))
    assert tuple(y3.shape) == (B, L, N)
    _check(to_host(y3).reshape(B * L, N), ref, O.BF16, "3-d x")


def test_f16_gemv_grid_beyond_two_to_the_32_work_items(dev):
    """f16 runs one wave per output element: M = 512 rows of a 151936-column
    projection (the Qwen3 vocabulary) is 4.98e9 work-items, more than one HIP
    launch holds; the kernel walks the outputs in a capped grid instead. The
    oracle checks the first and last rows."""
    M, N, K = 512, 151936, 64
    x, w, s, b = _case(3601, M, N, K, dt=O.F16)
    got = _run(dev, x, w, s, b, O.F16)
    for rows in (np.r_[0:4], np.r_[M - 4:M]):
        ref = O.quantized_matmul(x[rows], O.F16, w, s, b, O.F16)
        _check(got[rows], ref, O.F16, f"f16 M={M} N={N} rows {rows[0]}..{rows[-1]}")
