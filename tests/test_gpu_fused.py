"""GPU parity of the fused forms next to the path: residual add + RMSNorm
(transformer.rs:413-415) and the embedding gather + first RMSNorm
(transformer.rs:494, 407), through the C ABI against the oracle.

Bars: h (the add, or the dequantized embedding) bit-exact; y as the RMSNorm
tests (within 1 ulp, >= 99.99 % bit-exact; both sides round an f64 sum of
squares once, so in practice every value matches)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import higgs_amd as H
import oracle as O
from bits import exact_frac, ulp_dist
from gpu_util import tdtype, to_dev, to_host, words_dev

pytestmark = pytest.mark.gpu


def _check_y(got, ref, dt, what):
    d = ulp_dist(got, ref, dt)
    print(f"[fused] {what}: exact={exact_frac(got, ref, dt):.6f} max_ulp={int(d.max())}", flush=True)
    assert d.max() <= 1, what
    assert exact_frac(got, ref, dt) >= 0.9999, what


ADD_CASES = [
    # rows, n, dt, w_dt, plus_one, y_dt, eps
    (4096, 2048, O.BF16, O.BF16, False, O.BF16, 1e-5),   # Llama-3.2-1B block boundary
    (256, 4096, O.BF16, O.BF16, False, O.BF16, 1e-6),    # Qwen3-8B
    (64, 3584, O.BF16, O.BF16, True, O.F32, 1e-6),       # Gemma (1+w): f32 out
    (64, 2048, O.F16, O.F16, False, O.F16, 1e-5),
    (64, 2048, O.F32, O.F32, False, O.F32, 1e-5),
    (64, 2048, O.BF16, O.F32, False, O.F32, 1e-5),       # f32 weight promotes
    (2048, 128, O.BF16, O.BF16, False, O.BF16, 1e-6),    # head rows
    (33, 100, O.BF16, O.BF16, False, O.BF16, 1e-5),      # generic path
    (7, 8192, O.BF16, O.BF16, False, O.BF16, 1e-5),      # 16 chunks per lane
    (1, 2048, O.BF16, O.BF16, False, O.BF16, 1e-5),
]


@pytest.mark.parametrize("case", ADD_CASES,
                         ids=lambda c: f"{c[0]}x{c[1]}-x{c[2]}w{c[3]}p{int(c[4])}y{c[5]}")
def test_add_rms_norm(dev, case):
    rows, n, dt, wdt, p1, ydt, eps = case
    key = 3000 + rows + n
    x = O.from_f32(O.normal(key, (rows, n)), dt)
    r = O.from_f32(O.normal(key + 1, (rows, n)), dt)
    w = O.from_f32(O.normal(key + 2, (n,), 0.0 if p1 else 1.0, 0.02), wdt)
    h_ref, y_ref = O.add_rms_norm(x, r, dt, w, wdt, eps, plus_one=p1, out_dt=ydt)
    h, y = H.add_rms_norm(to_dev(x, dt, dev), to_dev(r, dt, dev), to_dev(w, wdt, dev), eps,
                          plus_one=p1, out_dtype=tdtype(ydt))
    assert np.array_equal(to_host(h), h_ref)
    _check_y(to_host(y), y_ref, ydt, f"add_rms_norm {case}")


def test_add_rms_norm_in_place_strided_and_without_h(dev):
    rows, n, pad = 300, 2048, 64
    buf = O.from_f32(O.normal(3101, (rows, n + pad)), O.BF16)
    r = O.from_f32(O.normal(3102, (rows, n)), O.BF16)
    w = O.from_f32(O.normal(3103, (n,), 1.0, 0.02), O.BF16)
    h_ref, y_ref = O.add_rms_norm(buf[:, :n], r, O.BF16, w, O.BF16, 1e-5)
    tb = to_dev(buf, O.BF16, dev)
    tr, tw = to_dev(r, O.BF16, dev), to_dev(w, O.BF16, dev)
    # h written over x itself (the residual stream updated in place)
    h, y = H.add_rms_norm(tb[:, :n], tr, tw, 1e-5, h_out=tb[:, :n])
    got = to_host(tb)
    assert np.array_equal(got[:, :n], h_ref)
    assert np.array_equal(got[:, n:], buf[:, n:])  # pad columns untouched
    _check_y(to_host(y), y_ref, O.BF16, "in place")
    # h over r
    tx = to_dev(buf[:, :n], O.BF16, dev)
    tr2 = to_dev(r, O.BF16, dev)
    H.add_rms_norm(tx, tr2, tw, 1e-5, h_out=tr2)
    assert np.array_equal(to_host(tr2), h_ref)
    # y only
    h, y = H.add_rms_norm(to_dev(buf[:, :n], O.BF16, dev), tr, tw, 1e-5, write_h=False)
    assert h is None
    _check_y(to_host(y), y_ref, O.BF16, "no h")


def test_add_rms_norm_chain_of_blocks(dev):
    """Three block boundaries in a row (h <- h + r_i, y_i = norm(h)), the
    residual stream kept in place on the device, against the oracle's chain."""
    rows, n = 512, 2048
    w = O.from_f32(O.normal(3201, (n,), 1.0, 0.02), O.BF16)
    h_ref = O.from_f32(O.normal(3202, (rows, n)), O.BF16)
    th = to_dev(h_ref, O.BF16, dev)
    tw = to_dev(w, O.BF16, dev)
    for i in range(3):
        r = O.from_f32(O.normal(3210 + i, (rows, n), 0.0, 0.5), O.BF16)
        h_ref, y_ref = O.add_rms_norm(h_ref, r, O.BF16, w, O.BF16, 1e-5)
        _, y = H.add_rms_norm(th, to_dev(r, O.BF16, dev), tw, 1e-5, h_out=th)
        assert np.array_equal(to_host(th), h_ref), f"block {i}"
        _check_y(to_host(y), y_ref, O.BF16, f"block {i}")


def _table(V, Hd, group, sdt, key):
    wq = O.u32(key, (V, Hd // 8))
    s = O.from_f32(O.uniform(key + 1, (V, Hd // group), 0.005, 0.02), sdt)
    b = O.from_f32(O.uniform(key + 2, (V, Hd // group), -0.1, 0.1), sdt)
    return wq, s, b


QEMB_NORM_CASES = [
    # V, H, n_ids, group, scales dt, norm w dt, plus_one, out_scale, y dt, eps
    (128256, 2048, 4096, 64, O.BF16, O.BF16, False, 0.0, O.BF16, 1e-5),   # Llama-3.2-1B
    (256000, 3584, 1024, 64, O.BF16, O.BF16, True, math.sqrt(3584.0), O.F32, 1e-6),  # Gemma-2
    (151936, 2048, 512, 64, O.BF16, O.BF16, False, 0.0, O.BF16, 1e-6),    # Qwen3-Next
    (32000, 4096, 300, 64, O.F16, O.F16, False, 0.0, O.F16, 1e-5),
    (5000, 8192, 200, 64, O.BF16, O.BF16, False, 0.0, O.BF16, 1e-5),      # 16 steps per lane
    (5000, 1024, 300, 32, O.BF16, O.F32, False, 0.0, O.F32, 1e-5),        # f32 norm weight
    (5000, 1024, 300, 128, O.BF16, O.F16, False, 0.0, O.F32, 1e-5),       # generic path
    (50, 96, 70, 32, O.BF16, O.BF16, False, 0.0, O.BF16, 1e-5),           # 12 words per row
    (5000, 512, 300, 64, O.BF16, O.BF16, False, 0.0, O.BF16, 1e-5),       # 1 step per lane
    (5000, 1024, 257, 64, O.F16, O.BF16, False, 0.0, O.F32, 1e-6),        # 2 steps, f16 scales
]


@pytest.mark.parametrize("case", QEMB_NORM_CASES, ids=lambda c: f"V{c[0]}H{c[1]}n{c[2]}g{c[3]}")
def test_qembed_rms_norm(dev, case):
    V, Hd, n, group, sdt, wdt, p1, osc, ydt, eps = case
    key = 3300 + Hd + group
    wq, s, b = _table(V, Hd, group, sdt, key)
    ids = O.ids(key + 3, n, V)
    w = O.from_f32(O.normal(key + 4, (Hd,), 0.0 if p1 else 1.0, 0.02), wdt)
    h_ref, y_ref = O.qembed_rms_norm(ids, wq, s, b, sdt, w, wdt, eps, group=group,
                                     out_scale=osc, plus_one=p1, out_dt=ydt)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(s, sdt, dev), to_dev(b, sdt, dev),
                               group_size=group)
    h, y = emb.forward_rms_norm(to_dev(ids, O.U32, dev), to_dev(w, wdt, dev), eps, plus_one=p1,
                                out_scale=osc, out_dtype=tdtype(ydt))
    assert np.array_equal(to_host(h), h_ref)
    _check_y(to_host(y), y_ref, ydt, f"qembed_rms_norm {case}")


def test_qembed_rms_norm_invalid_ids_and_no_h(dev):
    V, Hd = 50, 256
    wq, s, b = _table(V, Hd, 64, O.BF16, 3401)
    w = O.from_f32(O.normal(3405, (Hd,), 1.0, 0.02), O.BF16)
    ids = np.array([3, -1, -50, 50, -51, 0, 49], np.int32)
    h_ref, y_ref = O.qembed_rms_norm(ids, wq, s, b, O.BF16, w, O.BF16, 1e-5)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev))
    tids = to_dev(ids, O.I32, dev)
    h, y = emb.forward_rms_norm(tids, to_dev(w, O.BF16, dev), 1e-5)
    assert np.array_equal(to_host(h), h_ref)
    assert np.array_equal(to_host(y), y_ref)
    assert not to_host(y)[3].any() and not to_host(y)[4].any()
    h, y2 = emb.forward_rms_norm(tids, to_dev(w, O.BF16, dev), 1e-5, write_h=False)
    assert h is None and np.array_equal(to_host(y2), y_ref)


def test_fused_equals_unfused_calls(dev):
    """The fused entry points give exactly what the two separate calls give."""
    V, Hd, T = 128256, 2048, 1024
    wq, s, b = _table(V, Hd, 64, O.BF16, 3501)
    w = to_dev(O.from_f32(O.normal(3505, (Hd,), 1.0, 0.02), O.BF16), O.BF16, dev)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev))
    ids = to_dev(O.ids(3506, T, V), O.U32, dev)
    h1, y1 = emb.forward_rms_norm(ids, w, 1e-5)
    h2 = emb.forward(ids)
    y2 = H.rms_norm(h2, w, 1e-5)
    assert torch.equal(h1.view(torch.int16), h2.view(torch.int16))
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    r = to_dev(O.from_f32(O.normal(3507, (T, Hd)), O.BF16), O.BF16, dev)
    h3, y3 = H.add_rms_norm(h1, r, w, 1e-5)
    h4 = (h1.float() + r.float()).to(torch.bfloat16)
    assert torch.equal(h3.view(torch.int16), h4.view(torch.int16))
    assert torch.equal(y3.view(torch.int16), H.rms_norm(h4, w, 1e-5).view(torch.int16))
