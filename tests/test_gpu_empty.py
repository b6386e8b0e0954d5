"""Empty inputs: zero rows, tokens, ids or pairs. Every entry point returns an
empty result without an error and without touching its outputs, as the
reference's ops return empty arrays for empty inputs; the gated-delta
recurrence over zero steps leaves the state as it was."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import higgs_amd as H
import oracle as O
from gpu_util import to_dev, to_host, words_dev

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def test_norms_and_glu_with_no_rows(dev):
    x = torch.empty((0, 2048), dtype=BF, device=dev)
    w = torch.ones(2048, dtype=BF, device=dev)
    assert H.rms_norm(x, w, 1e-5).shape == (0, 2048)
    assert H.rms_norm(x, w, 1e-6, plus_one=True, out_dtype=torch.float32).shape == (0, 2048)
    h, y = H.add_rms_norm(x, x, w, 1e-5)
    assert h.shape == (0, 2048) and y.shape == (0, 2048)
    assert H.gated_rms_norm(x, x, w, 1e-6).shape == (0, 2048)
    assert H.swiglu(x, x).shape == (0, 2048)
    assert H.gelu_approximate_mul(x, x, out_dtype=torch.float32).shape == (0, 2048)
    assert H.fused_gate_up_swiglu(torch.empty((0, 1024), dtype=BF, device=dev)).shape == (0, 512)


def test_rope_with_no_tokens(dev):
    q = torch.empty((2, 0, 4, 64), dtype=BF, device=dev)
    k = torch.empty((2, 0, 2, 64), dtype=BF, device=dev)
    qw = torch.ones(64, dtype=BF, device=dev)
    qo, ko = H.qk_norm_rope(q, k, qw, qw, 1e-6, 64, 10000.0)
    assert qo.shape == (2, 4, 0, 64) and ko.shape == (2, 2, 0, 64)
    qo, ko = H.qk_norm_rope(torch.empty((0, 5, 4, 64), dtype=BF, device=dev), None, None, None,
                            1e-6, 64, 10000.0)
    assert qo.shape == (0, 4, 5, 64) and ko is None
    x = torch.empty((1, 3, 0, 64), dtype=BF, device=dev)
    assert H.rope(x, 64, False, 10000.0, 1.0, 0).shape == (1, 3, 0, 64)


def test_embedding_with_no_ids(dev):
    V, Hd, g = 40, 256, 64
    wq = O.u32(3901, (V, Hd // 8))
    s = O.from_f32(O.uniform(3902, (V, Hd // g), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(3903, (V, Hd // g), -0.1, 0.1), O.BF16)
    emb = H.QuantizedEmbedding(words_dev(wq, dev), to_dev(s, O.BF16, dev), to_dev(b, O.BF16, dev))
    ids = torch.empty((0,), dtype=torch.int32, device=dev)
    assert emb(ids).shape == (0, Hd)
    h, y = emb.forward_rms_norm(ids, torch.ones(Hd, dtype=BF, device=dev), 1e-5)
    assert h.shape == (0, Hd) and y.shape == (0, Hd)
    # and a real call right after still gives the oracle's rows
    ids2 = np.array([3, 0, 39], np.int32)
    got = to_host(emb(to_dev(ids2, O.I32, dev)))
    assert np.array_equal(got, O.qembed(ids2, wq, s, b, O.BF16, group=g))


def test_contractions_with_no_rows(dev):
    E, N, K = 4, 128, 512
    w = words_dev(O.u32(3911, (E, N, K // 8)), dev)
    s = to_dev(O.from_f32(O.uniform(3912, (E, N, K // 64), 0.005, 0.02), O.BF16), O.BF16, dev)
    x = torch.empty((0, K), dtype=BF, device=dev)
    ex = torch.empty((0,), dtype=torch.int32, device=dev)
    assert H.gather_qmm(x, w, s, s, ex).shape == (0, N)
    assert H.gather_qmm_swiglu(x, w, s, s, w, s, s, ex).shape == (0, N)
    assert H.quantized_matmul(x, w[0], s[0], s[0]).shape == (0, N)


def test_gated_delta_with_no_steps(dev):
    B, Hk, Dk, Hv, Dv = 2, 2, 128, 4, 128
    q = torch.empty((B, 0, Hk, Dk), dtype=BF, device=dev)
    v = torch.empty((B, 0, Hv, Dv), dtype=BF, device=dev)
    ab = torch.empty((B, 0, Hv), dtype=BF, device=dev)
    alog = torch.zeros(Hv, dtype=torch.float32, device=dev)
    st = torch.randn((B, Hv, Dv, Dk), device=dev).to(BF)
    y, st2 = H.gated_delta(q, q, v, alog, ab, alog, ab, st)
    assert y.shape == (B, 0, Hv, Dv)
    assert torch.equal(st2, st)
    # without an input state the state after zero steps is zeros
    st3 = torch.full((B, Hv, Dv, Dk), 7.0, dtype=BF, device=dev)
    y, st4 = H.gated_delta(q, q, v, alog, ab, alog, ab, None, state_out=st3)
    assert st4 is st3 and not st3.any()
    # in place: the state is left as it is
    y, st5 = H.gated_delta(q, q, v, alog, ab, alog, ab, st, state_out=st)
    assert torch.equal(st5, st2)
