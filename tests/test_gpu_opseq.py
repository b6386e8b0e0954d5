"""The decode op sequence in one launch (hgk_op_list_upload / hgk_op_list_run,
Python OpSequence) against the separate calls it replaces, bit for bit, and
the residual chain against the oracle.

The sequence is the Qwen3-Next decode layer's per-layer ops in the order of
the reference loop (qwen3_next.rs:1508-1547): input_layernorm as residual add
+ RMSNorm, the gated RMSNorm (linear-attention layers, z read in place from
in_proj_qkvz) or q/k RMSNorm + partial RoPE (every fourth layer, q the first
256 of each 512-wide block, per-sequence offsets), post_attention_layernorm
(add + RMSNorm), the routed experts' and the shared expert's SwiGLU. The
projections' outputs are random stand-ins."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import higgs_amd as H
import oracle as O
from higgs_amd._lib import ACT_SILU
from bits import exact_frac, ulp_dist
from gpu_util import to_host

pytestmark = pytest.mark.gpu


def _layers(dev, dt, T, n_layers, seed):
    """Buffers of an n-layer decode step: the residual chain and every op's
    inputs and outputs (Qwen3-Next-80B-A3B shapes)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def rnd(*shape, mean=0.0, std=1.0):
        t = torch.empty(shape, dtype=torch.float32, device=dev)
        t.normal_(mean, std, generator=g)
        return t.to(dt)

    Hd, Hv, Dv, Hq, Hk, D, E, I = 2048, 32, 128, 16, 2, 256, 10, 512
    L = dict(h0=rnd(T, Hd), w_in=rnd(Hd, mean=1.0, std=0.02), w_post=rnd(Hd, mean=1.0, std=0.02),
             w_g=rnd(Dv, mean=1.0, std=0.02), wq=rnd(D, mean=1.0, std=0.02),
             wk=rnd(D, mean=1.0, std=0.02),
             offsets=torch.randint(1, 32769, (T,), dtype=torch.int32, device=dev, generator=g),
             layers=[])
    for layer in range(n_layers):
        d = dict(r_prev=rnd(T, Hd), r_attn=rnd(T, Hd), gate=rnd(T, E, I), up=rnd(T, E, I),
                 sgate=rnd(T, I), sup=rnd(T, I))
        if layer % 4 == 3:
            d["q"] = rnd(T, Hq, 2 * D)[:, :, :D]
            d["k"] = rnd(T, Hk, D)
        else:
            d["y"] = rnd(T, Hv, Dv)
            d["z"] = rnd(T, Hv // 2, 768)[:, :, 512:].unflatten(-1, (2, Dv))
        L["layers"].append(d)
    return L


def _outputs(L, dev, dt, T):
    Hd, Hv, Dv, Hq, Hk, D, E, I = 2048, 32, 128, 16, 2, 256, 10, 512
    e = lambda *s: torch.full(s, float("nan"), dtype=dt, device=dev)
    outs = []
    for d in L["layers"]:
        o = dict(h_a=e(T, Hd), y_a=e(T, Hd), h_b=e(T, Hd), y_b=e(T, Hd), act=e(T, E, I),
                 sact=e(T, I))
        if "q" in d:
            o["qo"], o["ko"] = e(T, Hq, D), e(T, Hk, D)
        else:
            o["go"] = e(T, Hv, Dv)
        outs.append(o)
    return outs


def _record(L, outs, dt):
    seq = H.OpSequence(dt, L["h0"].device)
    h = L["h0"]
    for d, o in zip(L["layers"], outs):
        seq.add_rms_norm(h, d["r_prev"], L["w_in"], 1e-6, o["y_a"], o["h_a"])
        if "q" in d:
            seq.qk_norm_rope(d["q"], d["k"], L["wq"], L["wk"], 1e-6, 64, 1e7, o["qo"], o["ko"],
                             offsets=L["offsets"])
        else:
            seq.gated_rms_norm(d["y"], d["z"], L["w_g"], 1e-6, o["go"])
        seq.add_rms_norm(o["h_a"], d["r_attn"], L["w_post"], 1e-6, o["y_b"], o["h_b"])
        seq.glu(ACT_SILU, d["gate"], d["up"], o["act"])
        seq.glu(ACT_SILU, d["sgate"], d["sup"], o["sact"])
        h = o["h_b"]
    return seq


def _separate(L, outs, T):
    """The same ops as the separate calls, into `outs`."""
    h = L["h0"]
    for d, o in zip(L["layers"], outs):
        H.add_rms_norm(h[:T], d["r_prev"][:T], L["w_in"], 1e-6, h_out=o["h_a"][:T], out=o["y_a"][:T])
        if "q" in d:
            qo, ko = H.qk_norm_rope(d["q"][:T].unsqueeze(1), d["k"][:T].unsqueeze(1), L["wq"],
                                    L["wk"], 1e-6, 64, 1e7, 1.0, 0, offsets=L["offsets"][:T])
            o["qo"][:T] = qo[:, :, 0, :]
            o["ko"][:T] = ko[:, :, 0, :]
        else:
            H.gated_rms_norm(d["y"][:T], d["z"][:T], L["w_g"], 1e-6, out=o["go"][:T])
        H.add_rms_norm(o["h_a"][:T], d["r_attn"][:T], L["w_post"], 1e-6, h_out=o["h_b"][:T],
                       out=o["y_b"][:T])
        H.swiglu(d["gate"][:T], d["up"][:T], out=o["act"][:T])
        H.swiglu(d["sgate"][:T], d["sup"][:T], out=o["sact"][:T])
        h = o["h_b"]


def _same_bits(a, b, what):
    a16, b16 = a.view(torch.int16), b.view(torch.int16)
    bad = (a16 != b16)
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} elements differ, first at {bad.nonzero()[0].tolist()}"


@pytest.mark.parametrize("dt,T,n_layers", [(torch.bfloat16, 64, 8), (torch.float16, 9, 4)])
def test_op_sequence_matches_the_separate_calls_bitwise(dev, dt, T, n_layers):
    """Every output of an n-layer op sequence (the full 64-sequence batch in
    bf16; 9 sequences in f16) equals the separate calls' bit for bit."""
    L = _layers(dev, dt, T, n_layers, 71)
    got, ref = _outputs(L, dev, dt, T), _outputs(L, dev, dt, T)
    seq = _record(L, got, dt)
    print(f"[opseq] {len(seq)} ops, {T} tokens, {dt}", flush=True)
    seq.run(T)
    _separate(L, ref, T)
    torch.cuda.synchronize()
    for layer, (g, r) in enumerate(zip(got, ref)):
        for k in g:
            _same_bits(g[k], r[k], f"layer {layer} {k}")


def test_op_sequence_residual_chain_against_the_oracle(dev):
    """Two layers' residual chain (h = x + r, y = rms_norm(h)) of the op
    sequence against the oracle's add and RMSNorm, composed on the CPU."""
    T, dt = 64, torch.bfloat16
    L = _layers(dev, dt, T, 2, 72)
    got = _outputs(L, dev, dt, T)
    _record(L, got, dt).run(T)
    torch.cuda.synchronize()
    h = to_host(L["h0"])
    for layer, (d, o) in enumerate(zip(L["layers"], got)):
        for r, w, hk, yk in ((d["r_prev"], L["w_in"], "h_a", "y_a"),
                             (d["r_attn"], L["w_post"], "h_b", "y_b")):
            h = O.add(h, to_host(r), O.BF16)
            y = O.rms_norm(h, O.BF16, to_host(w), O.BF16, 1e-6)
            assert np.array_equal(to_host(o[hk]), h), f"layer {layer} {hk}"
            gy = to_host(o[yk])
            assert ulp_dist(gy, y, O.BF16).max() <= 1 and exact_frac(gy, y, O.BF16) >= 0.9999


def test_op_sequence_fewer_tokens_and_a_foreign_list(dev):
    """A run over the first 5 tokens writes only their rows; a list the upload
    did not write (zeros) launches and touches nothing."""
    T, dt = 16, torch.bfloat16
    L = _layers(dev, dt, T, 4, 73)
    got, ref = _outputs(L, dev, dt, T), _outputs(L, dev, dt, T)
    seq = _record(L, got, dt)
    seq.run(5)
    _separate(L, ref, 5)
    torch.cuda.synchronize()
    for layer, (g, r) in enumerate(zip(got, ref)):
        for k in g:
            _same_bits(g[k][:5], r[k][:5], f"layer {layer} {k}")
            assert bool(torch.isnan(g[k][5:].float()).all()), f"layer {layer} {k}: rows past 5 written"
    from higgs_amd import _lib
    blank = torch.zeros(int(_lib.lib().hgk_op_list_bytes(len(seq))) + 16, dtype=torch.uint8,
                        device=dev)
    before = {k: v.clone() for k, v in got[0].items()}
    _lib.check(_lib.lib().hgk_op_list_run(_lib.BF16, H.ops._ptr(blank), len(seq), T,
                                          H.ops._stream(blank.device)))
    # the f16 kernel given the bf16 list is also refused by the list's header
    _lib.check(_lib.lib().hgk_op_list_run(_lib.F16, H.ops._ptr(seq._list), len(seq), T,
                                          H.ops._stream(blank.device)))
    torch.cuda.synchronize()
    for k, v in got[0].items():
        _same_bits(v, before[k], f"foreign list {k}")
