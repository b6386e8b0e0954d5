"""Benchmark of the per-layer op kernels on one MI355X.

Default workload: the Gemma-2-9B-shaped prefill ops over 16384 tokens (batch
4 x seq 4096), the largest single-GPU configuration: 4-bit QuantizedEmbedding
gather (vocab 256000 x hidden 3584, group 64) scaled by bf16(sqrt(3584)) ->
(1+w) RMSNorm [16384, 3584] written in f32 -> RoPE (head_dim 256, theta 1e4)
on q [4,16,4096,256] and k [4,8,4096,256] -> GeGLU [16384, 14336] written in
f32. One step = one pass of the chain over one batch of synthetic inputs
already resident in HBM. The metric is achieved HBM bandwidth: algorithmic
bytes (every input element read once, every output written once,
weights/tables once; the gather gets no reuse credit) per second.

    python bench.py [--steps K] [--warmup W] [--settle S] [--config NAME] [--table] [--no-cpu]

Prints ONE JSON line. --table additionally measures every workload and writes
gpurun_out/bench_table.json. Input/output buffer sets rotate so the bytes
touched per pass exceed the 256 MB Infinity Cache.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA, MI355X
BF16, F32, F16, U32, I32 = 1, 0, 2, 3, 4
SILU, GELU = 0, 1


def _vp(t):
    return C.c_void_p(t.data_ptr())


def _i64s(vals):
    return (C.c_int64 * len(vals))(*[int(v) for v in vals])


class Kernel:
    """One launch type: a C-ABI entry point with one pre-built ctypes argument
    tuple per buffer set (the stream is the last argument).

    The tuples carry raw device addresses only, so `keep` must hold every
    tensor they point into: a tensor freed after the builder returns would go
    back to torch's caching allocator, and graph capture (which empties that
    cache) would unmap it under the launches."""

    def __init__(self, name, nbytes, fn, argsets, tokens=0, keep=(), cpu=None, flops=0,
                 wbytes=None):
        self.name, self.bytes, self.fn, self.tokens = name, nbytes, fn, tokens
        self.flops = flops  # MFMA-bound kernels: algorithmic flops per launch
        self.wbytes = wbytes  # of `bytes`, those written (the rest are read)
        self.argsets = [tuple(a) for a in argsets]
        self.keep = keep
        self.cpu = cpu  # (kind, params) for the oracle's timing of the same op

    def launch(self, s):
        st = self.fn(*self.argsets[s])
        if st:
            raise RuntimeError(f"{self.name}: status {st}")


class Workload:
    def __init__(self, name, config, kernels, nsets, tokens, graph=False, cpu_sample=None):
        self.name, self.config, self.kernels = name, config, kernels
        self.nsets, self.tokens, self.graph, self.cpu_sample = nsets, tokens, graph, cpu_sample

    @property
    def bytes(self):
        return sum(k.bytes for k in self.kernels)

    def step(self, i):
        s = i % self.nsets
        for k in self.kernels:
            k.launch(s)


# ---------------------------------------------------------------- builders
class Ctx:
    def __init__(self):
        import torch

        from higgs_amd import _lib

        self.torch = torch
        self.lib = _lib.lib()
        self.dev = torch.device("cuda:0")
        self.stream = C.c_void_p(torch.cuda.current_stream(self.dev).cuda_stream)
        self.gen = torch.Generator(device=self.dev)
        self.gen.manual_seed(2)

    def check(self, st):
        if st != 0:
            raise RuntimeError(self.lib.hgk_last_error().decode())

    def randn(self, shape, dtype, mean=0.0, std=1.0):
        t = self.torch.empty(shape, dtype=self.torch.float32, device=self.dev)
        t.normal_(mean, std, generator=self.gen)
        return t.to(dtype)

    def empty(self, shape, dtype):
        return self.torch.empty(shape, dtype=dtype, device=self.dev)

    def qtable(self, V, Hd, group=64):
        torch = self.torch
        wq = torch.randint(0, 2 ** 32, (V, Hd // 8), dtype=torch.int64, device=self.dev,
                           generator=self.gen).to(torch.int32)
        sc = (torch.rand((V, Hd // group), device=self.dev, generator=self.gen) * 0.015 + 0.005)
        bi = (torch.rand((V, Hd // group), device=self.dev, generator=self.gen) * 0.2 - 0.1)
        return wq, sc.to(torch.bfloat16), bi.to(torch.bfloat16)

    def qtable_experts(self, E, N, K, group=64):
        torch = self.torch
        wq = torch.randint(0, 2 ** 32, (E, N, K // 8), dtype=torch.int64, device=self.dev,
                           generator=self.gen).to(torch.int32)
        sc = (torch.rand((E, N, K // group), device=self.dev, generator=self.gen) * 0.015 + 0.005)
        bi = (torch.rand((E, N, K // group), device=self.dev, generator=self.gen) * 0.2 - 0.1)
        return wq, sc.to(torch.bfloat16), bi.to(torch.bfloat16)

    def ids(self, n, V):
        return self.torch.randint(0, V, (n,), dtype=self.torch.int32, device=self.dev,
                                  generator=self.gen)


def nsets_for(set_bytes, target=1 << 30):
    return max(2, math.ceil(target / max(set_bytes, 1)))


def nsets_per_kernel(kernel_bytes, target=1 << 30):
    """Buffer sets such that every kernel's launches, timed back to back over
    the sets, touch at least `target` bytes: twice and more the 256 MB
    Infinity Cache, so no kernel is timed on cache hits."""
    return max(2, math.ceil(target / max(1, min(kernel_bytes))))


def qtables(cx, V, Hd, target=600 << 20):
    """Enough copies of a 4-bit table that rotating over them exceeds the
    Infinity Cache."""
    tb = V * (Hd // 2 + 4 * (Hd // 64))
    return [cx.qtable(V, Hd) for _ in range(max(1, math.ceil(target / tb)))]


def _f(x):
    return C.c_float(x)


def k_embed(cx, name, sets, tabs, V, Hd, n, scale=0.0, group=64):
    """4-bit embedding gather; buffer set s reads table tabs[s % len(tabs)] (one
    table per set, so back-to-back launches cannot find the table in the
    256 MB Infinity Cache)."""
    nbytes = n * (Hd // 2 + 2 * 2 * (Hd // group) + 4 + Hd * 2)
    args = []
    for s, (ids, out) in enumerate(sets):
        wq, sc, bi = tabs[s % len(tabs)]
        args.append((_vp(ids), I32, n, _vp(wq), _vp(sc), _vp(bi), BF16, V, Hd, group, 4,
                     _f(scale), _vp(out), Hd, cx.stream))
    return Kernel(name, nbytes, cx.lib.hgk_quantized_embedding, args, n, keep=(sets, tabs),
                  cpu=("qembed", dict(V=V, H=Hd, n=n, scale=scale, group=group)),
                  wbytes=n * Hd * 2)


def k_rmsnorm(cx, name, sets, w, rows, n, eps, plus_one=0, ydt=BF16):
    nbytes = rows * n * 2 + rows * n * (4 if ydt == F32 else 2) + n * 2
    args = [(_vp(x), BF16, n, _vp(w), BF16, plus_one, _f(eps), _vp(y), ydt, n, rows, n,
             cx.stream) for x, y in sets]
    return Kernel(name, nbytes, cx.lib.hgk_rms_norm, args, rows, keep=(sets, w),
                  cpu=("rms", dict(rows=rows, n=n, eps=eps, plus_one=plus_one, ydt=ydt)),
                  wbytes=rows * n * (4 if ydt == F32 else 2))


def k_embed_norm(cx, name, sets, tabs, w, V, Hd, n, eps, scale=0.0, group=64, plus_one=0,
                 ydt=BF16):
    """Embedding gather + the first RMSNorm in one kernel: writes h and y (one
    table per buffer set, as k_embed)."""
    nbytes = n * (Hd // 2 + 2 * 2 * (Hd // group) + 4 + Hd * 2 + Hd * (4 if ydt == F32 else 2))
    nbytes += Hd * 2
    args = []
    for s, (ids, h, y) in enumerate(sets):
        wq, sc, bi = tabs[s % len(tabs)]
        args.append((_vp(ids), I32, n, _vp(wq), _vp(sc), _vp(bi), BF16, V, Hd, group, 4,
                     _f(scale), _vp(h), Hd, _vp(w), BF16, plus_one, _f(eps), _vp(y), ydt, Hd,
                     cx.stream))
    return Kernel(name, nbytes, cx.lib.hgk_quantized_embedding_rms_norm, args, n,
                  keep=(sets, tabs, w),
                  cpu=("qembed_rms", dict(V=V, H=Hd, n=n, scale=scale, group=group, eps=eps)),
                  wbytes=n * Hd * (2 + (4 if ydt == F32 else 2)))


def k_add_rmsnorm(cx, name, sets, w, rows, n, eps):
    """Residual add + RMSNorm: reads x and r, writes h and y."""
    nbytes = 4 * rows * n * 2 + n * 2
    args = [(BF16, _vp(x), n, _vp(r), n, _vp(w), BF16, 0, _f(eps), _vp(h), n, _vp(y), BF16, n,
             rows, n, cx.stream) for x, r, h, y in sets]
    return Kernel(name, nbytes, cx.lib.hgk_add_rms_norm, args, rows, keep=(sets, w),
                  cpu=("add_rms", dict(rows=rows, n=n, eps=eps)), wbytes=2 * rows * n * 2)


def k_glu(cx, name, sets, rows, n, act, ydt=BF16):
    nbytes = rows * n * (2 + 2 + (4 if ydt == F32 else 2))
    args = [(act, BF16, _vp(g), n, _vp(u), n, _vp(o), ydt, n, rows, n, cx.stream)
            for g, u, o in sets]
    return Kernel(name, nbytes, cx.lib.hgk_glu, args, rows, keep=(sets,),
                  cpu=("glu", dict(rows=rows, n=n, act=act, ydt=ydt)),
                  wbytes=rows * n * (4 if ydt == F32 else 2))


def k_qkrope(cx, name, sets, B, L, Hq, Hk, D, dims, base, freqs=None, wq=None, wk=None,
             eps=1e-6, offsets=None, q_block=None):
    """q/k from projection layout [B,L,H,D] (q heads q_block wide), out [B,H,L,D]."""
    qb = q_block or D
    nbytes = B * L * (Hq + Hk) * D * 2 * 2
    if wq is not None:
        nbytes += 2 * D * 2
    if offsets is not None:
        nbytes += B * 4
    fr = None if freqs is None else (C.c_float * len(freqs))(*freqs)
    qs = _i64s([L * Hq * qb, Hq * qb, qb])
    ks = _i64s([L * Hk * D, Hk * D, D])
    qos = _i64s([Hq * L * D, D, L * D])
    kos = _i64s([Hk * L * D, D, L * D])

    args = [(BF16, _vp(q), qs, _vp(qo), qos, Hq, None if wq is None else _vp(wq),
             _vp(k), ks, _vp(ko), kos, Hk, None if wk is None else _vp(wk), BF16, _f(eps),
             B, L, D, dims, _f(base), _f(1.0), fr, 0,
             None if offsets is None else _vp(offsets), cx.stream) for q, k, qo, ko in sets]
    return Kernel(name, nbytes, cx.lib.hgk_qk_norm_rope, args, B * L,
                  keep=(sets, wq, wk, offsets, fr, qs, ks, qos, kos),
                  cpu=("rope", dict(B=B, L=L, Hq=Hq, Hk=Hk, D=D, dims=dims, base=base,
                                    freqs=freqs, norm=wq is not None, eps=eps,
                                    offsets=offsets is not None)),
                  wbytes=B * L * (Hq + Hk) * D * 2)


def k_gated(cx, name, sets, w, rows, n, eps, zrow, zgroup, zgs):
    nbytes = 3 * rows * n * 2 + n * 2
    args = [(BF16, _vp(y), n, _vp(z), zrow, zgroup, zgs, _vp(w), BF16, _f(eps), _vp(o), BF16,
             n, rows, n, cx.stream) for y, z, o in sets]
    return Kernel(name, nbytes, cx.lib.hgk_gated_rms_norm, args, rows, keep=(sets, w),
                  cpu=("gated", dict(rows=rows, n=n, eps=eps)), wbytes=rows * n * 2)


def wl_llama_chain(cx):
    torch = cx.torch
    V, Hd, T, B, L, I = 128256, 2048, 4096, 4, 1024, 8192
    tabs = qtables(cx, V, Hd)
    from higgs_amd.ops import llama3_rope_freqs
    freqs = llama3_rope_freqs(500000.0, 64, 32.0, 1.0, 4.0, 8192.0)
    w = cx.randn((Hd,), torch.bfloat16, 1.0, 0.02)
    ns = nsets_per_kernel([T * (Hd // 2 + 4 * (Hd // 64) + 4 + 2 * Hd), T * Hd * 4,
                           B * L * 40 * 64 * 4, T * I * 6])
    hs = [cx.empty((T, Hd), torch.bfloat16) for _ in range(ns)]
    emb = [(cx.ids(T, V), hs[s]) for s in range(ns)]
    # the norm reads the embedding output of another set (written a whole
    # step earlier), so it is timed on HBM rather than on the cache
    nrm = [(hs[(s + ns // 2) % ns], cx.empty((T, Hd), torch.bfloat16)) for s in range(ns)]
    rp = [(cx.randn((B, L, 32, 64), torch.bfloat16), cx.randn((B, L, 8, 64), torch.bfloat16),
           cx.empty((B, 32, L, 64), torch.bfloat16), cx.empty((B, 8, L, 64), torch.bfloat16))
          for _ in range(ns)]
    gl = [(cx.randn((T, I), torch.bfloat16), cx.randn((T, I), torch.bfloat16),
           cx.empty((T, I), torch.bfloat16)) for _ in range(ns)]
    ks = [k_embed(cx, "qembed_gather", emb, tabs, V, Hd, T),
          k_rmsnorm(cx, "rms_norm", nrm, w, T, Hd, 1e-5),
          k_qkrope(cx, "rope_llama3", rp, B, L, 32, 8, 64, 64, 500000.0, freqs=freqs),
          k_glu(cx, "swiglu", gl, T, I, SILU)]
    cfg = {"workload": "llama3.2-1b layer-op chain", "tokens": T, "batch": B, "seq_len": L,
           "hidden": Hd, "vocab": V, "intermediate": I, "q_heads": 32, "kv_heads": 8,
           "head_dim": 64, "rope": "llama3 factor 32, theta 5e5", "quant": "4-bit g64",
           "buffer_sets": ns, "tables": len(tabs)}
    return Workload("llama32_1b_chain", cfg, ks, ns, T, cpu_sample=cpu_sample_llama)


def wl_llama_chain_fused(cx):
    """The Llama-3.2-1B chain with the embedding gather and the first RMSNorm
    in one kernel (gather+norm -> llama3 RoPE -> SwiGLU over 4096 tokens)."""
    torch = cx.torch
    V, Hd, T, B, L, I = 128256, 2048, 4096, 4, 1024, 8192
    tabs = qtables(cx, V, Hd)
    from higgs_amd.ops import llama3_rope_freqs
    freqs = llama3_rope_freqs(500000.0, 64, 32.0, 1.0, 4.0, 8192.0)
    w = cx.randn((Hd,), torch.bfloat16, 1.0, 0.02)
    ns = nsets_per_kernel([T * (Hd // 2 + 4 * (Hd // 64) + 4 + 4 * Hd), B * L * 40 * 64 * 4,
                           T * I * 6])
    emb = [(cx.ids(T, V), cx.empty((T, Hd), torch.bfloat16), cx.empty((T, Hd), torch.bfloat16))
           for _ in range(ns)]
    rp = [(cx.randn((B, L, 32, 64), torch.bfloat16), cx.randn((B, L, 8, 64), torch.bfloat16),
           cx.empty((B, 32, L, 64), torch.bfloat16), cx.empty((B, 8, L, 64), torch.bfloat16))
          for _ in range(ns)]
    gl = [(cx.randn((T, I), torch.bfloat16), cx.randn((T, I), torch.bfloat16),
           cx.empty((T, I), torch.bfloat16)) for _ in range(ns)]
    ks = [k_embed_norm(cx, "qembed_rms_norm", emb, tabs, w, V, Hd, T, 1e-5),
          k_qkrope(cx, "rope_llama3", rp, B, L, 32, 8, 64, 64, 500000.0, freqs=freqs),
          k_glu(cx, "swiglu", gl, T, I, SILU)]
    cfg = {"workload": "llama3.2-1b layer-op chain, embedding+norm fused", "tokens": T,
           "batch": B, "seq_len": L, "hidden": Hd, "vocab": V, "intermediate": I,
           "buffer_sets": ns, "tables": len(tabs)}
    return Workload("llama32_1b_chain_fused", cfg, ks, ns, T)


def wl_block_boundary(cx):
    """Residual add + RMSNorm at the Llama-3.2-1B (4096 x 2048) and Qwen3-8B
    (16384 x 4096) prefill shapes."""
    torch = cx.torch
    ks, tot = [], 0
    for name, rows, n, eps in (("add_rms_norm_llama", 4096, 2048, 1e-5),
                               ("add_rms_norm_qwen3", 16384, 4096, 1e-6)):
        ns = nsets_for(rows * n * 8, 2 << 30)
        w = cx.randn((n,), torch.bfloat16, 1.0, 0.02)
        sets = [(cx.randn((rows, n), torch.bfloat16), cx.randn((rows, n), torch.bfloat16),
                 cx.empty((rows, n), torch.bfloat16), cx.empty((rows, n), torch.bfloat16))
                for _ in range(ns)]
        ks.append(k_add_rmsnorm(cx, name, sets, w, rows, n, eps))
        tot = max(tot, ns)
    for k in ks:  # equal set counts so one step index serves both
        k.argsets = [k.argsets[i % len(k.argsets)] for i in range(tot)]
    cfg = {"workload": "residual add + rmsnorm (block boundary)", "shapes": "4096x2048, 16384x4096",
           "buffer_sets": tot}
    return Workload("block_boundary_add_rms_norm", cfg, ks, tot, 4096 + 16384)


def k_qmm(cx, name, sets, tab, E, N, K, T, top_k, x_div, group=64):
    """gather_qmm over (token, expert) pairs; bytes = the distinct experts'
    weights (no credit for re-reads) + x + y + the expert ids."""
    wq, sc, bi = tab
    P = T * top_k
    per_expert = N * K // 2 + 2 * N * (K // group) * 2
    uniq = sum(len(set(st[1].tolist())) for st in sets) / len(sets)
    x_rows = P // x_div
    nbytes = int(uniq * per_expert) + x_rows * K * 2 + P * N * 2 + P * 4
    args = [(BF16, _vp(x), x_rows, K, x_div, None, _vp(wq), _vp(sc), _vp(bi), BF16, E, N, K,
             group, 4, _vp(exd), I32, P, _vp(y), N, cx.stream) for x, ex, exd, y in sets]
    return Kernel(name, nbytes, cx.lib.hgk_gather_qmm, args, T, keep=(sets, tab),
                  cpu=("qmm", dict(E=E, N=N, K=K, group=group, x_div=x_div)))


def wl_qwen3_next_moe_decode(cx):
    """Qwen3-Next-80B-A3B routed experts for one decode step of 64 sequences:
    top-10 of 512 experts; gate and up (512 x 2048) gather_qmm, SwiGLU, down
    (2048 x 512) gather_qmm, 4-bit group-64 weights;
    two layers' expert tables (~1.8 GB) alternate so the weights stream from
    HBM."""
    torch = cx.torch
    T, top_k, E, D, I = 64, 10, 512, 2048, 512
    P = T * top_k
    layers = 2
    tabs = []
    for _ in range(layers):
        tabs.append({nm: cx.qtable_experts(E, N, K) for nm, N, K in
                     (("gate", I, D), ("up", I, D), ("down", D, I))})
    ns = 8
    g = torch.Generator().manual_seed(5)
    exs = [torch.stack([torch.randperm(E, generator=g)[:top_k] for _ in range(T)]).reshape(-1)
           .to(torch.int32) for _ in range(ns)]
    xs = [cx.randn((T, D), torch.bfloat16) for _ in range(ns)]
    exd = [ex.to(cx.dev) for ex in exs]
    ks, outs = [], {}
    for nm, N, K, xdiv in (("gate", I, D, top_k), ("up", I, D, top_k), ("down", D, I, 1)):
        outs[nm] = [cx.empty((P, N), torch.bfloat16) for _ in range(ns)]
        # buffer set si uses layer si % layers's expert tables
        per_set = []
        for si in range(ns):
            x = xs[si] if nm != "down" else cx.randn((P, I), torch.bfloat16)
            st = (x, exs[si], exd[si], outs[nm][si])
            per_set.append(k_qmm(cx, f"qmm_{nm}", [st], tabs[si % layers][nm], E, N, K, T,
                                 top_k, xdiv))
        k = per_set[0]
        k.argsets = [kk.argsets[0] for kk in per_set]
        k.bytes = sum(kk.bytes for kk in per_set) // ns
        k.keep = tuple(kk.keep for kk in per_set)
        ks.append(k)
    act = [(outs["gate"][si], outs["up"][si], cx.empty((P, I), torch.bfloat16))
           for si in range(ns)]
    ks.insert(2, k_glu(cx, "swiglu_moe", act, P, I, SILU))
    cfg = {"workload": "qwen3-next-80b-a3b routed experts, one decode step", "sequences": T,
           "experts": E, "top_k": top_k, "hidden": D, "expert_dim": I, "quant": "4-bit g64",
           "expert_tables": layers, "buffer_sets": ns}
    return Workload("qwen3_next_moe_decode", cfg, ks, ns, T)


def k_qlinear(cx, name, sets, M, N, K, group=64):
    """quantized_matmul x [M, K] . W^T (W [N, K] 4-bit group 64): bytes =
    weights + scales/biases + x + y; flops = 2 M N K."""
    nbytes = N * K // 2 + 2 * N * (K // group) * 2 + M * K * 2 + M * N * 2
    args = [(BF16, _vp(x), M, K, _vp(wq), _vp(sc), _vp(bi), BF16, N, K, group, 4, _vp(y), N,
             cx.stream) for x, (wq, sc, bi), y in sets]
    return Kernel(name, nbytes, cx.lib.hgk_quantized_matmul, args, M, keep=(sets,),
                  cpu=("qlinear", dict(M=M, N=N, K=K, group=group)), flops=2 * M * N * K)


def wl_qwen3_next_qlinear(cx):
    """Qwen3-Next-80B-A3B GatedDeltaNet input projection in_proj_qkvz
    (hidden 2048 -> 2 x 16 x 128 + 2 x 32 x 128 = 12288, 4-bit group 64) as
    QLinear::forward runs it: a decode step of 64 sequences (M = 64; 24 weight
    sets, ~340 MB, rotate so the weights stream from HBM) and a 4096-token
    prefill (M = 4096, matrix-core bound)."""
    torch = cx.torch
    N, K = 12288, 2048
    nd = 24
    tabs = [tuple(t[0] for t in cx.qtable_experts(1, N, K)) for _ in range(nd)]
    dec = [(cx.randn((64, K), torch.bfloat16), tabs[i], cx.empty((64, N), torch.bfloat16))
           for i in range(nd)]
    npf = 2
    pre = [(cx.randn((4096, K), torch.bfloat16), tabs[i], cx.empty((4096, N), torch.bfloat16))
           for i in range(npf)]
    k_pre = k_qlinear(cx, "qlinear_prefill_4096", pre, 4096, N, K)
    k_pre.argsets = [k_pre.argsets[i % npf] for i in range(nd)]
    ks = [k_qlinear(cx, "qlinear_decode_64", dec, 64, N, K), k_pre]
    cfg = {"workload": "qwen3-next-80b-a3b in_proj_qkvz quantized_matmul", "N": N, "K": K,
           "quant": "4-bit g64", "decode_rows": 64, "prefill_rows": 4096, "weight_sets": nd}
    return Workload("qwen3_next_qlinear", cfg, ks, nd, 64 + 4096)


def wl_qwen3_next_moe_prefill(cx, fused=False):
    """Qwen3-Next-80B-A3B routed experts over a 4096-token prefill: top-10 of
    512 experts (40,960 pairs, ~80 per expert), gate and up (512 x 2048)
    gather_qmm, SwiGLU, down (2048 x 512) gather_qmm, 4-bit group 64 -- the
    expert-grouped matrix-core path; flops = 2 x pairs x N x K per
    projection. fused: gate, up and SwiGLU as one hgk_gather_qmm_swiglu
    launch."""
    torch = cx.torch
    T, top_k, E, D, I = 4096, 10, 512, 2048, 512
    P = T * top_k
    tab = {nm: cx.qtable_experts(E, N, K) for nm, N, K in
           (("gate", I, D), ("up", I, D), ("down", D, I))}
    ns = 2
    g = torch.Generator().manual_seed(6)
    exs = [torch.stack([torch.randperm(E, generator=g)[:top_k] for _ in range(T)]).reshape(-1)
           .to(torch.int32) for _ in range(ns)]
    exd = [ex.to(cx.dev) for ex in exs]
    xs = [cx.randn((T, D), torch.bfloat16) for _ in range(ns)]
    acts = [cx.randn((P, I), torch.bfloat16) for _ in range(ns)]
    ks, outs = [], {}
    for nm, N, K, xdiv in (("gate", I, D, top_k), ("up", I, D, top_k), ("down", D, I, 1)):
        outs[nm] = [cx.empty((P, N), torch.bfloat16) for _ in range(ns)]
        sets = [((xs[si] if nm != "down" else acts[si]), exs[si], exd[si], outs[nm][si])
                for si in range(ns)]
        k = k_qmm(cx, f"qmm_{nm}_prefill", sets, tab[nm], E, N, K, T, top_k, xdiv)
        k.flops = 2 * P * N * K
        ks.append(k)
    act = [(outs["gate"][si], outs["up"][si], cx.empty((P, I), torch.bfloat16)) for si in range(ns)]
    ks.insert(2, k_glu(cx, "swiglu_moe_prefill", act, P, I, SILU))
    if fused:
        sets = [(xs[si], exs[si], exd[si], act[si][2]) for si in range(ns)]
        kf = k_qmm_swiglu(cx, "qmm_gate_up_swiglu_prefill", sets, tab["gate"], tab["up"], E, I, D,
                          T, top_k)
        kf.flops = 2 * 2 * P * I * D
        ks = [kf, ks[3]]
    cfg = {"workload": "qwen3-next-80b-a3b routed experts, 4096-token prefill" +
           (", gate + up + SwiGLU in one launch" if fused else ""), "tokens": T,
           "experts": E, "top_k": top_k, "hidden": D, "expert_dim": I, "quant": "4-bit g64",
           "buffer_sets": ns}
    return Workload("qwen3_next_moe_prefill" + ("_fused" if fused else ""), cfg, ks, ns, T)


def k_gdn(cx, name, sets, wq, wk, alog, dtb, B, T, Hk, Dk, Hv, Dv):
    """Gated-delta recurrence with the fused q/k norm; bytes = state read and
    written once + q, k, v, a, b read + y written."""
    nbytes = (2 * B * Hv * Dv * Dk * 2 + B * T * (2 * Hk * Dk + Hv * Dv + 2 * Hv) * 2 +
              B * T * Hv * Dv * 2 + 2 * Dk * 2 + 2 * Hv * 4)
    args = [(BF16, _vp(q), _vp(k), _vp(v), _vp(alog), _vp(a), _vp(dtb), _vp(b), F32, _vp(st),
             _vp(wq), _vp(wk), _f(1e-6), B, T, Hk, Dk, Hv, Dv, _vp(y), _vp(so), cx.stream)
            for q, k, v, a, b, st, y, so in sets]
    return Kernel(name, nbytes, cx.lib.hgk_gated_delta, args, B * T,
                  keep=(sets, wq, wk, alog, dtb),
                  cpu=("gdn", dict(B=B, T=T, Hk=Hk, Dk=Dk, Hv=Hv, Dv=Dv)))


def _gdn_sets(cx, ns, B, T, Hk, Dk, Hv, Dv):
    torch = cx.torch
    r = lambda shape, lo, hi: (torch.rand(shape, device=cx.dev, generator=cx.gen) * (hi - lo) + lo
                               ).to(torch.bfloat16)
    return [(r((B, T, Hk, Dk), -1, 1), r((B, T, Hk, Dk), -1, 1), r((B, T, Hv, Dv), -1, 1),
             r((B, T, Hv), -1, 1), r((B, T, Hv), -1, 1), r((B, Hv, Dv, Dk), -0.1, 0.1),
             cx.empty((B, T, Hv, Dv), torch.bfloat16), cx.empty((B, Hv, Dv, Dk), torch.bfloat16))
            for _ in range(ns)]


def wl_qwen3_next_gdn(cx):
    """Qwen3-Next-80B-A3B linear-attention recurrence (Hk 16, Dk 128, Hv 32,
    Dv 128, bf16, the constant-weight q/k norm fused): one decode token for 64
    sequences (bound by the 1 MB bf16 state per sequence), and a 4 x 512-token
    prefill."""
    torch = cx.torch
    Hk, Dk, Hv, Dv = 16, 128, 32, 128
    from higgs_amd.ops import gdn_qk_norm_weights
    wq, wk = gdn_qk_norm_weights(Dk, torch.bfloat16, cx.dev)
    alog = (torch.rand(Hv, device=cx.dev, generator=cx.gen) - 1.0).contiguous()
    dtb = (torch.rand(Hv, device=cx.dev, generator=cx.gen) - 0.5).contiguous()
    ns = 8
    ks = [k_gdn(cx, "gdn_decode_64seq", _gdn_sets(cx, ns, 64, 1, Hk, Dk, Hv, Dv), wq, wk, alog,
                dtb, 64, 1, Hk, Dk, Hv, Dv),
          k_gdn(cx, "gdn_prefill_4x512", _gdn_sets(cx, ns, 4, 512, Hk, Dk, Hv, Dv), wq, wk, alog,
                dtb, 4, 512, Hk, Dk, Hv, Dv)]
    cfg = {"workload": "qwen3-next-80b-a3b gated-delta recurrence", "k_heads": Hk, "head_k_dim": Dk,
           "v_heads": Hv, "head_v_dim": Dv, "decode_sequences": 64, "prefill": "4 x 512",
           "buffer_sets": ns}
    return Workload("qwen3_next_gdn", cfg, ks, ns, 64 + 4 * 512)


def wl_rmsnorm_512(cx):
    torch = cx.torch
    rows, n = 512, 2048
    ns = nsets_for(rows * n * 4)
    sets = [(cx.randn((rows, n), torch.bfloat16), cx.empty((rows, n), torch.bfloat16))
            for _ in range(ns)]
    w = cx.randn((n,), torch.bfloat16, 1.0, 0.02)
    cfg = {"workload": "rmsnorm alone", "rows": rows, "hidden": n, "eps": 1e-5,
           "buffer_sets": ns}
    return Workload("rmsnorm_512x2048", cfg, [k_rmsnorm(cx, "rms_norm", sets, w, rows, n, 1e-5)],
                    ns, rows, graph=True)


def wl_qwen3_prefill(cx):
    torch = cx.torch
    B, L, Hd, I, D = 8, 2048, 4096, 12288, 128
    T = B * L
    ns = nsets_per_kernel([T * Hd * 4, T * 40 * D * 4, T * I * 6])
    w = cx.randn((Hd,), torch.bfloat16, 1.0, 0.02)
    wq = cx.randn((D,), torch.bfloat16, 1.0, 0.02)
    wk = cx.randn((D,), torch.bfloat16, 1.0, 0.02)
    nrm = [(cx.randn((T, Hd), torch.bfloat16), cx.empty((T, Hd), torch.bfloat16))
           for _ in range(ns)]
    rp = [(cx.randn((B, L, 32, D), torch.bfloat16), cx.randn((B, L, 8, D), torch.bfloat16),
           cx.empty((B, 32, L, D), torch.bfloat16), cx.empty((B, 8, L, D), torch.bfloat16))
          for _ in range(ns)]
    gl = [(cx.randn((T, I), torch.bfloat16), cx.randn((T, I), torch.bfloat16),
           cx.empty((T, I), torch.bfloat16)) for _ in range(ns)]
    ks = [k_rmsnorm(cx, "rms_norm", nrm, w, T, Hd, 1e-6),
          k_qkrope(cx, "qk_norm_rope", rp, B, L, 32, 8, D, D, 1e6, wq=wq, wk=wk, eps=1e-6),
          k_glu(cx, "swiglu", gl, T, I, SILU)]
    cfg = {"workload": "qwen3-8b prefill ops", "tokens": T, "batch": B, "seq_len": L,
           "hidden": Hd, "intermediate": I, "q_heads": 32, "kv_heads": 8, "head_dim": D,
           "buffer_sets": ns}
    return Workload("qwen3_8b_prefill", cfg, ks, ns, T, cpu_sample=cpu_sample_ops)


def wl_gemma2(cx):
    """Gemma-2-9B-shaped prefill ops over 16384 tokens (batch 4 x seq 4096):
    4-bit embedding gather x bf16(sqrt(3584)) -> (1+w) RMSNorm -> RoPE on q
    [4,16,4096,256] and k [4,8,4096,256] -> GeGLU [16384, 14336].

    Output dtypes are the reference's: its load-time `w + 1.0_f32` promotes
    every norm weight to f32, so the (1+w) norm writes f32
    (gemma2.rs:799-826), and gelu_approximate is built from f32 scalar
    arrays, so GeGLU on bf16 gate/up computes and writes f32
    (gemma2.rs:422-427)."""
    torch = cx.torch
    B, L, Hd, I, D, V = 4, 4096, 3584, 14336, 256, 256000
    T = B * L
    tabs = qtables(cx, V, Hd)
    ns = nsets_per_kernel([T * (Hd // 2 + 4 * (Hd // 64) + 4 + 2 * Hd), T * Hd * 6,
                           B * L * 24 * D * 4, T * I * 8])
    w = cx.randn((Hd,), torch.bfloat16, 0.0, 0.02)
    hs = [cx.empty((T, Hd), torch.bfloat16) for _ in range(ns)]
    emb = [(cx.ids(T, V), hs[s]) for s in range(ns)]
    # the norm reads the embedding output of another set (written a whole
    # step earlier), so it is timed on HBM rather than on the cache
    nrm = [(hs[(s + ns // 2) % ns], cx.empty((T, Hd), torch.float32)) for s in range(ns)]
    rp = [(cx.randn((B, L, 16, D), torch.bfloat16), cx.randn((B, L, 8, D), torch.bfloat16),
           cx.empty((B, 16, L, D), torch.bfloat16), cx.empty((B, 8, L, D), torch.bfloat16))
          for _ in range(ns)]
    gl = [(cx.randn((T, I), torch.bfloat16), cx.randn((T, I), torch.bfloat16),
           cx.empty((T, I), torch.float32)) for _ in range(ns)]
    ks = [k_embed(cx, "qembed_gather_x59.75", emb, tabs, V, Hd, T, scale=math.sqrt(3584.0)),
          k_rmsnorm(cx, "rms_norm_1p", nrm, w, T, Hd, 1e-6, plus_one=1, ydt=F32),
          k_qkrope(cx, "rope_d256", rp, B, L, 16, 8, D, D, 10000.0),
          k_glu(cx, "geglu_tanh", gl, T, I, GELU, ydt=F32)]
    cfg = {"workload": "gemma2-9b-shaped prefill ops", "tokens": T, "batch": B, "seq_len": L,
           "hidden": Hd, "vocab": V, "intermediate": I, "q_heads": 16, "kv_heads": 8,
           "head_dim": D, "quant": "4-bit g64", "embed_scale": "bf16(sqrt(3584)) = 59.75",
           "outputs": "embedding bf16, (1+w) norm f32, rope bf16, geglu f32",
           "buffer_sets": ns, "tables": len(tabs)}
    return Workload("gemma2_9b_prefill", cfg, ks, ns, T, cpu_sample=cpu_sample_gemma)


def _decode_sequence_sets(cx, S=64, n_layers=48):
    """Buffers of the 48-layer decode op sequence (64 sequences, one new token
    each), one set per rotation slot: per layer the input_layernorm (residual
    add + RMSNorm over hidden 2048, the residual chained from the previous
    layer), the gated RMSNorm (36 linear-attention layers: y [64, 32, 128], z
    read in place from in_proj_qkvz [64, 16, 768]) or the q/k RMSNorm +
    partial RoPE (12 full-attention layers: q the first 256 of each 512-wide
    block of [64, 16, 512], k [64, 2, 256], 64 rotated dims, theta 1e7,
    offsets uniform in 1..32768), the post_attention_layernorm (add + RMSNorm)
    and the routed experts' SwiGLU [64, 10, 512]. The projections' outputs are
    random stand-ins. Returns (sets, weights, offsets, bytes per sequence)."""
    torch = cx.torch
    Hd, nk, vpk, dv, Hq, Hk, D, E, I = 2048, 16, 2, 128, 16, 2, 256, 10, 512
    offs = torch.randint(1, 32769, (S,), dtype=torch.int32, device=cx.dev, generator=cx.gen)
    wts = dict(w_in=cx.randn((Hd,), torch.bfloat16, 1.0, 0.02),
               w_post=cx.randn((Hd,), torch.bfloat16, 1.0, 0.02),
               wg=cx.randn((dv,), torch.bfloat16, 1.0, 0.02),
               wq=cx.randn((D,), torch.bfloat16, 1.0, 0.02),
               wk=cx.randn((D,), torch.bfloat16, 1.0, 0.02))
    norm_b = 4 * S * Hd * 2 + Hd * 2
    per_seq = 0
    for layer in range(n_layers):
        per_seq += 2 * norm_b + S * E * I * 6
        per_seq += (S * (Hq * D + Hk * D) * 4 + 2 * D * 2 + S * 4 if layer % 4 == 3
                    else 3 * S * nk * vpk * dv * 2 + dv * 2)
    ns = nsets_for(per_seq, 1 << 30)
    sets = []
    for _ in range(ns):
        h = cx.randn((S, Hd), torch.bfloat16)
        layers = []
        for layer in range(n_layers):
            d = dict(x=h, r_prev=cx.randn((S, Hd), torch.bfloat16),
                     r_attn=cx.randn((S, Hd), torch.bfloat16),
                     h_a=cx.empty((S, Hd), torch.bfloat16), y_a=cx.empty((S, Hd), torch.bfloat16),
                     h_b=cx.empty((S, Hd), torch.bfloat16), y_b=cx.empty((S, Hd), torch.bfloat16),
                     gate=cx.randn((S, E, I), torch.bfloat16), up=cx.randn((S, E, I), torch.bfloat16),
                     act=cx.empty((S, E, I), torch.bfloat16))
            if layer % 4 == 3:
                d["q"] = cx.randn((S, Hq, 2 * D), torch.bfloat16)[:, :, :D]
                d["k"] = cx.randn((S, Hk, D), torch.bfloat16)
                d["qo"] = cx.empty((S, Hq, D), torch.bfloat16)
                d["ko"] = cx.empty((S, Hk, D), torch.bfloat16)
            else:
                d["y"] = cx.randn((S, nk * vpk, dv), torch.bfloat16)
                d["z"] = cx.randn((S, nk, 768), torch.bfloat16)[:, :, 512:].unflatten(-1, (vpk, dv))
                d["go"] = cx.empty((S, nk * vpk, dv), torch.bfloat16)
            layers.append(d)
            h = d["h_b"]
        sets.append(layers)
    return sets, wts, offs, per_seq


def _decode_cfg(S, n_layers, launches, ns):
    return {"workload": "qwen3-next-80b-a3b decode op sequence", "sequences": S, "layers": n_layers,
            "hidden": 2048, "value_heads": 32, "head_v_dim": 128, "q_heads": 16, "kv_heads": 2,
            "head_dim": 256, "rotary_dims": 64, "experts_per_token": 10, "expert_dim": 512,
            "hidden_norms": "residual add + rmsnorm", "launches": launches, "buffer_sets": ns}


def wl_qwen3_next_decode(cx):
    """48-layer op sequence of continuous-batching decode (64 sequences) as
    192 separate launches, replayed as captured graphs."""
    torch = cx.torch
    S = 64
    sets, W, offs, per_seq = _decode_sequence_sets(cx, S)
    ns = len(sets)
    kernels = []
    for layer in range(48):
        L = [st[layer] for st in sets]
        n1 = [(d["x"], d["r_prev"], d["h_a"], d["y_a"]) for d in L]
        kernels.append(k_add_rmsnorm(cx, "add_rms_norm", n1, W["w_in"], S, 2048, 1e-6))
        if layer % 4 == 3:
            rp = [(d["q"].unsqueeze(1), d["k"].unsqueeze(1), d["qo"], d["ko"]) for d in L]
            kernels.append(k_qkrope(cx, "qk_norm_partial_rope", rp, S, 1, 16, 2, 256, 64, 1e7,
                                    wq=W["wq"], wk=W["wk"], eps=1e-6, offsets=offs, q_block=512))
        else:
            gs = [(d["y"], d["z"].flatten(-2), d["go"]) for d in L]
            kernels.append(k_gated(cx, "gated_rms_norm", gs, W["wg"], S * 32, 128, 1e-6, 128, 2, 768))
        n2 = [(d["h_a"], d["r_attn"], d["h_b"], d["y_b"]) for d in L]
        kernels.append(k_add_rmsnorm(cx, "add_rms_norm", n2, W["w_post"], S, 2048, 1e-6))
        gl = [(d["gate"], d["up"], d["act"]) for d in L]
        kernels.append(k_glu(cx, "swiglu_experts", gl, S * 10, 512, SILU))
    return Workload("qwen3_next_decode", _decode_cfg(S, 48, len(kernels), ns), kernels, ns, S,
                    graph=True, cpu_sample=cpu_sample_ops)


def wl_qwen3_next_decode_opseq(cx):
    """The same 48-layer op sequence (same ops, same buffers) in one launch:
    one workgroup per sequence walks the 192 ops in the layer loop's order,
    each op waiting for the previous op's stores (hgk_op_list_run)."""
    from higgs_amd.ops import OpSequence
    torch = cx.torch
    S = 64
    sets, W, offs, per_seq = _decode_sequence_sets(cx, S)
    seqs, args = [], []
    for layers in sets:
        seq = OpSequence(torch.bfloat16, cx.dev)
        for d in layers:
            seq.add_rms_norm(d["x"], d["r_prev"], W["w_in"], 1e-6, d["y_a"], d["h_a"])
            if "q" in d:
                seq.qk_norm_rope(d["q"], d["k"], W["wq"], W["wk"], 1e-6, 64, 1e7, d["qo"], d["ko"],
                                 offsets=offs)
            else:
                seq.gated_rms_norm(d["y"], d["z"], W["wg"], 1e-6, d["go"])
            seq.add_rms_norm(d["h_a"], d["r_attn"], W["w_post"], 1e-6, d["y_b"], d["h_b"])
            seq.glu(SILU, d["gate"], d["up"], d["act"])
        seq.upload()
        seqs.append(seq)
        args.append((BF16, _vp(seq._list), len(seq), S, cx.stream))
    k = Kernel("op_sequence_48_layers", per_seq, cx.lib.hgk_op_list_run, args, S,
               keep=(sets, W, offs, seqs))
    return Workload("qwen3_next_decode_opseq", _decode_cfg(S, 48, 1, len(sets)), [k], len(sets), S)


def k_qmm_swiglu(cx, name, sets, tab_g, tab_u, E, N, K, T, top_k, group=64):
    """The gate and up gather_qmm and the SwiGLU in one launch; bytes = both
    projections' distinct experts' weights + x + the activation + ids."""
    P = T * top_k
    per_expert = N * K // 2 + 2 * N * (K // group) * 2
    uniq = sum(len(set(st[1].tolist())) for st in sets) / len(sets)
    nbytes = int(2 * uniq * per_expert) + T * K * 2 + P * N * 2 + P * 4
    (wg, sg, bg), (wu, su, bu) = tab_g, tab_u
    args = [(BF16, _vp(x), T, K, top_k, None, _vp(wg), _vp(sg), _vp(bg), _vp(wu), _vp(su),
             _vp(bu), BF16, E, N, K, group, 4, _vp(exd), I32, P, _vp(y), N, cx.stream)
            for x, ex, exd, y in sets]
    return Kernel(name, nbytes, cx.lib.hgk_gather_qmm_swiglu, args, T,
                  keep=(sets, tab_g, tab_u))


def k_gdn_gated(cx, name, sets, wq, wk, alog, dtb, wn, B, Hk, Dk, Hv, Dv, zrow, zgroup, zgs):
    """One decode token of the recurrence and its gated output norm in one
    launch; bytes = state read and written + q, k, v, a, b, z + the output."""
    nbytes = (2 * B * Hv * Dv * Dk * 2 + B * (2 * Hk * Dk + Hv * Dv + 2 * Hv) * 2 +
              2 * B * Hv * Dv * 2 + 2 * Dk * 2 + Dv * 2 + 2 * Hv * 4)
    args = [(BF16, _vp(q), _vp(k), _vp(v), _vp(alog), _vp(a), _vp(dtb), _vp(b), F32, _vp(st),
             _vp(wq), _vp(wk), _f(1e-6), B, Hk, Dk, Hv, Dv, _vp(st), None, _vp(z), zrow, zgroup,
             zgs, _vp(wn), BF16, _f(1e-6), _vp(o), cx.stream) for q, k, v, a, b, st, z, o in sets]
    return Kernel(name, nbytes, cx.lib.hgk_gated_delta_gated_norm, args, B,
                  keep=(sets, wq, wk, alog, dtb, wn))


def wl_qwen3_next_decode_layers(cx, fused=False):
    """One decode step of 64 sequences through the 48 Qwen3-Next-80B-A3B
    layers' per-layer kernels around the dense projections: per layer the
    input_layernorm as residual add + RMSNorm [64, 2048] (the residual stream
    chained from layer to layer, qwen3_next.rs:1539-1540); for the 36
    linear-attention layers the
    gated-delta recurrence (Hk 16, Dk 128, Hv 32, Dv 128, fused q/k norm, the
    state updated in place) and its gated output norm (z read in place from
    in_proj_qkvz), for the 12 full-attention layers the q/k-norm + partial
    RoPE; the post_attention_layernorm (add + RMSNorm); the routed experts' gate and up
    gather_qmm (top-10 of 512, 512 x 2048, 4-bit) and SwiGLU. Unfused: the
    reference's separate calls (7 launches per linear-attention layer).
    Fused: recurrence + gated norm in one launch and gate + up + SwiGLU in
    one launch (4 per layer). Replayed as one captured graph per step."""
    torch = cx.torch
    S, Hd, Hk, Dk, Hv, Dv, Hq, Hkv, D, E, top_k, I = 64, 2048, 16, 128, 32, 128, 16, 2, 256, 512, 10, 512
    P = S * top_k
    from higgs_amd.ops import gdn_qk_norm_weights
    gwq, gwk = gdn_qk_norm_weights(Dk, torch.bfloat16, cx.dev)
    alog = (torch.rand(Hv, device=cx.dev, generator=cx.gen) - 1.0).contiguous()
    dtb = (torch.rand(Hv, device=cx.dev, generator=cx.gen) - 0.5).contiguous()
    wn = cx.randn((Hd,), torch.bfloat16, 1.0, 0.02)
    wg = cx.randn((Dv,), torch.bfloat16, 1.0, 0.02)
    wq = cx.randn((D,), torch.bfloat16, 1.0, 0.02)
    wk = cx.randn((D,), torch.bfloat16, 1.0, 0.02)
    offs = torch.randint(1, 32769, (S,), dtype=torch.int32, device=cx.dev, generator=cx.gen)
    ntab = 4  # expert table sets, rotated over the layers (~0.6 GB each)
    tabs = [{nm: cx.qtable_experts(E, I, Hd) for nm in ("gate", "up")} for _ in range(ntab)]
    g = torch.Generator().manual_seed(7)
    ns = 1  # one set: every layer has its own buffers and the step walks ~6 GB
    r = lambda shape, lo, hi: (torch.rand(shape, device=cx.dev, generator=cx.gen) * (hi - lo) + lo
                               ).to(torch.bfloat16)
    kernels = []
    h = cx.randn((S, Hd), torch.bfloat16)  # the residual stream, chained through the layers
    for layer in range(48):
        h_a, h_b = cx.empty((S, Hd), torch.bfloat16), cx.empty((S, Hd), torch.bfloat16)
        n1 = [(h, cx.randn((S, Hd), torch.bfloat16), h_a, cx.empty((S, Hd), torch.bfloat16))]
        n2 = [(h_a, cx.randn((S, Hd), torch.bfloat16), h_b, cx.empty((S, Hd), torch.bfloat16))]
        h = h_b
        kernels.append(k_add_rmsnorm(cx, "add_rms_norm", n1, wn, S, Hd, 1e-6))
        if layer % 4 == 3:
            rp = [(cx.randn((S, 1, Hq, 512), torch.bfloat16), cx.randn((S, 1, Hkv, D), torch.bfloat16),
                   cx.empty((S, Hq, 1, D), torch.bfloat16), cx.empty((S, Hkv, 1, D), torch.bfloat16))]
            kernels.append(k_qkrope(cx, "qk_norm_partial_rope", rp, S, 1, Hq, Hkv, D, 64, 1e7,
                                    wq=wq, wk=wk, eps=1e-6, offsets=offs, q_block=512))
        else:
            q, k = r((S, 1, Hk, Dk), -1, 1), r((S, 1, Hk, Dk), -1, 1)
            v, a, b = r((S, 1, Hv, Dv), -1, 1), r((S, 1, Hv), -1, 1), r((S, 1, Hv), -1, 1)
            st = r((S, Hv, Dv, Dk), -0.1, 0.1)
            qkvz = cx.randn((S, Hk, 768), torch.bfloat16)
            z = qkvz[:, :, 512:]
            if fused:
                o = cx.empty((S, Hv, Dv), torch.bfloat16)
                kernels.append(k_gdn_gated(cx, "gdn_gated_norm", [(q, k, v, a, b, st, z, o)], gwq,
                                           gwk, alog, dtb, wg, S, Hk, Dk, Hv, Dv, Dv, 2, 768))
            else:
                y = cx.empty((S, 1, Hv, Dv), torch.bfloat16)
                kernels.append(k_gdn(cx, "gdn_decode", [(q, k, v, a, b, st, y, st)], gwq, gwk, alog,
                                     dtb, S, 1, Hk, Dk, Hv, Dv))
                o = cx.empty((S * Hv, Dv), torch.bfloat16)
                kernels.append(k_gated(cx, "gated_rms_norm", [(y, z, o)], wg, S * Hv, Dv, 1e-6,
                                       Dv, 2, 768))
        kernels.append(k_add_rmsnorm(cx, "add_rms_norm", n2, wn, S, Hd, 1e-6))
        ex = torch.stack([torch.randperm(E, generator=g)[:top_k] for _ in range(S)]).reshape(-1).to(
            torch.int32)
        exd = ex.to(cx.dev)
        x = cx.randn((S, Hd), torch.bfloat16)
        tb = tabs[layer % ntab]
        if fused:
            act = cx.empty((P, I), torch.bfloat16)
            kernels.append(k_qmm_swiglu(cx, "qmm_gate_up_swiglu", [(x, ex, exd, act)], tb["gate"],
                                        tb["up"], E, I, Hd, S, top_k))
        else:
            go, uo = cx.empty((P, I), torch.bfloat16), cx.empty((P, I), torch.bfloat16)
            kernels.append(k_qmm(cx, "qmm_gate", [(x, ex, exd, go)], tb["gate"], E, I, Hd, S, top_k,
                                 top_k))
            kernels.append(k_qmm(cx, "qmm_up", [(x, ex, exd, uo)], tb["up"], E, I, Hd, S, top_k,
                                 top_k))
            kernels.append(k_glu(cx, "swiglu_experts", [(go, uo, cx.empty((P, I), torch.bfloat16))],
                                 P, I, SILU))
    cfg = {"workload": "qwen3-next-80b-a3b decode step, 48 layers' per-layer kernels" +
                       (" (fused)" if fused else " (separate calls)"),
           "sequences": S, "layers": 48, "launches": len(kernels), "hidden": Hd,
           "gdn": "Hk 16 x 128, Hv 32 x 128", "experts": f"top-{top_k} of {E}, {I} x {Hd}, 4-bit"}
    return Workload("qwen3_next_decode_layers" + ("_fused" if fused else ""), cfg, kernels, ns, S,
                    graph=True)


WORKLOADS = {
    "llama32_1b_chain": wl_llama_chain,
    "rmsnorm_512x2048": wl_rmsnorm_512,
    "qwen3_8b_prefill": wl_qwen3_prefill,
    "gemma2_9b_prefill": wl_gemma2,
    "qwen3_next_decode": wl_qwen3_next_decode,
    "qwen3_next_decode_opseq": wl_qwen3_next_decode_opseq,
    "llama32_1b_chain_fused": wl_llama_chain_fused,
    "block_boundary_add_rms_norm": wl_block_boundary,
    "qwen3_next_moe_decode": wl_qwen3_next_moe_decode,
    "qwen3_next_gdn": wl_qwen3_next_gdn,
    "qwen3_next_qlinear": wl_qwen3_next_qlinear,
    "qwen3_next_moe_prefill": wl_qwen3_next_moe_prefill,
    "qwen3_next_moe_prefill_fused": lambda cx: wl_qwen3_next_moe_prefill(cx, fused=True),
    "qwen3_next_decode_layers": wl_qwen3_next_decode_layers,
    "qwen3_next_decode_layers_fused": lambda cx: wl_qwen3_next_decode_layers(cx, fused=True),
}


# ---------------------------------------------------------------- measurement
class HipEvents:
    """HIP events through the runtime's C API, recorded on the stream the
    kernels are launched on (the C ABI gets the same stream handle)."""

    def __init__(self):
        h = C.CDLL("libamdhip64.so")
        h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        h.hipEventDestroy.argtypes = [C.c_void_p]
        h.hipEventSynchronize.argtypes = [C.c_void_p]
        self.h = h

    def create(self, n):
        out = []
        for _ in range(n):
            e = C.c_void_p()
            if self.h.hipEventCreate(C.byref(e)):
                raise RuntimeError("hipEventCreate failed")
            out.append(e)
        return out

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        if self.h.hipEventElapsedTime(C.byref(ms), a, b):
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.h.hipEventDestroy(e)


def _capture(cx, launches):
    """One HIP graph holding `launches` (callables taking a stream), captured
    on a side stream at the default priority."""
    torch = cx.torch
    side = torch.cuda.Stream(cx.dev)
    sh = C.c_void_p(side.cuda_stream)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        for fn in launches:
            fn(sh)  # eager pass on the capture stream first
        side.synchronize()
        with torch.cuda.graph(g, stream=side):
            for fn in launches:
                fn(sh)
    return g


def _launcher(k, s):
    def fn(stream):
        a = k.argsets[s]
        if k.fn(*(a[:-1] + (stream,))):
            raise RuntimeError(f"{k.name}: status != 0")
    return fn


def kernel_times(cx, wl, graph, per_group=20, groups=5):
    """Average launch duration of each distinct kernel: `per_group` launches
    of it back to back over the rotating buffer sets, in `groups` groups
    bracketed by HIP events on the stream the kernels run on.

    Eager (graph=False): launched from the host; this agrees with rocprofv3's
    per-dispatch durations for kernels longer than the host launch cost
    (~6 us through ctypes). Graph (graph=True): each group is one captured
    HIP graph, which hides the host cost but adds a per-node dispatch cost of
    its own (~3 us per node measured on MI355X), so small kernels read high;
    rocprofv3's kernel trace gives their device durations."""
    torch = cx.torch
    he = HipEvents()
    rec = he.h.hipEventRecord
    st = cx.stream
    # every instance of a kernel (e.g. one per layer, each on its own buffers)
    # takes its turn, so a kernel's launches walk all of its buffers
    inst, order = {}, []
    for k in wl.kernels:
        if k.name not in inst:
            inst[k.name] = []
            order.append(k.name)
        inst[k.name].append(k)
    per = []
    for name in order:
        ks = inst[name]
        k = ks[0]
        plan = [(ks[i % len(ks)], (i // len(ks)) % wl.nsets) for i in range(per_group)]
        if graph:
            g = _capture(cx, [_launcher(kk, si) for kk, si in plan])
            go = g.replay
        else:
            calls = [(kk.fn, kk.argsets[si]) for kk, si in plan]

            def go(calls=calls, name=k.name):
                for fn, a in calls:
                    if fn(*a):
                        raise RuntimeError(f"{name}: {cx.lib.hgk_last_error().decode()}")
        go()  # warm
        torch.cuda.synchronize()
        evs = he.create(groups + 1)
        rec(evs[0], st)
        for i in range(groups):
            go()
            rec(evs[i + 1], st)
        torch.cuda.synchronize()
        d = sorted(he.elapsed_ms(evs[i], evs[i + 1]) / per_group for i in range(groups))
        he.destroy(evs)
        if graph:
            del g
        avg = sum(d) / len(d)
        per.append({"kernel": k.name, "bytes": k.bytes, "avg_us": avg * 1e3,
                    "median_us": d[len(d) // 2] * 1e3, "best_us": d[0] * 1e3,
                    "launches": groups * per_group, "method": "graph" if graph else "eager",
                    "gbs": k.bytes / (avg * 1e-3) / 1e9,
                    "frac_of_peak": k.bytes / (avg * 1e-3) / 1e9 / PEAK_HBM_GBS})
        if k.flops:
            per[-1]["tflops"] = k.flops / (avg * 1e-3) / 1e12
            per[-1]["frac_of_mfma_peak"] = per[-1]["tflops"] / PEAK_BF16_TFLOPS
        elif not graph:
            # the same bytes through a plain copy: a ratio near or above 1 means
            # the kernel is as fast as moving its bytes can be at this size
            cu = copy_floor(cx, k.bytes, per_group, groups)
            per[-1]["copy_us"] = cu
            per[-1]["copy_over_kernel"] = cu / (avg * 1e3)
            if k.wbytes is not None:
                # the measured floors: an empty kernel at this kernel's own
                # grid, and the streaming kernel at its read:write split
                blocks, threads = launch_grid(cx, k)
                per[-1]["grid"] = [blocks, threads]
                per[-1]["empty_us"] = empty_floor(cx, blocks, threads, per_group, groups)
                su = stream_floor(cx, k.bytes - k.wbytes, k.wbytes, per_group, groups)
                per[-1]["stream_us"] = su
                per[-1]["stream_over_kernel"] = su / (avg * 1e3)
    return per


def launch_grid(cx, k):
    """(workgroups, threads per workgroup) of one launch of kernel k, as the
    library noted it."""
    k.launch(0)
    blocks, threads = C.c_int64(), C.c_int()
    cx.check(cx.lib.hgk_last_launch_grid(C.byref(blocks), C.byref(threads)))
    cx.torch.cuda.synchronize()
    return blocks.value, threads.value


def _time_groups(cx, go, per_group, groups):
    """Average duration of one of `per_group` back-to-back launches made by
    go(), over `groups` groups bracketed by HIP events on the bench stream."""
    torch = cx.torch
    he = HipEvents()
    go()
    torch.cuda.synchronize()
    evs = he.create(groups + 1)
    he.h.hipEventRecord(evs[0], cx.stream)
    for i in range(groups):
        go()
        he.h.hipEventRecord(evs[i + 1], cx.stream)
    torch.cuda.synchronize()
    d = [he.elapsed_ms(evs[i], evs[i + 1]) / per_group for i in range(groups)]
    he.destroy(evs)
    return sum(d) / len(d) * 1e3


def empty_floor(cx, blocks, threads, per_group=20, groups=5):
    """Average duration of an empty kernel over the given grid: launch,
    dispatch and drain of that many workgroups with no work in them."""
    def go():
        for _ in range(per_group):
            cx.check(cx.lib.hgk_floor_empty(blocks, threads, cx.stream))
    return _time_groups(cx, go, per_group, groups)


def stream_floor(cx, read_bytes, write_bytes, per_group=20, groups=5, units=(2, 4, 8)):
    """Average duration of the library's streaming kernel (16-byte lanes,
    loads before stores, non-temporal stores, values computed from the loaded
    ones) reading read_bytes and writing write_bytes, source/destination pairs
    rotating over >= 1 GB: the fastest of 2, 4 and 8 units per thread."""
    torch = cx.torch
    rb = (int(read_bytes) + 15) // 16 * 16
    wb = (int(write_bytes) + 15) // 16 * 16
    npairs = max(2, math.ceil((1 << 30) / max(rb + wb, 1)))
    bufs = [(cx.empty((max(rb, 16),), torch.uint8), cx.empty((max(wb, 16),), torch.uint8))
            for _ in range(npairs)]

    best = None
    for u in units:
        def go(u=u):
            for i in range(per_group):
                src, dst = bufs[i % npairs]
                cx.check(cx.lib.hgk_floor_stream(_vp(src), rb, _vp(dst), wb, u, cx.stream))
        us = _time_groups(cx, go, per_group, groups)
        best = us if best is None else min(best, us)
    del bufs
    return best


def copy_floor(cx, nbytes, per_group=20, groups=5):
    """Average duration of a plain device-to-device copy (the runtime's blit
    kernel, hipMemcpyAsync) of nbytes / 2, i.e. nbytes of HBM traffic: what a
    kernel moving the same bytes costs with no arithmetic at all, launch and
    tail included. Source/destination pairs rotate over >= 1 GB like the
    kernels' buffer sets."""
    torch = cx.torch
    half = max(16, (int(nbytes) // 2 + 255) // 256 * 256)
    npairs = max(2, math.ceil((1 << 30) / (2 * half)))
    bufs = [(cx.empty((half,), torch.uint8), cx.empty((half,), torch.uint8))
            for _ in range(npairs)]
    he = HipEvents()
    h = he.h
    h.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    st = cx.stream

    def go():
        for i in range(per_group):
            src, dst = bufs[i % npairs]
            if h.hipMemcpyAsync(dst.data_ptr(), src.data_ptr(), half, 3, st):  # DeviceToDevice
                raise RuntimeError("hipMemcpyAsync failed")
    go()
    torch.cuda.synchronize()
    evs = he.create(groups + 1)
    h.hipEventRecord(evs[0], st)
    for i in range(groups):
        go()
        h.hipEventRecord(evs[i + 1], st)
    torch.cuda.synchronize()
    d = sorted(he.elapsed_ms(evs[i], evs[i + 1]) / per_group for i in range(groups))
    he.destroy(evs)
    del bufs
    return sum(d) / len(d) * 1e3


def settle(cx, fn, seconds):
    """Untimed whole steps until `seconds` of wall time have passed. The GPU's
    clocks ramp up over its first ~10-20 ms of work (a 36 us kernel reads
    38-39 us in its first ~10 ms on MI355X), which a warm-up counted in steps
    of a sub-millisecond workload would leave inside the timed region."""
    torch = cx.torch
    t0, i = time.perf_counter(), 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()


def measure(cx, wl, steps, warmup, settle_s=0.25):
    torch = cx.torch
    he = HipEvents()
    rec = he.h.hipEventRecord
    if wl.graph:
        # launch-bound sequence: captured graphs replayed back to back; each
        # graph holds `reps` whole steps so one replay's host cost is shared
        reps = max(1, 200 // len(wl.kernels))
        graphs = [_capture(cx, [_launcher(k, (si + r) % wl.nsets)
                                for r in range(reps) for k in wl.kernels])
                  for si in range(wl.nsets)]
        settle(cx, lambda i: graphs[i % wl.nsets].replay(), settle_s)
        for i in range(warmup):
            graphs[i % wl.nsets].replay()
        torch.cuda.synchronize()
        t0, t1 = he.create(2)
        w0 = time.perf_counter()
        rec(t0, cx.stream)
        for i in range(steps):
            graphs[i % wl.nsets].replay()
        rec(t1, cx.stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - w0
        ms = he.elapsed_ms(t0, t1) / (steps * reps)
        he.destroy([t0, t1])
        del graphs
        return {"ms_per_step": ms, "wall_ms_per_step": wall * 1e3 / (steps * reps),
                "steps_per_graph": reps, "kernels": kernel_times(cx, wl, graph=True)}
    settle(cx, wl.step, settle_s)
    for i in range(warmup):
        wl.step(i)
    torch.cuda.synchronize()
    st = cx.stream

    def run(plan):
        for fn, args, name in plan:
            if fn(*args):
                raise RuntimeError(f"{name}: {cx.lib.hgk_last_error().decode()}")

    # the K timed steps: events only at the two ends (an event between kernels
    # costs the stream ~4 us on this part, more than a small kernel's work)
    plan = [(k.fn, k.argsets[i % wl.nsets], k.name) for i in range(steps) for k in wl.kernels]
    t0, t1 = he.create(2)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    rec(t0, st)
    run(plan)
    rec(t1, st)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = he.elapsed_ms(t0, t1) / steps
    he.destroy([t0, t1])
    return {"ms_per_step": ms, "wall_ms_per_step": wall * 1e3 / steps,
            "kernels": kernel_times(cx, wl, graph=False)}


# ---------------------------------------------------------------- CPU baseline
def cpu_sample_llama(budget_s=10.0):
    """The oracle (C restatement, OpenMP) on 1/16 of the chain: 256 tokens
    through embedding, RMSNorm, llama3 RoPE (q 32 / k 8 heads) and SwiGLU."""
    import numpy as np

    import oracle as O

    T, V, Hd, I = 256, 128256, 2048, 8192
    wq = O.u32(5001, (V, Hd // 8))
    s = O.from_f32(O.uniform(5002, (V, Hd // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(5003, (V, Hd // 64), -0.1, 0.1), O.BF16)
    ids = O.ids(5004, T, V)
    w = O.from_f32(O.normal(5005, (Hd,), 1.0, 0.02), O.BF16)
    q = O.from_f32(O.normal(5006, (1, T, 32, 64)), O.BF16)
    k = O.from_f32(O.normal(5007, (1, T, 8, 64)), O.BF16)
    g = O.from_f32(O.normal(5008, (T, I)), O.BF16)
    u = O.from_f32(O.normal(5009, (T, I)), O.BF16)
    inv = O.rope_inv_freq(0.0, 64, O.llama3_freqs(500000.0, 64, 32.0, 1.0, 4.0, 8192.0))
    nbytes = (T * (Hd // 2 + 2 * 2 * (Hd // 64) + 4 + Hd * 2) + T * Hd * 4 + Hd * 2 +
              T * 40 * 64 * 4 + T * I * 6)
    reps, t0 = 0, time.perf_counter()
    while True:
        h = O.qembed(ids, wq, s, b, O.BF16)
        O.rms_norm(h, O.BF16, w, O.BF16, 1e-5)
        O.norm_rope(q, O.BF16, dims=64, inv_freq=inv)
        O.norm_rope(k, O.BF16, dims=64, inv_freq=inv)
        O.glu(O.ACT_SILU, g, u, O.BF16)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    cores = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    gbs = nbytes * reps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{T} of 4096 tokens through the whole chain, {reps} reps in {el:.1f} s "
                      f"(C restatement of the MLX CPU ops, OpenMP)",
            "tokens_per_s": round(T * reps / el, 1), "np_version": np.__version__}


def cpu_sample_gemma(budget_s=10.0):
    """The oracle (C restatement, OpenMP) on 64 of the 16384 tokens of the
    Gemma-2-9B-shaped chain: embedding gather x 59.75 over the full 256000 x
    3584 table, (1+w) RMSNorm to f32, RoPE on q (16 heads) and k (8 heads) at
    head_dim 256, GeGLU [64, 14336] to f32; same byte formulas as the GPU
    kernels."""
    import numpy as np

    import oracle as O

    T, V, Hd, I, D = 64, 256000, 3584, 14336, 256
    wq = O.u32(6001, (V, Hd // 8))
    s = O.from_f32(O.uniform(6002, (V, Hd // 64), 0.005, 0.02), O.BF16)
    b = O.from_f32(O.uniform(6003, (V, Hd // 64), -0.1, 0.1), O.BF16)
    ids = O.ids(6004, T, V)
    w = O.from_f32(O.normal(6005, (Hd,), 0.0, 0.02), O.BF16)
    q = O.from_f32(O.normal(6006, (1, T, 16, D)), O.BF16)
    k = O.from_f32(O.normal(6007, (1, T, 8, D)), O.BF16)
    g = O.from_f32(O.normal(6008, (T, I)), O.BF16)
    u = O.from_f32(O.normal(6009, (T, I)), O.BF16)
    inv = O.rope_inv_freq(10000.0, D)
    nbytes = (T * (Hd // 2 + 2 * 2 * (Hd // 64) + 4 + Hd * 2) + T * Hd * (2 + 4) + Hd * 2 +
              T * 24 * D * 4 + T * I * 8)
    reps, t0 = 0, time.perf_counter()
    while True:
        h = O.qembed(ids, wq, s, b, O.BF16, out_scale=math.sqrt(3584.0))
        O.rms_norm(h, O.BF16, w, O.BF16, 1e-6, plus_one=True, out_dt=O.F32)
        O.norm_rope(q, O.BF16, dims=D, inv_freq=inv)
        O.norm_rope(k, O.BF16, dims=D, inv_freq=inv)
        O.glu(O.ACT_GELU_TANH, g, u, O.BF16, out_dt=O.F32)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    cores = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    gbs = nbytes * reps / el / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{T} of 16384 tokens through the whole chain (full {V}x{Hd} table), "
                      f"{reps} reps in {el:.1f} s (C restatement of the MLX CPU ops, OpenMP)",
            "tokens_per_s": round(T * reps / el, 1), "np_version": np.__version__}


def cpu_sample_ops(budget_s=10.0, wl=None):
    """The oracle on a bounded sample of every kernel of the workload, each
    launch weighted as often as it occurs in a step: the step's bytes over
    the summed per-op CPU times at each op's sampled rate."""
    specs, count = {}, {}
    for k in wl.kernels:
        specs.setdefault(k.name, (k.cpu, k.bytes))
        count[k.name] = count.get(k.name, 0) + 1
    per = max(0.5, budget_s / len(specs))
    t_step, sample = 0.0, []
    cores = None
    for name, (spec, nbytes) in specs.items():
        r = cpu_op(spec, per)
        t_step += count[name] * nbytes / (r["gbs"] * 1e9)
        cores = r["cores"]
        sample.append(f"{name}: {r['sample']}")
    gbs = wl.bytes / t_step / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": "each op on a bounded sample, weighted by its launches per step (" +
                      "; ".join(sample) + "); C restatement of the MLX CPU ops, OpenMP",
            "tokens_per_s": round(wl.tokens / t_step, 1)}


def cpu_op(spec, budget_s=1.0):
    """The oracle timed on a bounded sample of one op of a workload, with the
    same algorithmic-byte formula as the GPU kernel. Returns GB/s, rows/s, the
    sample and the thread count."""
    import numpy as np

    import oracle as O

    kind, p = spec
    B16 = O.BF16
    if kind == "rms":
        R = min(p["rows"], 256)
        x = O.from_f32(O.normal(7001, (R, p["n"])), B16)
        w = O.from_f32(O.normal(7002, (p["n"],), 0.0 if p["plus_one"] else 1.0, 0.02), B16)
        od = O.F32 if p["ydt"] == F32 else B16
        fn = lambda: O.rms_norm(x, B16, w, B16, p["eps"], plus_one=bool(p["plus_one"]), out_dt=od)
        nbytes = R * p["n"] * (2 + (4 if od == O.F32 else 2)) + p["n"] * 2
        rows, what = R, f"{R} of {p['rows']} rows"
    elif kind == "glu":
        R = min(p["rows"], 64)
        g = O.from_f32(O.normal(7003, (R, p["n"])), B16)
        u = O.from_f32(O.normal(7004, (R, p["n"])), B16)
        od = O.F32 if p.get("ydt") == F32 else B16
        fn = lambda: O.glu(p["act"], g, u, B16, out_dt=od)
        nbytes = R * p["n"] * (4 + (4 if od == O.F32 else 2))
        rows, what = R, f"{R} of {p['rows']} rows"
    elif kind == "gated":
        R = min(p["rows"], 1024)
        y = O.from_f32(O.normal(7005, (R, p["n"])), B16)
        z = O.from_f32(O.normal(7006, (R, p["n"])), B16)
        w = O.from_f32(O.normal(7007, (p["n"],), 1.0, 0.02), B16)
        fn = lambda: O.gated_rms_norm(y, z, B16, w, B16, p["eps"])
        nbytes = 3 * R * p["n"] * 2 + p["n"] * 2
        rows, what = R, f"{R} of {p['rows']} rows"
    elif kind == "rope":
        D, dims = p["D"], p["dims"]
        if p["L"] == 1:
            Bs, Ls = min(p["B"], 64), 1
        else:
            Bs, Ls = 1, min(p["L"], 64)
        q = O.from_f32(O.normal(7008, (Bs, Ls, p["Hq"], D)), B16)
        k = O.from_f32(O.normal(7009, (Bs, Ls, p["Hk"], D)), B16)
        wn = O.from_f32(O.normal(7010, (D,), 1.0, 0.02), B16) if p["norm"] else None
        inv = (O.rope_inv_freq(0.0, dims, np.asarray(p["freqs"], np.float32))
               if p["freqs"] is not None else O.rope_inv_freq(p["base"], dims))
        offs = O.offsets(7011, Bs, 1, 32768) if p["offsets"] else None
        kw = dict(dims=dims, inv_freq=inv, offsets=offs, norm_w=wn,
                  w_dt=B16 if wn is not None else None, eps=p["eps"])
        fn = lambda: (O.norm_rope(q, B16, **kw), O.norm_rope(k, B16, **kw))
        nbytes = Bs * Ls * (p["Hq"] + p["Hk"]) * D * 4 + (2 * D * 2 if wn is not None else 0)
        rows, what = Bs * Ls, f"{Bs * Ls} of {p['B'] * p['L']} tokens"
    elif kind == "qembed":
        V, H, G = p["V"], p["H"], p["group"]
        T = min(p["n"], 256)
        wq = O.u32(7012, (V, H // 8))
        sc = O.from_f32(O.uniform(7013, (V, H // G), 0.005, 0.02), B16)
        bi = O.from_f32(O.uniform(7014, (V, H // G), -0.1, 0.1), B16)
        ids = O.ids(7015, T, V)
        scale = p["scale"]
        fn = lambda: O.qembed(ids, wq, sc, bi, B16, group=G, out_scale=scale)
        nbytes = T * (H // 2 + 4 * (H // G) + 4 + 2 * H)
        rows, what = T, f"{T} of {p['n']} ids (full {V}x{H} table)"
    elif kind == "add_rms":
        R = min(p["rows"], 256)
        x = O.from_f32(O.normal(7016, (R, p["n"])), B16)
        r = O.from_f32(O.normal(7017, (R, p["n"])), B16)
        w = O.from_f32(O.normal(7018, (p["n"],), 1.0, 0.02), B16)
        fn = lambda: O.add_rms_norm(x, r, B16, w, B16, p["eps"])
        nbytes = 4 * R * p["n"] * 2 + p["n"] * 2
        rows, what = R, f"{R} of {p['rows']} rows"
    elif kind == "qembed_rms":
        V, H, G = p["V"], p["H"], p["group"]
        T = min(p["n"], 256)
        wq = O.u32(7019, (V, H // 8))
        sc = O.from_f32(O.uniform(7020, (V, H // G), 0.005, 0.02), B16)
        bi = O.from_f32(O.uniform(7021, (V, H // G), -0.1, 0.1), B16)
        w = O.from_f32(O.normal(7022, (H,), 1.0, 0.02), B16)
        ids = O.ids(7023, T, V)
        fn = lambda: O.qembed_rms_norm(ids, wq, sc, bi, B16, w, B16, p["eps"], group=G,
                                       out_scale=p["scale"])
        nbytes = T * (H // 2 + 4 * (H // G) + 4 + 4 * H) + 2 * H
        rows, what = T, f"{T} of {p['n']} ids (full {V}x{H} table)"
    elif kind == "qmm":
        E, N, K, G = p["E"], p["N"], p["K"], p["group"]
        Pn = 16
        Es = min(E, 16)
        x = O.from_f32(O.normal(7024, (Pn, K)), B16)
        wq = O.u32(7025, (Es, N, K // 8))
        sc = O.from_f32(O.uniform(7026, (Es, N, K // G), 0.005, 0.02), B16)
        bi = O.from_f32(O.uniform(7027, (Es, N, K // G), -0.1, 0.1), B16)
        ex = np.arange(Pn, dtype=np.int32) % Es
        fn = lambda: O.gather_qmm(x, B16, wq, sc, bi, B16, ex, group=G)
        nbytes = Pn * (N * K // 2 + 4 * N * (K // G) + 2 * K + 2 * N)
        rows, what = Pn, f"{Pn} (token, expert) pairs, distinct experts"
    elif kind == "qlinear":
        Ms = min(p["M"], 4)
        N, K, group = p["N"], p["K"], p["group"]
        x = O.from_f32(O.normal(7040, (Ms, K)), B16)
        w = O.u32(7041, (N, K // 8))
        sc = O.from_f32(O.uniform(7042, (N, K // group), 0.005, 0.02), B16)
        bi = O.from_f32(O.uniform(7043, (N, K // group), -0.1, 0.1), B16)
        fn = lambda: O.quantized_matmul(x, B16, w, sc, bi, B16, group=group)
        nbytes = N * K // 2 + 2 * N * (K // group) * 2 + Ms * K * 2 + Ms * N * 2
        rows, what = Ms, f"{Ms} rows x {N} x {K} (f64 contraction)"
    elif kind == "gdn":
        Bs = min(p["B"], 4)
        Ts = min(p["T"], 16)
        Hk, Dk, Hv, Dv = p["Hk"], p["Dk"], p["Hv"], p["Dv"]
        u = lambda key, shape, lo, hi: O.from_f32(O.uniform(key, shape, lo, hi), B16)
        q, k = u(7028, (Bs, Ts, Hk, Dk), -1, 1), u(7029, (Bs, Ts, Hk, Dk), -1, 1)
        v = u(7030, (Bs, Ts, Hv, Dv), -1, 1)
        a_, b_ = u(7031, (Bs, Ts, Hv), -1, 1), u(7032, (Bs, Ts, Hv), -1, 1)
        st = u(7033, (Bs, Hv, Dv, Dk), -0.1, 0.1)
        al, db = O.uniform(7034, (Hv,), -1, 0), O.uniform(7035, (Hv,), -0.5, 0.5)
        wq, wk = O.gdn_qk_norm_weights(Dk, B16)
        fn = lambda: O.gated_delta(q, k, v, al, a_, db, b_, B16, state=st, qw=wq, kw=wk)
        nbytes = (2 * Bs * Hv * Dv * Dk * 2 + Bs * Ts * (2 * Hk * Dk + 2 * Hv * Dv + 2 * Hv) * 2)
        rows, what = Bs * Ts, f"{Bs} sequences x {Ts} tokens (f64 recurrence)"
    else:
        raise ValueError(kind)
    fn()
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s and reps >= 2:
            break
    cores = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    return {"gbs": nbytes * reps / el / 1e9, "rows_per_s": rows * reps / el, "cores": cores,
            "sample": what, "reps": reps}


# ---------------------------------------------------------------- main
def traffic_for(kernel_name, workload):
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    try:
        data = json.load(open(path))
        return data[workload][kernel_name]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def run_one(cx, name, steps, warmup, settle_s=0.25):
    wl = WORKLOADS[name](cx)
    r = measure(cx, wl, steps, warmup, settle_s)
    r["workload"] = wl
    return r


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle", type=float, default=0.25,
                    help="seconds of untimed steps before the warm-up, so the clocks are steady")
    ap.add_argument("--config", default="gemma2_9b_prefill", choices=sorted(WORKLOADS))
    ap.add_argument("--table", action="store_true", help="also measure every workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--cpu-op-budget", type=float, default=1.0,
                    help="seconds of oracle time per op for the --table CPU column")
    ap.add_argument("--calib", action="store_true",
                    help="run a plain 256 MiB copy first (counter calibration)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only; the per-layer ops shard by token "
              "or head with no communication, so --gpus > 1 is not run", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    cx = Ctx()
    if args.calib:
        src = torch.empty(64 << 20, dtype=torch.float32, device=cx.dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    torch.cuda.synchronize()
    res = run_one(cx, args.config, args.steps, args.warmup, args.settle)
    wl = res["workload"]
    ms = res["ms_per_step"]
    gbs = wl.bytes / (ms * 1e-3) / 1e9
    line = {"metric": "achieved HBM GB/s (% of 8 TB/s) per fused kernel; layer-op tokens/s",
            "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (device RNG; random-init tables and weights)",
            "config": dict(wl.config, parallelism="none (1 GPU)"),
            "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
            "tokens_per_s": round(wl.tokens / (ms * 1e-3), 1),
            "bytes_per_step": wl.bytes,
            "wall_ms_per_step": round(res["wall_ms_per_step"], 5)}
    if res["kernels"]:
        line["kernels"] = [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in d.items()}
                           for d in res["kernels"]]
        dom = max(res["kernels"], key=lambda d: d["bytes"])
        line["roofline"] = {"kernel": dom["kernel"], "bound": "hbm",
                            "achieved": round(dom["gbs"], 2), "peak": PEAK_HBM_GBS,
                            "unit": "GB/s", "frac": round(dom["gbs"] / PEAK_HBM_GBS, 4),
                            "traffic": traffic_for(dom["kernel"], wl.name),
                            "bytes_per_launch": dom["bytes"],
                            "avg_launch_us": round(dom["avg_us"], 3)}
        if dom.get("frac_of_mfma_peak", 0.0) > dom["frac_of_peak"]:
            # a matrix-core-bound kernel (e.g. a prefill projection): priced
            # against the dense bf16 MFMA peak
            line["roofline"].update({"bound": "mfma", "achieved": round(dom["tflops"], 2),
                                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                     "frac": round(dom["frac_of_mfma_peak"], 4)})
    if args.table:
        rows = []
        for name in WORKLOADS:
            r = line if name == args.config else None
            if r is None:
                torch.cuda.empty_cache()
                rr = run_one(cx, name, max(10, args.steps // 2), args.warmup, args.settle)
                w2 = rr["workload"]
                r = {"workload": name, "ms_per_step": rr["ms_per_step"], "bytes": w2.bytes,
                     "gbs": w2.bytes / (rr["ms_per_step"] * 1e-3) / 1e9,
                     "tokens_per_s": w2.tokens / (rr["ms_per_step"] * 1e-3),
                     "kernels": rr["kernels"]}
                specs = {k.name: k.cpu for k in w2.kernels}
                del rr, w2
            else:
                r = {"workload": name, "ms_per_step": ms, "bytes": wl.bytes, "gbs": gbs,
                     "tokens_per_s": line["tokens_per_s"], "kernels": res["kernels"]}
                specs = {k.name: k.cpu for k in wl.kernels}
            if not args.no_cpu:
                # the oracle on a bounded sample of each op, for the CPU column
                for kd in r["kernels"] or []:
                    spec = specs.get(kd["kernel"])
                    kd["cpu"] = None if spec is None else cpu_op(spec, args.cpu_op_budget)
            rows.append(r)
            print(f"[table] {name}: {r['ms_per_step'] * 1e3:.1f} us/step "
                  f"{r['gbs']:.0f} GB/s ({r['gbs'] / PEAK_HBM_GBS:.1%}) "
                  f"{r['tokens_per_s']:.0f} tok/s", file=sys.stderr, flush=True)
            for k in r["kernels"] or []:
                cpu = k.get("cpu")
                cpu_txt = (f"   cpu {cpu['gbs']:.2f} GB/s ({cpu['cores']} threads)" if cpu else "")
                cp_txt = (f"   copy of the same bytes {k['copy_us']:.2f} us"
                          if "copy_us" in k else "")
                if "stream_us" in k:
                    cp_txt += (f"   stream {k['stream_us']:.2f} us   empty kernel "
                               f"{k['empty_us']:.2f} us at {k['grid'][0]}x{k['grid'][1]}")
                print(f"[table]    {k['kernel']:<24} {k['avg_us']:9.2f} us  {k['gbs']:7.0f} GB/s "
                      f"({k['frac_of_peak']:.1%}){cp_txt}{cpu_txt}", file=sys.stderr, flush=True)
        os.makedirs("gpurun_out", exist_ok=True)
        with open(os.path.join("gpurun_out", "bench_table.json"), "w") as f:
            json.dump(rows, f, indent=1)
    if not args.no_cpu and wl.cpu_sample is not None:
        if wl.cpu_sample is cpu_sample_ops:
            line["cpu_baseline"] = cpu_sample_ops(args.cpu_budget, wl)
        else:
            line["cpu_baseline"] = wl.cpu_sample(args.cpu_budget)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
