"""bench.py host logic on the CPU: launch records keep their buffers alive,
byte accounting matches the algorithmic formulas, and --gpus > 1 is refused."""
from __future__ import annotations

import gc
import subprocess
import sys
import weakref

import torch

import bench


class _StubLib:
    def __getattr__(self, name):
        return lambda *a: 0


class _StubCtx:
    torch = torch
    lib = _StubLib()
    stream = None
    dev = torch.device("cpu")


def _alive(refs):
    gc.collect()
    return [r() is not None for r in refs]


def test_launch_records_keep_every_buffer_alive():
    """Kernels hold raw device addresses; the tensors behind them must live as
    long as the Kernel (graph capture empties torch's cache, unmapping freed
    blocks under any launch that still points into them)."""
    cx = _StubCtx()
    refs = []

    def track(*ts):
        refs.extend(weakref.ref(t) for t in ts)
        return ts

    def build():
        ks = []
        ks.append(bench.k_glu(cx, "glu", [track(torch.zeros(4, 8), torch.zeros(4, 8),
                                                torch.zeros(4, 8))], 4, 8, bench.SILU))
        w = track(torch.zeros(8))[0]
        ks.append(bench.k_rmsnorm(cx, "norm", [track(torch.zeros(4, 8), torch.zeros(4, 8))],
                                  w, 4, 8, 1e-5))
        q, k, qo, ko = track(torch.zeros(1, 2, 4, 64), torch.zeros(1, 2, 2, 64),
                             torch.zeros(1, 4, 2, 64), torch.zeros(1, 2, 2, 64))
        wq, wk = track(torch.zeros(64), torch.zeros(64))
        offs = track(torch.zeros(1, dtype=torch.int32))[0]
        ks.append(bench.k_qkrope(cx, "rope", [(q, k, qo, ko)], 1, 2, 4, 2, 64, 64, 1e4,
                                 wq=wq, wk=wk, offsets=offs))
        wg = track(torch.zeros(8))[0]
        ks.append(bench.k_gated(cx, "gated", [track(torch.zeros(4, 8), torch.zeros(4, 8),
                                                    torch.zeros(4, 8))], wg, 4, 8, 1e-6, 8, 0, 0))
        tab = track(torch.zeros(16, 2, dtype=torch.int32), torch.zeros(16, 1), torch.zeros(16, 1))
        ks.append(bench.k_embed(cx, "emb", [track(torch.zeros(3, dtype=torch.int32),
                                                  torch.zeros(3, 16))], [tab], 16, 16, 3, group=16))
        return ks

    kernels = build()
    assert all(_alive(refs)), "a launch record lost one of its buffers"
    del kernels
    assert not any(_alive(refs)), "buffers should be released with their launch records"


def test_algorithmic_bytes_match_the_published_table():
    cx = _StubCtx()
    z = torch.zeros(1)
    assert bench.k_rmsnorm(cx, "n", [(z, z)], z, 4096, 2048, 1e-5).bytes == 33_558_528
    assert bench.k_glu(cx, "g", [(z, z, z)], 4096, 8192, bench.SILU).bytes == 201_326_592
    assert bench.k_embed(cx, "e", [(z, z)], [(z, z, z)], 128256, 2048, 4096).bytes == 21_512_192
    # the Gemma-2-9B chain's f32-output kernels: (1+w) norm and GeGLU
    assert bench.k_rmsnorm(cx, "n", [(z, z)], z, 16384, 3584, 1e-6, plus_one=1,
                           ydt=bench.F32).bytes == 16384 * 3584 * 6 + 3584 * 2
    assert bench.k_glu(cx, "g", [(z, z, z)], 16384, 14336, bench.GELU,
                       ydt=bench.F32).bytes == 1_879_048_192

    r = bench.k_qkrope(cx, "r", [(z, z, z, z)], 4, 1024, 32, 8, 64, 64, 5e5)
    assert r.bytes == 41_943_040
    r = bench.k_qkrope(cx, "r", [(z, z, z, z)], 8, 2048, 32, 8, 128, 128, 1e6, wq=z, wk=z)
    assert r.bytes == 335_544_832


def test_multi_gpu_request_is_refused():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True,
                       text=True, cwd=bench.__file__.rsplit("/", 1)[0])
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_every_kernel_rotation_exceeds_the_infinity_cache():
    """Per-kernel timing cycles each kernel over the buffer sets: the bytes it
    touches per cycle must be well past the 256 MB cache."""
    for kb in ([21_512_192, 33_558_528, 41_943_040, 201_326_592],
               [150_536_192, 352_328_704, 402_653_184, 1_879_048_192]):
        ns = bench.nsets_per_kernel(kb)
        assert min(kb) * ns >= 1 << 30
