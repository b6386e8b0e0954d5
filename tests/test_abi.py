"""The C ABI without a GPU: the library loads, exports exactly what
include/higgs_hip.h declares, its host-side helpers agree with the oracle bit
for bit, and invalid arguments come back as error statuses with a message
(validation runs before any HIP call, so none of this touches a device)."""
from __future__ import annotations

import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import oracle as O
from higgs_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "higgs_hip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hgk_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    declared = header_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(L, name), f"{name} missing from {_lib.LIB_PATH}"
    assert sorted(_lib.PROTOTYPES) == declared, "ctypes prototypes drift from the header"
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                        text=True, check=True).stdout
    exported = sorted(set(re.findall(r"\b(hgk_\w+)$", nm, flags=re.M)))
    assert exported == declared, f"exported {exported} != declared {declared}"


def test_abi_version():
    assert _lib.lib().hgk_abi_version() == 1


@pytest.mark.parametrize("base,dims", [(500000.0, 64), (1e6, 128), (1e4, 256), (1e7, 64),
                                       (10000.0, 80)])
def test_inv_freq_helper_matches_oracle_bitexact(base, dims):
    got = (C.c_float * (dims // 2))()
    _lib.check(_lib.lib().hgk_rope_inv_freq(base, dims, None, got))
    assert np.array_equal(np.frombuffer(got, np.float32), O.rope_inv_freq(base, dims))


def test_llama3_helper_matches_oracle_bitexact():
    for args in ((500000.0, 64, 32.0, 1.0, 4.0, 8192.0), (500000.0, 128, 8.0, 1.0, 4.0, 8192.0)):
        got = (C.c_float * (args[1] // 2))()
        _lib.check(_lib.lib().hgk_llama3_rope_freqs(*args, got))
        ref = O.llama3_freqs(*args)
        assert np.array_equal(np.frombuffer(got, np.float32), ref)
        inv = (C.c_float * (args[1] // 2))()
        _lib.check(_lib.lib().hgk_rope_inv_freq(0.0, args[1], got, inv))
        assert np.array_equal(np.frombuffer(inv, np.float32), O.rope_inv_freq(0.0, args[1], ref))


def _status(fn, *args):
    st = fn(*args)
    return st, _lib.lib().hgk_last_error().decode()


def test_error_paths_return_status_and_message():
    L = _lib.lib()
    fake = C.c_void_p(0x1000)  # never dereferenced: every call below fails validation
    st, msg = _status(L.hgk_rms_norm, None, 1, 8, None, 1, 0, 1e-5, fake, 1, 8, 4, 8, None)
    assert st == _lib.ERR_ARG and "null" in msg
    st, msg = _status(L.hgk_rms_norm, fake, 7, 8, None, 1, 0, 1e-5, fake, 1, 8, 4, 8, None)
    assert st == _lib.ERR_ARG and "dtype" in msg
    st, msg = _status(L.hgk_rms_norm, fake, 1, 4, None, 1, 0, 1e-5, fake, 1, 8, 4, 8, None)
    assert st == _lib.ERR_ARG and "stride" in msg
    st, msg = _status(L.hgk_rms_norm, fake, 1, 8, None, 1, 1, 1e-5, fake, 1, 8, 4, 8, None)
    assert st == _lib.ERR_ARG and "plus_one" in msg
    st, msg = _status(L.hgk_rms_norm, fake, 1, 8, None, 1, 0, 1e-5, fake, 2, 8, 4, 8, None)
    assert st == _lib.ERR_UNSUPPORTED
    strides = _lib.i64_array([64, 64, 64])
    st, msg = _status(L.hgk_rope, 1, fake, strides, fake, strides, 1, 1, 1, 64, 64, 1,
                      1e4, 1.0, None, 0, None, None)
    assert st == _lib.ERR_UNSUPPORTED and "traditional" in msg
    st, msg = _status(L.hgk_rope, 1, fake, strides, fake, strides, 1, 1, 1, 64, 65, 0,
                      1e4, 1.0, None, 0, None, None)
    assert st == _lib.ERR_ARG and "dims" in msg
    st, msg = _status(L.hgk_rope, 1, fake, None, fake, strides, 1, 1, 1, 64, 64, 0,
                      1e4, 1.0, None, 0, None, None)
    assert st == _lib.ERR_ARG
    st, msg = _status(L.hgk_qk_norm_rope, 1, fake, strides, fake, strides, 1, fake,
                      None, None, None, None, 0, None, 0, 1e-6, 1, 1, 64, 64, 1e4, 1.0, None,
                      0, None, None)
    assert st == _lib.ERR_UNSUPPORTED and "weight dtype" in msg
    st, msg = _status(L.hgk_glu, 5, 1, fake, 8, fake, 8, fake, 1, 8, 1, 8, None)
    assert st == _lib.ERR_ARG and "activation" in msg
    st, msg = _status(L.hgk_glu, 0, 1, fake, 8, fake, 8, fake, 2, 8, 1, 8, None)
    assert st == _lib.ERR_UNSUPPORTED
    st, msg = _status(L.hgk_gated_rms_norm, 1, fake, 128, None, 128, 0, 0, fake, 1, 1e-6,
                      fake, 1, 128, 4, 128, None)
    assert st == _lib.ERR_ARG
    st, msg = _status(L.hgk_gated_rms_norm, 1, fake, 128, fake, 128, 2, 128, fake, 1, 1e-6,
                      fake, 1, 128, 4, 128, None)
    assert st == _lib.ERR_ARG and "overlap" in msg
    st, msg = _status(L.hgk_quantized_embedding, fake, 4, 4, fake, fake, fake, 1, 10, 2048,
                      64, 8, 0.0, fake, 2048, None)
    assert st == _lib.ERR_UNSUPPORTED and "bits" in msg
    st, msg = _status(L.hgk_quantized_embedding, fake, 4, 4, fake, fake, fake, 1, 10, 2048,
                      48, 4, 0.0, fake, 2048, None)
    assert st == _lib.ERR_UNSUPPORTED
    st, msg = _status(L.hgk_quantized_embedding, fake, 1, 4, fake, fake, fake, 1, 10, 2048,
                      64, 4, 0.0, fake, 2048, None)
    assert st == _lib.ERR_ARG and "ids" in msg
    # add + norm, gather_qmm, quantized_matmul, gated delta
    st, msg = _status(L.hgk_add_rms_norm, 1, fake, 8, None, 8, fake, 1, 0, 1e-5, fake, 8,
                      fake, 1, 8, 4, 8, None)
    assert st == _lib.ERR_ARG and "null" in msg
    st, msg = _status(L.hgk_gather_qmm, 1, fake, 4, 64, 1, None, fake, fake, fake, 1, 2, 64, 64,
                      64, 8, fake, 4, 4, fake, 64, None)
    assert st == _lib.ERR_UNSUPPORTED and "bits" in msg
    st, msg = _status(L.hgk_gather_qmm, 1, fake, 4, 64, 1, None, fake, fake, fake, 1, 2, 64, 64,
                      64, 4, fake, 0, 4, fake, 64, None)
    assert st == _lib.ERR_ARG and "indices" in msg
    st, msg = _status(L.hgk_gather_qmm, 1, fake, 2, 64, 1, None, fake, fake, fake, 1, 2, 64, 64,
                      64, 4, fake, 4, 4, fake, 64, None)
    assert st == _lib.ERR_ARG and "rows" in msg
    st, msg = _status(L.hgk_quantized_matmul, 1, fake, 4, 64, fake, fake, fake, 1, 64, 96, 64, 4,
                      fake, 64, None)
    assert st == _lib.ERR_ARG and "K" in msg
    st, msg = _status(L.hgk_quantized_matmul, 1, fake, 4, 64, fake, fake, fake, 2, 64, 64, 64, 4,
                      fake, 64, None)
    assert st == _lib.ERR_UNSUPPORTED and "scales" in msg
    st, msg = _status(L.hgk_quantized_matmul, 0, fake, 4, 64, fake, fake, fake, 0, 64, 64, 64, 4,
                      fake, 64, None)
    assert st == _lib.ERR_UNSUPPORTED and "bf16 or f16" in msg
    gd = lambda **kw: _status(L.hgk_gated_delta, 1, fake, fake, fake, fake, fake, fake, fake, 0,
                              None, kw.get("qw"), kw.get("kw"), 1e-6, 1, 1, kw.get("hk", 2),
                              kw.get("dk", 128), kw.get("hv", 4), 128, fake, fake, None)
    st, msg = gd(dk=96)
    assert st == _lib.ERR_UNSUPPORTED and "head_k_dim" in msg
    st, msg = gd(hk=3)
    assert st == _lib.ERR_ARG and "multiple" in msg
    st, msg = gd(qw=fake)
    assert st == _lib.ERR_ARG and "both" in msg
    # empty problems succeed without launching anything
    assert L.hgk_quantized_matmul(1, fake, 0, 64, fake, fake, fake, 1, 64, 64, 64, 4, fake, 64,
                                  None) == 0
    assert L.hgk_gated_delta(1, fake, fake, fake, fake, fake, fake, fake, 0, None, None, None,
                             1e-6, 0, 1, 2, 128, 4, 128, fake, fake, None) == 0
    assert L.hgk_rms_norm(fake, 1, 8, None, 1, 0, 1e-5, fake, 1, 8, 0, 8, None) == 0
    assert L.hgk_glu(0, 1, fake, 8, fake, 8, fake, 1, 8, 0, 8, None) == 0
    assert L.hgk_quantized_embedding(fake, 4, 0, fake, fake, fake, 1, 10, 2048, 64, 4, 0.0,
                                     fake, 2048, None) == 0
    # ... with NULL for the data an empty call would read or write
    assert L.hgk_rms_norm(None, 1, 8, None, 1, 0, 1e-5, None, 1, 8, 0, 8, None) == 0
    assert L.hgk_add_rms_norm(1, None, 8, None, 8, None, 1, 0, 1e-5, None, 8, None, 1, 8, 0, 8,
                              None) == 0
    assert L.hgk_glu(0, 1, None, 8, None, 8, None, 1, 8, 0, 8, None) == 0
    assert L.hgk_quantized_embedding(None, 4, 0, fake, fake, fake, 1, 10, 2048, 64, 4, 0.0,
                                     None, 2048, None) == 0
    assert L.hgk_gather_qmm(1, None, 0, 64, 1, None, fake, fake, fake, 1, 2, 64, 64, 64, 4, None,
                            4, 0, None, 64, None) == 0
    assert L.hgk_quantized_matmul(1, None, 0, 64, fake, fake, fake, 1, 64, 64, 64, 4, None, 64,
                                  None) == 0
    assert _lib.lib().hgk_last_error() == b""
    # the checks still hold for calls with data
    st, msg = _status(L.hgk_glu, 0, 1, None, 8, fake, 8, fake, 1, 8, 1, 8, None)
    assert st == _lib.ERR_ARG and "null" in msg
    st, msg = _status(L.hgk_gather_qmm, 1, None, 4, 64, 1, None, fake, fake, fake, 1, 2, 64, 64,
                      64, 4, fake, 4, 4, fake, 64, None)
    assert st == _lib.ERR_ARG and "null" in msg
    st, msg = _status(L.hgk_quantized_embedding, fake, 4, 0, None, fake, fake, 1, 10, 2048, 64,
                      4, 0.0, None, 2048, None)
    assert st == _lib.ERR_ARG and "null" in msg


def test_python_mirror_raises_on_missing_library(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(_lib.HgkError):
        _lib.lib()


def test_python_mirror_rejects_mixed_scale_and_bias_dtypes():
    """One scales dtype reaches the kernels for every scale and bias, so the
    host API refuses operands whose scales and biases disagree before any
    device work (the fused gate + up + SwiGLU compares all four)."""
    import torch

    import higgs_amd as H

    E, N, K, T, k = 4, 64, 512, 2, 2
    w = torch.zeros((E, N, K // 8), dtype=torch.int32)
    s16 = torch.zeros((E, N, K // 64), dtype=torch.bfloat16)
    h16 = torch.zeros((E, N, K // 64), dtype=torch.float16)
    x = torch.zeros((T, K), dtype=torch.bfloat16)
    idx = torch.zeros((T * k,), dtype=torch.int32)
    for sg, bg, su, bu in ((s16, s16, h16, h16), (s16, s16, s16, h16), (s16, h16, s16, s16)):
        with pytest.raises(_lib.HgkError, match="dtype"):
            H.gather_qmm_swiglu(x, w, sg, bg, w, su, bu, idx, x_row_div=k)
    with pytest.raises(_lib.HgkError, match="share a dtype"):
        H.gather_qmm(x, w, s16, h16, idx, x_row_div=k)
    with pytest.raises(_lib.HgkError, match="share a dtype"):
        H.quantized_matmul(x, w[0], s16[0], h16[0])


def test_op_list_layout_and_validation_without_a_device():
    """hgk_op as ctypes lays it out is the C struct (sizeof and field offsets
    from a C compile of the header); hgk_op_list_upload names the op index and
    the offending field values (which also shows the fields land where the
    library reads them); the run's argument checks come before any HIP call."""
    import shutil
    import tempfile

    from higgs_amd._lib import HgkOp
    L = _lib.lib()
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc:
        src = ("#include <stdio.h>\n#include <stddef.h>\n#include \"higgs_hip.h\"\n"
               "int main(void){printf(\"%zu\", sizeof(hgk_op));")
        fields = [f[0] for f in HgkOp._fields_]
        for f in fields:
            src += f"printf(\" %zu\", offsetof(hgk_op, {f}));"
        src += "return 0;}\n"
        with tempfile.TemporaryDirectory() as d:
            open(os.path.join(d, "l.c"), "w").write(src)
            subprocess.run([cc, "-I", os.path.join(ROOT, "include"), os.path.join(d, "l.c"), "-o",
                            os.path.join(d, "l")], check=True)
            got = [int(v) for v in subprocess.run([os.path.join(d, "l")], capture_output=True,
                                                  text=True, check=True).stdout.split()]
        assert got == [C.sizeof(HgkOp)] + [getattr(HgkOp, f).offset for f in fields]
    assert L.hgk_op_list_bytes(0) == -1 and L.hgk_op_list_bytes(4097) == -1
    assert L.hgk_op_list_bytes(192) > 192 * 200
    fake = C.c_void_p(1 << 20)
    ok = dict(x=1 << 20, x_tok=2048, y=1 << 21, y_tok=2048, r=1 << 22, r_tok=2048, h=1 << 23,
              h_tok=2048, w=1 << 24)

    def upload(*ops, dtype=1):
        arr = (HgkOp * len(ops))(*ops)
        st = L.hgk_op_list_upload(dtype, arr, len(ops), fake, 1 << 30, None)
        return st, L.hgk_last_error().decode()

    good = HgkOp(kind=1, rows=1, n=2048, eps=1e-6, **ok)
    st, msg = upload(good, HgkOp(kind=0, rows=3, n=12, **ok))
    assert st == 1 and "op 1" in msg and "rows=3" in msg and "n=12" in msg
    st, msg = upload(good, good, HgkOp(kind=3, rows=16, n=256, dims=40, k_heads=2, base=1e7, **ok))
    assert st == 2 and "op 2" in msg and "rotated dims 40" in msg
    st, msg = upload(HgkOp(kind=3, rows=16, n=192, dims=64, k_heads=2, base=1e7, **ok))
    assert st == 2 and "head_dim 192" in msg
    st, msg = upload(HgkOp(kind=4, rows=10, n=512, act=7, **ok))
    assert st == 1 and "activation 7" in msg
    st, msg = upload(HgkOp(kind=2, rows=32, n=128, eps=1e-6, **{**ok, "w": None}))
    assert st == 1 and "needs a weight" in msg
    st, msg = upload(HgkOp(kind=1, rows=1, n=2048, eps=1e-6, **{**ok, "x_tok": 2047}))
    assert st == 1 and "whole 16-byte units" in msg
    st, msg = upload(good, dtype=0)
    assert st == 2 and "bf16 or f16" in msg
    assert L.hgk_op_list_run(0, fake, 1, 64, None) == 2
    assert L.hgk_op_list_run(1, None, 1, 64, None) == 1
    assert L.hgk_op_list_run(1, fake, 0, 64, None) == 1
    assert L.hgk_op_list_run(1, fake, 4, -1, None) == 1
    assert L.hgk_op_list_run(1, fake, 4, 0, None) == 0  # nothing to run: no launch
