"""Checkpoint-to-kernel parity on the GPU: a checkpoint in the MLX 4-bit layout
(written by the `safetensors` package), loaded through the library's reader
(hgk_st_upload, pinned staging) with the reference's remapping, drives the
embedding + first-norm kernel; the oracle gets the same tensors from the
`safetensors` package's own reader. Bars as for the kernels: h and y
bit-exact."""
from __future__ import annotations

import numpy as np
import pytest
import safetensors.torch as stt
import torch

import oracle as O
from gpu_util import to_host
from higgs_amd.weights import (SafetensorsFile, load_quantized_safetensors_weights,
                               quantized_embedding_from)
from test_weights import write_mlx_checkpoint

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("sharded", [True, False])
def test_llama_sized_checkpoint_drives_embedding_and_norm(dev, tmp_path, sharded):
    V, Hd, T = 128256, 2048, 1024
    write_mlx_checkpoint(tmp_path, V=V, H=Hd, sharded=sharded, key=7)
    names = ["model.embed_tokens.inner.weight", "model.embed_tokens.inner.scales",
             "model.embed_tokens.inner.biases", "model.layers.0.input_layernorm.weight"]
    w = load_quantized_safetensors_weights(names, str(tmp_path), True, dev)
    assert sorted(w) == sorted(names)
    emb = quantized_embedding_from(w, "model.embed_tokens")
    ln = w["model.layers.0.input_layernorm.weight"]
    ids = torch.randint(0, V, (T,), dtype=torch.int32, generator=torch.Generator().manual_seed(3))
    h, y = emb.forward_rms_norm(ids.to(dev), ln, 1e-5)

    # the oracle, fed by the safetensors package's own reader
    ref = {}
    for name in (["model-00001-of-00002.safetensors", "model-00002-of-00002.safetensors"]
                 if sharded else ["model.safetensors"]):
        ref.update(stt.load_file(str(tmp_path / name)))
    wq = ref["model.embed_tokens.weight"].numpy()
    sc = _bits(ref["model.embed_tokens.scales"])
    bi = _bits(ref["model.embed_tokens.biases"])
    lw = _bits(ref["model.layers.0.input_layernorm.weight"])
    h_ref, y_ref = O.qembed_rms_norm(ids.numpy(), wq, sc, bi, O.BF16, lw, O.BF16, 1e-5)
    assert np.array_equal(to_host(h), h_ref)
    assert np.array_equal(to_host(y), y_ref)


def test_upload_spans_several_staging_chunks(dev, tmp_path):
    """A 100 MB tensor (several 32 MiB staging chunks, both buffers reused)
    and a few small ones arrive intact."""
    g = torch.Generator().manual_seed(11)
    big = torch.randint(-2**31, 2**31 - 1, (25 * 2**20,), dtype=torch.int64, generator=g).to(torch.int32)
    small = torch.randn(3, 7, generator=g).to(torch.bfloat16)
    path = tmp_path / "model.safetensors"
    stt.save_file({"big": big, "small": small, "empty": torch.zeros(0, dtype=torch.float16)}, str(path))
    with SafetensorsFile(str(path)) as f:
        d_big = f.to_device("big", dev)
        d_small = f.to_device("small", dev)
        d_empty = f.to_device("empty", dev)
        # into a preallocated, larger destination
        out = torch.full((25 * 2**20 + 5,), -1, dtype=torch.int32, device=dev)
        f.to_device("big", dev, out=out)
    assert torch.equal(d_big.cpu(), big)
    assert torch.equal(d_small.cpu().view(torch.int16), small.view(torch.int16))
    assert d_empty.numel() == 0
    assert torch.equal(out[: big.numel()].cpu(), big) and (out[big.numel():] == -1).all()


def test_f16_scales_checkpoint(dev, tmp_path):
    """MLX checkpoints also ship f16 scales/biases (the mlx_rs format notes)."""
    V, Hd, T = 4096, 1024, 333
    write_mlx_checkpoint(tmp_path, V=V, H=Hd, sharded=False, key=9, sdtype=torch.float16)
    names = ["model.embed_tokens.weight", "model.embed_tokens.scales", "model.embed_tokens.biases"]
    w = load_quantized_safetensors_weights(names, str(tmp_path), False, dev)
    emb = quantized_embedding_from(w, "model.embed_tokens")
    ids = torch.randint(0, V, (T,), dtype=torch.int32, generator=torch.Generator().manual_seed(4))
    got = to_host(emb.forward(ids.to(dev)))
    ref = stt.load_file(str(tmp_path / "model.safetensors"))
    want = O.qembed(ids.numpy(), ref["model.embed_tokens.weight"].numpy(),
                    _bits(ref["model.embed_tokens.scales"]), _bits(ref["model.embed_tokens.biases"]),
                    O.F16)
    assert np.array_equal(got, want)
