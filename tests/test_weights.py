"""The checkpoint reader without a GPU: safetensors files written by the
`safetensors` package (an independent implementation of the format) read
back bit for bit through the C ABI; malformed files rejected; the
reference's key remapping and shard collection (crates/higgs-models/src/
lib.rs:682-723 and its tests at lib.rs:771-904)."""
from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest
import safetensors.numpy as stn
import safetensors.torch as stt
import torch

from higgs_amd import HgkError
from higgs_amd.weights import (SafetensorsFile, collect_safetensors_files,
                               load_quantized_safetensors_weights, remap_quantized_key)


# ------------------------------------------------------------------ remap (lib.rs:771-818)
@pytest.mark.parametrize("key,want", [
    ("model.layers.0.self_attn.q_proj.weight", "model.layers.0.self_attn.q_proj.inner.weight"),
    ("model.layers.0.self_attn.q_proj.bias", "model.layers.0.self_attn.q_proj.inner.bias"),
    ("model.layers.0.self_attn.q_proj.biases", "model.layers.0.self_attn.q_proj.inner.biases"),
    ("model.layers.0.self_attn.q_proj.scales", "model.layers.0.self_attn.q_proj.inner.scales"),
    ("model.embed_tokens.weight", "model.embed_tokens.inner.weight"),
    ("model.norm.weight", "model.norm.inner.weight"),
    ("lm_head.something", None),
    ("weight", None),
])
def test_remap_quantized_key(key, want):
    assert remap_quantized_key(key) == want


# ------------------------------------------------------------------ collect (lib.rs:863-904)
def test_collect_missing_both_files(tmp_path):
    with pytest.raises(HgkError) as e:
        collect_safetensors_files(str(tmp_path))
    assert "MissingWeight" in str(e.value)


def test_collect_single_file(tmp_path):
    (tmp_path / "model.safetensors").write_bytes(b"dummy")
    got = collect_safetensors_files(str(tmp_path))
    assert len(got) == 1 and got[0].endswith("model.safetensors")


def test_collect_index_json_unique_shards(tmp_path):
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({
        "metadata": {"total_size": 12345},
        "weight_map": {"model.embed_tokens.weight": "model-00001-of-00002.safetensors",
                       "model.layers.0.weight": "model-00001-of-00002.safetensors",
                       "model.layers.1.weight": "model-00002-of-00002.safetensors"}}))
    got = collect_safetensors_files(str(tmp_path))
    assert [os.path.basename(p) for p in got] == ["model-00001-of-00002.safetensors",
                                                  "model-00002-of-00002.safetensors"]


def test_collect_rejects_paths_outside_the_model_dir(tmp_path):
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"metadata": {}, "weight_map": {"a": "../evil.safetensors"}}))
    with pytest.raises(HgkError):
        collect_safetensors_files(str(tmp_path))
    (tmp_path / "model.safetensors.index.json").write_text('{"metadata": {}, "weight_map": {}}')
    assert collect_safetensors_files(str(tmp_path)) == []


# ------------------------------------------------------------------ reading files
def test_reads_every_dtype_bit_exact(tmp_path):
    rng = np.random.default_rng(5)
    tensors = {
        "w": torch.from_numpy(rng.integers(0, 2**32, (64, 16), dtype=np.uint64).astype(np.uint32)),
        "s": torch.randn(64, 2).to(torch.bfloat16),
        "h": torch.randn(3, 5).to(torch.float16),
        "f": torch.randn(7),
        "i": torch.arange(-5, 5, dtype=torch.int32),
        "l": torch.arange(6, dtype=torch.int64).reshape(2, 3),
        "u8": torch.arange(9, dtype=torch.uint8),
        "scalar": torch.tensor(2.5),
        "empty": torch.zeros(0, 4, dtype=torch.bfloat16),
    }
    path = tmp_path / "model.safetensors"
    stt.save_file(tensors, str(path), metadata={"format": "mlx"})
    with SafetensorsFile(str(path)) as f:
        assert sorted(f.keys()) == sorted(tensors)
        for k, t in tensors.items():
            info = f.info(k)
            assert info.shape == tuple(t.shape), k
            assert info.nbytes == t.numel() * t.element_size(), k
            got = f.numpy(k)
            ref = t.numpy() if t.dtype not in (torch.bfloat16, torch.float16) else \
                t.view(torch.int16).numpy().view(np.uint16)
            assert got.shape == ref.shape, k
            assert np.array_equal(got.reshape(-1).view(np.uint8), ref.reshape(-1).view(np.uint8)), k
        assert f.info("s").dtype_name == "BF16" and f.info("w").dtype_name == "U32"
        assert f.info("l").dtype == -1  # not a dtype the kernels take, still readable


def test_numpy_writer_and_header_padding(tmp_path):
    arrs = {"a": np.arange(12, dtype=np.float32).reshape(3, 4), "b": np.array([7], np.int32)}
    path = tmp_path / "x.safetensors"
    stn.save_file(arrs, str(path))
    with SafetensorsFile(str(path)) as f:
        for k, a in arrs.items():
            assert np.array_equal(f.numpy(k), a)


def _raw_file(path, header: dict, payload: bytes, pad: int = 0):
    h = json.dumps(header).encode() + b" " * pad
    path.write_bytes(struct.pack("<Q", len(h)) + h + payload)


@pytest.mark.parametrize("case", ["short", "hdr_len", "json", "dtype", "size", "offsets", "gap",
                                  "overlap", "trailing", "dup_shape"])
def test_malformed_files_are_rejected(tmp_path, case):
    p = tmp_path / "bad.safetensors"
    good = {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
            "b": {"dtype": "U8", "shape": [4], "data_offsets": [8, 12]}}
    payload = bytes(12)
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "hdr_len":
        p.write_bytes(struct.pack("<Q", 10**6) + b"{}")
    elif case == "json":
        h = b'{"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]'
        p.write_bytes(struct.pack("<Q", len(h)) + h + payload)
    elif case == "dtype":
        _raw_file(p, {**good, "a": {"dtype": "F33", "shape": [2], "data_offsets": [0, 8]}}, payload)
    elif case == "size":
        _raw_file(p, {**good, "a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}, payload)
    elif case == "offsets":
        _raw_file(p, {**good, "b": {"dtype": "U8", "shape": [4], "data_offsets": [8, 40]}}, payload)
    elif case == "gap":
        _raw_file(p, {"a": good["a"], "b": {"dtype": "U8", "shape": [3], "data_offsets": [9, 12]}},
                  payload)
    elif case == "overlap":
        _raw_file(p, {"a": good["a"], "b": {"dtype": "U8", "shape": [8], "data_offsets": [4, 12]}},
                  payload)
    elif case == "trailing":
        _raw_file(p, good, payload + b"xx")
    elif case == "dup_shape":
        _raw_file(p, {**good, "a": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}, payload)
    with pytest.raises(HgkError) as e:
        SafetensorsFile(str(p))
    assert e.value.status == 1


def test_missing_tensor_and_small_destination(tmp_path):
    path = tmp_path / "model.safetensors"
    stn.save_file({"a": np.zeros(4, np.float32)}, str(path))
    f = SafetensorsFile(str(path))
    with pytest.raises(HgkError):
        f.info("nope")
    import ctypes as C
    from higgs_amd._lib import lib
    small = np.zeros(2, np.float32)
    assert lib().hgk_st_copy_to_host(f._h, 0, small.ctypes.data_as(C.c_void_p), small.nbytes) == 1
    idx = C.c_int64()
    assert lib().hgk_st_find(f._h, b"a", C.byref(idx)) == 0 and idx.value == 0
    assert lib().hgk_st_find(f._h, b"b", C.byref(idx)) == 1
    f.close()


def write_mlx_checkpoint(root, V=512, H=256, group=64, sharded=True, key=0, sdtype=torch.bfloat16):
    """A small checkpoint in the MLX 4-bit layout: a quantized embedding
    (u32 codes, scales, biases) and bf16 norm weights, split over two shards
    with an index, as mlx-lm writes Llama-style models."""
    g = torch.Generator().manual_seed(key)
    codes = torch.randint(0, 2**32, (V, H // 8), generator=g, dtype=torch.int64).to(torch.uint32)
    scales = (torch.rand(V, H // group, generator=g) * 0.015 + 0.005).to(sdtype)
    biases = (torch.rand(V, H // group, generator=g) * 0.2 - 0.1).to(sdtype)
    ln = (1.0 + 0.02 * torch.randn(H, generator=g)).to(torch.bfloat16)
    norm = (1.0 + 0.02 * torch.randn(H, generator=g)).to(torch.bfloat16)
    shard1 = {"model.embed_tokens.weight": codes, "model.embed_tokens.scales": scales,
              "model.embed_tokens.biases": biases}
    shard2 = {"model.layers.0.input_layernorm.weight": ln, "model.norm.weight": norm}
    if sharded:
        stt.save_file(shard1, str(root / "model-00001-of-00002.safetensors"), metadata={"format": "mlx"})
        stt.save_file(shard2, str(root / "model-00002-of-00002.safetensors"), metadata={"format": "mlx"})
        wm = {k: "model-00001-of-00002.safetensors" for k in shard1}
        wm.update({k: "model-00002-of-00002.safetensors" for k in shard2})
        (root / "model.safetensors.index.json").write_text(json.dumps(
            {"metadata": {"total_size": 0}, "weight_map": wm}))
    else:
        stt.save_file({**shard1, **shard2}, str(root / "model.safetensors"))
    return {**shard1, **shard2}


def test_load_quantized_weights_remaps_inner_names(tmp_path):
    """The reference's parameter tree names the quantized embedding
    `embed_tokens.inner.weight` (and .scales/.biases under `.inner` too,
    lib.rs:709-723); with quantized=True those load from the flat keys, and
    keys that match nothing are skipped."""
    ckpt = write_mlx_checkpoint(tmp_path)
    names = ["model.embed_tokens.inner.weight", "model.embed_tokens.inner.scales",
             "model.embed_tokens.inner.biases", "model.layers.0.input_layernorm.weight",
             "model.norm.weight", "model.not_in_checkpoint.weight"]
    got = load_quantized_safetensors_weights(names, str(tmp_path), True, device="cpu")
    assert sorted(got) == sorted(names[:-1])
    src = {"model.embed_tokens.inner.weight": "model.embed_tokens.weight",
           "model.embed_tokens.inner.scales": "model.embed_tokens.scales",
           "model.embed_tokens.inner.biases": "model.embed_tokens.biases"}
    for name, t in got.items():
        want = ckpt[src.get(name, name)]
        assert t.dtype == want.dtype and torch.equal(t.view(-1).view(torch.uint8),
                                                      want.view(-1).view(torch.uint8)), name
    # without quantized=True the `.inner.` names stay unmatched
    plain = load_quantized_safetensors_weights(names, str(tmp_path), False, device="cpu")
    assert sorted(plain) == ["model.layers.0.input_layernorm.weight", "model.norm.weight"]
