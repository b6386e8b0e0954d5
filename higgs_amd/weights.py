"""MLX checkpoint loading over the C ABI's safetensors reader.

Mirrors the reference loader (crates/higgs-models/src/lib.rs:574-723):

    collect_safetensors_files(model_dir)      lib.rs:682-705 (index.json shards,
                                              else model.safetensors, else
                                              MissingWeight)
    remap_quantized_key(key)                  lib.rs:709-723 (`.weight` ->
                                              `.inner.weight`, and `.scales`,
                                              `.biases`, `.bias`)
    load_quantized_safetensors_weights(names, model_dir, quantized)
                                              lib.rs:600-632: every checkpoint
                                              key that names a parameter (directly
                                              or, for quantized models, after the
                                              remap) is loaded
    SafetensorsFile(path)                     Array::load_safetensors, per tensor

Tensors land on the device through pinned staging buffers (hgk_st_upload);
the file itself is memory-mapped and never read whole into Python.
"""
from __future__ import annotations

import ctypes as C
from typing import Dict, Iterable, List, Optional

import numpy as np
import torch

from ._lib import ERR_UNSUPPORTED, HgkError, check, lib

# safetensors dtype string -> (numpy storage dtype, torch dtype); bf16/f16
# travel as raw 16-bit codes on the host
_NP = {"F32": np.float32, "F16": np.uint16, "BF16": np.uint16, "U32": np.uint32,
       "I32": np.int32, "F64": np.float64, "I64": np.int64, "U64": np.uint64,
       "I16": np.int16, "U16": np.uint16, "I8": np.int8, "U8": np.uint8, "BOOL": np.bool_,
       "F8_E4M3": np.uint8, "F8_E5M2": np.uint8}
_TORCH = {"F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16,
          "I32": torch.int32, "F64": torch.float64, "I64": torch.int64, "I16": torch.int16,
          "I8": torch.int8, "U8": torch.uint8, "BOOL": torch.bool}
if hasattr(torch, "uint32"):
    _TORCH["U32"] = torch.uint32


class TensorInfo:
    __slots__ = ("name", "dtype_name", "dtype", "shape", "nbytes", "index")

    def __init__(self, name, dtype_name, dtype, shape, nbytes, index):
        self.name, self.dtype_name, self.dtype = name, dtype_name, dtype
        self.shape, self.nbytes, self.index = shape, nbytes, index

    def __repr__(self):
        return f"TensorInfo({self.name!r}, {self.dtype_name}, {self.shape})"


class SafetensorsFile:
    """An open, validated safetensors file (memory-mapped by the library)."""

    def __init__(self, path: str):
        self.path = str(path)
        h = C.c_void_p()
        check(lib().hgk_st_open(self.path.encode(), C.byref(h)))
        self._h = h
        self._infos: Dict[str, TensorInfo] = {}
        self._order: List[str] = []
        n = lib().hgk_st_count(h)
        for i in range(n):
            name, dn = C.c_char_p(), C.c_char_p()
            dt, nd = C.c_int(), C.c_int()
            shape = (C.c_int64 * 8)()
            nb = C.c_int64()
            check(lib().hgk_st_tensor(h, i, C.byref(name), C.byref(dn), C.byref(dt), C.byref(nd),
                                      shape, C.byref(nb)))
            key = name.value.decode()
            self._infos[key] = TensorInfo(key, dn.value.decode(), dt.value,
                                          tuple(shape[k] for k in range(nd.value)), nb.value, i)
            self._order.append(key)

    def close(self):
        if self._h:
            lib().hgk_st_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def keys(self) -> List[str]:
        return list(self._order)

    def __contains__(self, name: str) -> bool:
        return name in self._infos

    def __len__(self) -> int:
        return len(self._order)

    def info(self, name: str) -> TensorInfo:
        try:
            return self._infos[name]
        except KeyError:
            raise HgkError(1, f"no tensor '{name}' in {self.path}") from None

    def numpy(self, name: str) -> np.ndarray:
        """Host copy; bf16/f16 come back as their uint16 codes."""
        t = self.info(name)
        out = np.empty(t.shape, _NP[t.dtype_name])
        check(lib().hgk_st_copy_to_host(self._h, t.index, out.ctypes.data_as(C.c_void_p),
                                        out.nbytes))
        return out

    def to_device(self, name: str, device, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Device copy on the device's current stream (complete on return); a
        CPU `device` gets a host tensor."""
        t = self.info(name)
        if torch.device(device).type == "cpu" and out is None:
            a = self.numpy(name)
            if t.dtype_name in ("BF16", "F16"):
                return torch.from_numpy(a.view(np.int16)).view(_TORCH[t.dtype_name])
            return torch.from_numpy(a)
        if out is None:
            if t.dtype_name not in _TORCH:
                raise HgkError(ERR_UNSUPPORTED, f"no torch dtype for {t.dtype_name} ('{name}')")
            out = torch.empty(t.shape, dtype=_TORCH[t.dtype_name], device=device)
        nbytes = out.numel() * out.element_size()
        if not out.is_contiguous() or nbytes < t.nbytes:
            raise HgkError(1, f"destination for '{name}' must be contiguous with {t.nbytes} bytes")
        stream = C.c_void_p(torch.cuda.current_stream(out.device).cuda_stream)
        check(lib().hgk_st_upload(self._h, t.index, C.c_void_p(out.data_ptr()), nbytes, stream))
        return out


def collect_safetensors_files(model_dir: str) -> List[str]:
    """The checkpoint's files, as the reference's collect_safetensors_files."""
    need = C.c_int64()
    check(lib().hgk_st_collect_files(str(model_dir).encode(), None, 0, C.byref(need)))
    buf = C.create_string_buffer(need.value)
    check(lib().hgk_st_collect_files(str(model_dir).encode(), buf, need.value, C.byref(need)))
    return [p for p in buf.value.decode().split("\n") if p]


def remap_quantized_key(key: str) -> Optional[str]:
    """`x.weight` -> `x.inner.weight` (and `.scales`, `.biases`, `.bias`); None
    for keys with no quantized form."""
    buf = C.create_string_buffer(len(key.encode()) + 16)
    st = lib().hgk_remap_quantized_key(key.encode(), buf, len(buf))
    if st == ERR_UNSUPPORTED:
        return None
    check(st)
    return buf.value.decode()


def load_quantized_safetensors_weights(names: Iterable[str], model_dir: str, quantized: bool,
                                       device) -> Dict[str, torch.Tensor]:
    """Load every checkpoint tensor whose key is one of `names`, directly or
    (for quantized models) after remap_quantized_key, onto `device`. Returns
    {parameter name: tensor}; keys that match nothing are skipped, as the
    reference does."""
    wanted = set(names)
    out: Dict[str, torch.Tensor] = {}
    for path in collect_safetensors_files(model_dir):
        with SafetensorsFile(path) as f:
            for key in f.keys():
                target = key if key in wanted else None
                if target is None and quantized:
                    rk = remap_quantized_key(key)
                    target = rk if rk in wanted else None
                if target is not None:
                    out[target] = f.to_device(key, device)
    return out


def quantized_embedding_from(weights: Dict[str, torch.Tensor], prefix: str,
                             group_size: int = 64, bits: int = 4):
    """A QuantizedEmbedding from loaded `{prefix}.weight|scales|biases` (or the
    `.inner.` names of the remapped form)."""
    from .ops import QuantizedEmbedding

    def pick(suffix):
        for k in (f"{prefix}.{suffix}", f"{prefix}.inner.{suffix}"):
            if k in weights:
                return weights[k]
        raise HgkError(1, f"missing {prefix}.{suffix}")

    w = pick("weight")
    if w.dtype != torch.int32:
        w = w.view(torch.int32)
    return QuantizedEmbedding(w, pick("scales"), pick("biases"), group_size=group_size, bits=bits)


__all__ = ["SafetensorsFile", "TensorInfo", "collect_safetensors_files", "remap_quantized_key",
           "load_quantized_safetensors_weights", "quantized_embedding_from"]
