"""safetensors access through the library's reader (rmda_st_*), plus a small
writer used by the tests and the benchmark to make weight files.

Host-only: no GPU and no torch needed.  The writer follows the published
safetensors layout (8-byte little-endian header length, JSON header of
name -> {dtype, shape, data_offsets}, raw bytes), the format the reference
reads in src/safet.c.
"""
import ctypes
import json
import os
import struct

import numpy as np

from . import _lib

DTYPE_NAMES = {_lib.ST_BF16: "BF16", _lib.ST_F16: "F16", _lib.ST_F32: "F32", _lib.ST_I64: "I64",
               _lib.ST_I32: "I32", _lib.ST_U8: "U8"}
_NP = {_lib.ST_BF16: np.uint16, _lib.ST_F16: np.float16, _lib.ST_F32: np.float32, _lib.ST_I64: np.int64,
       _lib.ST_I32: np.int32, _lib.ST_U8: np.uint8}


class StError(RuntimeError):
    pass


class SafeTensors:
    """A mapped .safetensors file or sharded directory (rmda_st_open)."""

    def __init__(self, path):
        self.L = _lib.lib()
        h = ctypes.c_void_p()
        rc = self.L.rmda_st_open(os.fsencode(path), ctypes.byref(h))
        if rc != _lib.OK:
            raise StError(self.L.rmda_st_message().decode())
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            self.L.rmda_st_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self):
        return [self.L.rmda_st_name(self.h, i).decode() for i in range(self.L.rmda_st_count(self.h))]

    def info(self, name):
        t = _lib.StTensor()
        rc = self.L.rmda_st_find(self.h, name.encode(), ctypes.byref(t))
        if rc != _lib.OK:
            raise KeyError(self.L.rmda_st_message().decode())
        return t

    def array(self, name):
        """numpy view (a copy) of a tensor's bytes; bf16 comes back as uint16 bits."""
        t = self.info(name)
        shape = tuple(t.shape[i] for i in range(t.ndim))
        buf = (ctypes.c_uint8 * t.bytes).from_address(t.data) if t.bytes else b""
        return np.frombuffer(bytes(buf), dtype=_NP[t.dtype]).reshape(shape)


def write(path, tensors, metadata=None):
    """Write {name: (dtype_name, numpy array)} as one .safetensors file; bf16
    arrays are given as uint16 bit patterns."""
    header = {}
    if metadata:
        header["__metadata__"] = dict(metadata)
    blobs = []
    off = 0
    for name, (dt, arr) in tensors.items():
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for b in blobs:
            f.write(b)


def write_sharded(directory, shards, metadata=None):
    """Write several shards plus model.safetensors.index.json (the Hugging
    Face layout: weight_map name -> shard file)."""
    os.makedirs(directory, exist_ok=True)
    n = len(shards)
    weight_map = {}
    for i, tensors in enumerate(shards):
        fname = "model-%05d-of-%05d.safetensors" % (i + 1, n)
        write(os.path.join(directory, fname), tensors)
        for name in tensors:
            weight_map[name] = fname
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": dict(metadata or {}), "weight_map": weight_map}, f)


def f32_to_bf16_bits(a):
    """fp32 -> bf16 bit patterns, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def moe_layer_tensors(prefix, shape, rng, std=0.02, dtype="BF16"):
    """One layer's MoE tensors under the reference's names (src/qwen.c:441-452)
    in the given expert dtype ("BF16" or "F16"); the router as BF16."""
    E, d, I, S = shape["experts"], shape["d"], shape["inter"], shape["shared"]

    def w(*dims):
        a = (rng.standard_normal(dims) * std).astype(np.float32)
        return ("BF16", f32_to_bf16_bits(a)) if dtype == "BF16" else ("F16", a.astype(np.float16))

    t = {prefix + "gate.weight": ("BF16", f32_to_bf16_bits(rng.standard_normal((E, d)).astype(np.float32) * std)),
         prefix + "experts.gate_up_proj": w(E, 2 * I, d),
         prefix + "experts.down_proj": w(E, d, I)}
    if S:
        t[prefix + "shared_expert_gate.weight"] = ("BF16", f32_to_bf16_bits(
            rng.standard_normal((1, d)).astype(np.float32) * std))
        t[prefix + "shared_expert.gate_proj.weight"] = w(S, d)
        t[prefix + "shared_expert.up_proj.weight"] = w(S, d)
        t[prefix + "shared_expert.down_proj.weight"] = w(d, S)
    return t
