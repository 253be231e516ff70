"""Minimal safetensors writer for the loader tests: 8-byte little-endian
header length, JSON header, tensor bytes (the published format; BF16 has no
numpy dtype, so tensors are given as raw little-endian arrays)."""
import json
import struct

import numpy as np

_ITEM = {"BF16": 2, "F16": 2, "F32": 4, "I32": 4, "F64": 8, "U8": 1}


def bf16_bits(x) -> np.ndarray:
    """float32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def as_stored(dtype: str, values) -> np.ndarray:
    """The raw array a tensor of `dtype` holds for float `values`."""
    v = np.asarray(values, dtype=np.float32)
    if dtype == "BF16":
        return bf16_bits(v).reshape(v.shape)
    if dtype == "F16":
        return v.astype(np.float16).view(np.uint16).reshape(v.shape)
    if dtype == "F32":
        return v
    raise ValueError(dtype)


def widen(dtype: str, raw) -> np.ndarray:
    """f32 values of a stored array (what the reference's loader computes)."""
    raw = np.asarray(raw)
    if dtype == "BF16":
        return bf16_to_f32(raw).reshape(raw.shape)
    if dtype == "F16":
        return raw.view(np.float16).astype(np.float32)
    return raw.astype(np.float32)


def write(path, tensors, metadata=None, pad_header=0):
    """tensors: {name: (dtype, raw array)} in file order."""
    header, chunks, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, (dtype, raw) in tensors.items():
        raw = np.asarray(raw)  # keeps 0-d arrays 0-d
        b = raw.tobytes(order="C")
        assert len(b) == raw.size * _ITEM[dtype]
        header[name] = {"dtype": dtype, "shape": list(raw.shape), "data_offsets": [off, off + len(b)]}
        chunks.append(b)
        off += len(b)
    h = json.dumps(header).encode() + b" " * pad_header
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for c in chunks:
            f.write(c)
