"""Minimal safetensors container reader/writer for tests (no pickle, no torch).

Format: 8-byte little-endian header length, a JSON header
({name: {dtype, shape, data_offsets}, "__metadata__": {...}}), then the
packed data section. Raw payloads are returned as numpy arrays of the storage
type: uint8 for F8_E4M3/F8_E5M2, uint16 for BF16/F16, float32 for F32.
"""
import json
import struct

import numpy as np

STORAGE = {
    "F8_E4M3": np.uint8,
    "F8_E5M2": np.uint8,
    "BF16": np.uint16,
    "F16": np.uint16,
    "F32": np.float32,
    "I32": np.int32,
    "U8": np.uint8,
}


def read(path):
    """Return (tensors, metadata); tensors maps name -> (dtype, shape, array)."""
    with open(path, "rb") as f:
        blob = f.read()
    (hlen,) = struct.unpack("<Q", blob[:8])
    header = json.loads(blob[8 : 8 + hlen].decode("utf-8"))
    meta = header.pop("__metadata__", {}) or {}
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        s, e = info["data_offsets"]
        raw = blob[base + s : base + e]
        arr = np.frombuffer(raw, dtype=STORAGE[info["dtype"]]).copy()
        out[name] = (info["dtype"], list(info["shape"]), arr)
    return out, meta


def write(path, tensors, metadata=None):
    """tensors: list of (name, dtype_str, shape, numpy array of storage type)."""
    header = {}
    if metadata is not None:
        header["__metadata__"] = dict(metadata)
    parts = []
    off = 0
    for name, dtype, shape, arr in tensors:
        raw = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        parts.append(raw)
        off += len(raw)
    hb = json.dumps(header, separators=(",", ":")).encode("utf-8")
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for p in parts:
            f.write(p)


def open_mmap(path):
    """{name: (dtype, shape, read-only memory-mapped array of the storage
    type)} of a safetensors file; reads only the header, so sampled rows of
    a multi-GB file cost only their own pages."""
    with open(path, "rb") as f:
        (hlen,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(hlen).decode("utf-8"))
    header.pop("__metadata__", None)
    base = 8 + hlen
    out = {}
    for name, info in header.items():
        s, e = info["data_offsets"]
        dt = STORAGE[info["dtype"]]
        n = (e - s) // np.dtype(dt).itemsize
        arr = np.memmap(path, dtype=dt, mode="r", offset=base + s, shape=(n,)) if n else np.zeros(0, dt)
        out[name] = (info["dtype"], list(info["shape"]), arr)
    return out
