"""Minimal safetensors reader/writer (F32 only), numpy-backed.

The weight file is the contract the reference's loader reads: an 8-byte
little-endian header length, a JSON header mapping tensor names to
``{"dtype", "shape", "data_offsets"}`` plus a ``__metadata__`` map of strings,
then the raw little-endian tensor bytes (src/weights.rs:101-185 reads it through
lightgpu::safetensors; tools/reference.py:49-65 reads it with numpy).

Nothing here executes anything stored in the file: the header is JSON and the
payload is raw floats.
"""
import json
import struct

import numpy as np

__all__ = ["write_safetensors", "read_safetensors"]


def write_safetensors(path, tensors, metadata):
    """Write ``{name: float32 ndarray}`` in the given order with ``metadata``."""
    header = {"__metadata__": {str(k): str(v) for k, v in metadata.items()}}
    offset = 0
    blobs = []
    for name, arr in tensors.items():
        a = np.ascontiguousarray(arr, dtype="<f4")
        header[name] = {
            "dtype": "F32",
            "shape": list(a.shape),
            "data_offsets": [offset, offset + a.nbytes],
        }
        offset += a.nbytes
        blobs.append(a)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * ((8 - len(hb) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for a in blobs:
            f.write(a.tobytes())


def read_safetensors(path, mmap=True):
    """``({name: float32 ndarray}, metadata)``; arrays are read-only views when mmapped."""
    with open(path, "rb") as f:
        n = struct.unpack("<Q", f.read(8))[0]
        header = json.loads(f.read(n))
    meta = header.pop("__metadata__", {})
    base = 8 + n
    if mmap:
        raw = np.memmap(path, dtype=np.uint8, mode="r")
    else:
        raw = np.fromfile(path, dtype=np.uint8)
    out = {}
    for name, info in header.items():
        if info["dtype"] != "F32":
            raise ValueError(f"{name}: dtype {info['dtype']} is not F32")
        a, b = info["data_offsets"]
        arr = raw[base + a: base + b].view("<f4").reshape(info["shape"])
        out[name] = arr
    return out, meta
