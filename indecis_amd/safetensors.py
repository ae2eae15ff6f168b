"""The safetensors format as indecis reads and writes it
(safetensors/safetensors.go): an 8-byte little-endian header length, a
JSON header {name: {dtype, shape, data_offsets}, "__metadata__": {...}},
then the raw little-endian data.

tensor() reads through the library (ixh_safetensors_tensor: the same
checks as Parse, the same float32 decoding as File.Tensor); write() mirrors
Write (names sorted, header padded with spaces to 8 bytes, F32 / BF16 /
I8 write formats)."""
import ctypes as C
import json
import struct

import numpy as np

from . import _lib


def tensor(path, name):
    """File.Tensor (safetensors.go:160-173): the tensor decoded to float32
    (flat). Raises IxhError for a malformed file or a missing name."""
    L = _lib.lib()
    n = C.c_int64(0)
    p, nm = str(path).encode(), name.encode()
    _lib.check(L.ixh_safetensors_tensor(p, nm, None, 0, C.byref(n)))
    out = np.zeros(n.value, np.float32)
    _lib.check(L.ixh_safetensors_tensor(p, nm, out.ctypes.data_as(C.c_void_p), n.value, C.byref(n)))
    return out


def to_bf16(v):
    """ToBF16 (safetensors.go:334-342): nearest bfloat16, ties to even; NaN
    stays NaN."""
    b = np.ascontiguousarray(v, np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(v, np.float32))
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), r).astype(np.uint16)


def write(path, tensors, meta=None):
    """Write (safetensors.go:266-331). tensors: name -> (array, dtype) with
    dtype "F32", "BF16" (rounded to nearest even) or "I8" (values already
    integers, clamped to [-128, 127]); or name -> array (F32)."""
    names = sorted(tensors)
    header = {}
    if meta:
        header["__metadata__"] = dict(meta)
    blobs, off = [], 0
    for name in names:
        t = tensors[name]
        arr, dt = (t if isinstance(t, tuple) else (t, "F32"))
        arr = np.asarray(arr, np.float32)
        if dt == "F32":
            raw = np.ascontiguousarray(arr, "<f4").tobytes()
        elif dt == "BF16":
            raw = to_bf16(arr.reshape(-1)).astype("<u2").tobytes()
        elif dt == "I8":
            raw = np.clip(arr.reshape(-1), -128, 127).astype(np.int8).tobytes()
        else:
            raise ValueError(f"safetensors: {name}: unsupported write dtype {dt!r}")
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    hb = json.dumps(header, separators=(",", ":")).encode()
    hb += b" " * (-len(hb) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)))
        f.write(hb)
        for raw in blobs:
            f.write(raw)
