"""Minimal GGUF v3 writer for test fixtures, following the layout the
reference documents (docs/WEIGHT_FORMAT.md §1-4 of Larynx): magic, version 3,
i64 tensor / KV counts, KV entries (u64-length strings, i32 type tags), tensor
infos (name, u32 n_dims, i64 ne[] = torch shape reversed, i32 ggml type, u64
offset into the data section), zero padding to the 32-byte alignment, then
each tensor's bytes padded to the alignment.
"""
import struct

import numpy as np

GGML_TYPE = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int8): 24,
             np.dtype(np.int16): 25, np.dtype(np.int32): 26, np.dtype(np.int64): 27,
             np.dtype(np.float64): 28}
ALIGN = 32


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _pad(n, a):
    return (-n) % a


def write_gguf(path, tensors, arch="cosyvoice3.flow", name="synthetic", extra_kv=(),
               align=ALIGN):
    """tensors: ordered (name, numpy array) pairs.  extra_kv: (key, gguf type, packed value);
    a general.alignment entry there must match `align`."""
    kv = [("general.architecture", 8, _str(arch)), ("general.name", 8, _str(name)),
          ("general.file_type", 4, struct.pack("<I", 0))] + list(extra_kv)
    head = b"GGUF" + struct.pack("<Iqq", 3, len(tensors), len(kv))
    for key, typ, val in kv:
        head += _str(key) + struct.pack("<i", typ) + val
    infos, blobs, off = b"", [], 0
    for tname, arr in tensors:
        arr = np.ascontiguousarray(arr)
        ne = list(arr.shape[::-1]) or [1]
        infos += _str(tname) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}q", *ne)
        infos += struct.pack("<iQ", GGML_TYPE[arr.dtype], off)
        data = arr.tobytes()
        blobs.append(data + b"\0" * _pad(len(data), align))
        off += len(blobs[-1])
    meta = head + infos
    with open(path, "wb") as f:
        f.write(meta + b"\0" * _pad(len(meta), align))
        for b in blobs:
            f.write(b)
