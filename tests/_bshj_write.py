"""Test fixture writer of .bshj files, from the container layout documented in mashbox_amd/bshj.py (the reference's
format: src/mashbox/bshj.py:3-14). Tensors are aligned to `align` bytes and packed in the order given."""
import json
import struct

import numpy as np

CODES = {"uint16": "bf16", "float16": "f16", "float32": "f32", "int8": "i8", "uint8": "u8", "int32": "i32"}


def write(path, tensors, meta=None, align=4096, minor=0, major=1, magic=b"BSHJ", reserved=bytes(16), dtype_names=None):
    """tensors: name -> NumPy array (uint16 arrays are written as bf16 bits unless dtype_names says otherwise)"""
    pos, ents, bufs = 0, {}, []
    for name, a in tensors.items():
        a = np.ascontiguousarray(a)
        pos = -(-pos // align) * align
        dt = (dtype_names or {}).get(name, CODES[a.dtype.name])
        ents[name] = dict(dtype=dt, shape=list(a.shape), offset=pos, nbytes=a.nbytes, layout="row@1")
        bufs.append((pos, a.tobytes()))
        pos += a.nbytes
    hdr = dict(meta or {}, format="bshj", version=f"{major}.{minor}", data_len=pos, tensors=ents)
    raw = json.dumps(hdr, separators=(",", ":")).encode()
    off = -(-(64 + len(raw)) // align) * align
    raw += b" " * (off - 64 - len(raw))
    with open(path, "wb") as f:
        f.write(struct.pack("<4sHHQQIIQQ16s", magic, major, minor, len(raw), off, align, 1, pos, 0, reserved) + raw)
        for p, b in bufs:
            f.seek(off + p)
            f.write(b)
        f.truncate(off + pos)
    return ents
