"""A writer of little-endian GGUF v3 files from the container layout (test fixtures only): metadata of scalars,
strings and arrays, and tensors given as raw block bytes (uint8 (..., rows, row_bytes)) with a ggml type and logical
shape. Split models are written as shards that each hold some tensors, the first one all the metadata."""
import struct

import numpy as np

_SCALARS = {"u8": (0, "<B"), "i8": (1, "<b"), "u16": (2, "<H"), "i16": (3, "<h"), "u32": (4, "<I"), "i32": (5, "<i"),
            "f32": (6, "<f"), "bool": (7, "<?"), "u64": (10, "<Q"), "i64": (11, "<q"), "f64": (12, "<d")}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(v):
    """-> (value type, bytes): str, bool, int (i64), float (f64), (kind, value) for an explicit scalar kind, or a list /
    NumPy array (arrays of numbers, strings)"""
    if isinstance(v, tuple):
        vt, fmt = _SCALARS[v[0]]
        return vt, struct.pack(fmt, v[1])
    if isinstance(v, bool):
        return 7, struct.pack("<?", v)
    if isinstance(v, int):
        return 11, struct.pack("<q", v)
    if isinstance(v, float):
        return 12, struct.pack("<d", v)
    if isinstance(v, str):
        return 8, _str(v)
    if isinstance(v, np.ndarray):
        code = {np.dtype("int32"): 5, np.dtype("float32"): 6, np.dtype("uint8"): 0, np.dtype("int64"): 11}[v.dtype]
        return 9, struct.pack("<IQ", code, v.size) + v.astype(v.dtype.newbyteorder("<")).tobytes()
    if isinstance(v, list):
        assert all(isinstance(e, str) for e in v)
        return 9, struct.pack("<IQ", 8, len(v)) + b"".join(_str(e) for e in v)
    raise TypeError(type(v))


def write(path, meta: dict, tensors: dict, align: int = 32):
    """tensors: name -> (ggml type, logical shape outermost first, raw uint8 bytes)"""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta))
    for k, v in meta.items():
        vt, b = _value(v)
        head += _str(k) + struct.pack("<I", vt) + b
    offsets, off = [], 0
    for name, (t, shape, raw) in tensors.items():
        offsets.append(off)
        off += (np.asarray(raw).nbytes + align - 1) // align * align
    for (name, (t, shape, raw)), o in zip(tensors.items(), offsets):
        dims = list(reversed(shape))                          # innermost first
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, o)
    pad = (len(head) + align - 1) // align * align - len(head)
    with open(path, "wb") as f:
        f.write(head + bytes(pad))
        for (name, (t, shape, raw)), o in zip(tensors.items(), offsets):
            b = np.ascontiguousarray(raw, dtype=np.uint8).tobytes()
            f.write(b + bytes((len(b) + align - 1) // align * align - len(b)))


def write_split(stem, meta: dict, tensors: dict, shards: int):
    """the model as `stem-0000i-of-0000N.gguf`: tensors dealt round robin, metadata in shard 1 plus the split keys"""
    names = list(tensors)
    paths = []
    for i in range(shards):
        part = {n: tensors[n] for n in names[i::shards]}
        m = dict(meta) if i == 0 else {}
        m.update({"split.no": ("u16", i), "split.count": ("u16", shards)})
        p = f"{stem}-{i + 1:05d}-of-{shards:05d}.gguf"
        write(p, m, part)
        paths.append(p)
    return paths
