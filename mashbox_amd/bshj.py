"""Reader of .bshj weight files and the int8 per-row linears they hold.

The container (reference src/mashbox/bshj.py:1-16, the format of the reference's TPU weight files), little endian:

    0   4    magic b"BSHJ"             28  4   flags (bit 0: tensors packed back to back in header order)
    4   2+2  major (1), minor (<= 1)   32  8   data_len
    8   8    JSON header bytes         40  8   header hash (0 = not set)
    16  8    data_offset (% align = 0) 48  16  reserved, zero
    24  4    align (>= 4096)           64  ..  JSON {"tensors": {name: {dtype, shape, offset, nbytes, layout}}, ...}

Tensors start at data_offset + offset. A tensor is a zero-copy NumPy view of the memory-mapped file; bfloat16 tensors
are viewed as their uint16 bits (`torch_tensor` gives torch.bfloat16). The checks on open follow reference
src/mashbox/bshj.py:33-53: a bad magic, major, newer minor, nonzero reserved bytes, a misaligned or overlapping data
section, or a tensor record whose bytes disagree with its shape or run past the data raise ValueError.

int8 per-row linears (reference src/mashbox/models/qwen3_8_27b/weights.py:31-118): `<name>.weight` int8 (out, in) plus
`<name>.weight_scale` float32 (out,), weight = q * s per output row. `int8_weight` moves one to the GPU as the
{"q", "s"} form mashbox_amd.int8.linear / embed take; `int8_stack` fills one (L, out, in) + (L, out) buffer pair in
place, layer by layer, for the layer loop (weight l is {"q": q[l], "s": s[l]}).
"""
from __future__ import annotations

import json
import mmap
import struct

import numpy as np

FIXED = struct.Struct("<4sHHQQIIQQ16s")      # the 64-byte fixed header
MAX_MINOR = 1
DTYPES = {"bf16": np.dtype("<u2"), "f16": np.dtype("<f2"), "f32": np.dtype("<f4"), "f64": np.dtype("<f8"),
          "i8": np.dtype("i1"), "u8": np.dtype("u1"), "i16": np.dtype("<i2"), "u16": np.dtype("<u2"),
          "i32": np.dtype("<i4"), "u32": np.dtype("<u4"), "i64": np.dtype("<i8"), "u64": np.dtype("<u8")}


class File:
    """an open .bshj file: header(), meta(), tensors (name -> record), array(name), torch_tensor(name, device)"""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        try:
            self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError as e:                                       # an empty file cannot be mapped
            self._f.close()
            raise ValueError(f"{path}: not a BSHJ 1.x file ({e})") from None
        try:
            self._open()
        except Exception:
            self.close()
            raise

    def _open(self):
        path, mm = self.path, self._mm
        if len(mm) < FIXED.size:
            raise ValueError(f"{path}: not a BSHJ 1.x file (shorter than its fixed header)")
        magic, major, minor, jl, off, align, _flags, data_len, _hash, reserved = FIXED.unpack(mm[:FIXED.size])
        if magic != b"BSHJ" or major != 1:
            raise ValueError(f"{path}: not a BSHJ 1.x file")
        if minor > MAX_MINOR:
            raise ValueError(f"{path}: BSHJ 1.{minor} is newer than this reader (1.{MAX_MINOR})")
        if any(reserved) or align == 0 or off % align or off < FIXED.size + jl or off + data_len > len(mm):
            raise ValueError(f"{path}: bad container header")
        self.data_offset, self.align, self.data_len = off, align, data_len
        self.header = json.loads(bytes(mm[FIXED.size:FIXED.size + jl]).rstrip(b" \t\n\r").decode("utf-8"))
        self.tensors = self.header["tensors"]
        for name, t in self.tensors.items():
            dt = DTYPES.get(t["dtype"])
            if dt is None:
                raise ValueError(f"{path}: tensor {name} has unknown dtype {t['dtype']!r}")
            n = int(np.prod(t["shape"], dtype=np.int64)) * dt.itemsize
            if t["nbytes"] != n or t["offset"] % align or t["offset"] + n > data_len:
                raise ValueError(f"{path}: bad tensor record {name}")

    def meta(self) -> dict:
        return {k: v for k, v in self.header.items() if k != "tensors"}

    def array(self, name: str) -> np.ndarray:
        """zero-copy view of a tensor (bfloat16 as uint16 bits)"""
        t = self.tensors[name]
        dt = DTYPES[t["dtype"]]
        return np.frombuffer(self._mm, dtype=dt, count=t["nbytes"] // dt.itemsize,
                             offset=self.data_offset + t["offset"]).reshape(t["shape"])

    def torch_tensor(self, name: str, device=None):
        """a tensor copied into a torch tensor (bfloat16 as torch.bfloat16), on `device` if given"""
        import torch
        a = self.array(name)
        x = torch.from_numpy(np.array(a))                            # own the bytes: the map may close
        if self.tensors[name]["dtype"] == "bf16":
            x = x.view(torch.int16).view(torch.bfloat16)
        return x if device is None else x.to(device)

    def advise(self, name: str) -> None:
        """tell the OS a tensor is about to be read (read-ahead on a cold page cache)"""
        t = self.tensors[name]
        start = (self.data_offset + t["offset"]) & ~(mmap.PAGESIZE - 1)
        try:
            self._mm.madvise(mmap.MADV_WILLNEED, start, self.data_offset + t["offset"] + t["nbytes"] - start)
        except (AttributeError, OSError, ValueError):
            pass

    def close(self) -> None:
        try:
            self._mm.close()
        except BufferError:                                           # a caller still holds a view
            pass
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()


def prefix(names) -> str:
    """the tensor-name prefix of a file's layers (reference src/mashbox/models/qwen3_8_27b/weights.py:27-28)"""
    return "model.language_model." if any(k.startswith("model.language_model.") for k in names) else "model."


def quantised(f: File, name: str) -> bool:
    """True when `name` (a weight name without ".weight") is stored int8 per row: `<name>.weight_scale` exists"""
    return name + ".weight_scale" in f.tensors


def _check_int8(f: File, name: str):
    q, s = f.tensors.get(name), f.tensors.get(name + "_scale")
    if q is None or s is None or q["dtype"] != "i8" or s["dtype"] != "f32" or len(q["shape"]) != 2 \
            or list(s["shape"]) != [q["shape"][0]]:
        raise ValueError(f"{f.path}: {name} is not an int8 (out, in) weight with a float32 (out,) scale")
    return tuple(q["shape"])


def int8_weight(f: File, name: str, device="cuda") -> dict:
    """`<name>` (ending in ".weight") -> {"q": int8 (out, in), "s": float32 (out,)} on the device"""
    import torch
    _check_int8(f, name)
    f.advise(name)
    q = torch.from_numpy(np.array(f.array(name))).to(device)
    s = torch.from_numpy(np.array(f.array(name + "_scale"))).to(device)
    return {"q": q, "s": s}


def int8_stack(f: File, names, device="cuda") -> dict:
    """the int8 weights `names` (one per layer, same shape) -> {"q": (L, out, in), "s": (L, out)}, each buffer
    allocated once on the device and filled in place layer by layer"""
    import torch
    names = list(names)
    shapes = {_check_int8(f, n) for n in names}
    if len(shapes) != 1:
        raise ValueError(f"{f.path}: a stack needs one shape, got {sorted(shapes)}")
    (out, inp), = shapes
    q = torch.empty((len(names), out, inp), dtype=torch.int8, device=device)
    s = torch.empty((len(names), out), dtype=torch.float32, device=device)
    for i, n in enumerate(names):
        f.advise(n)
        q[i].copy_(torch.from_numpy(np.array(f.array(n))))
        s[i].copy_(torch.from_numpy(np.array(f.array(n + "_scale"))))
    return {"q": q, "s": s}


__all__ = ["File", "FIXED", "DTYPES", "prefix", "quantised", "int8_weight", "int8_stack"]
