"""Reader of .bshj weight files and the int8 per-row linears they hold.

The container is the reference's TPU weight format (reference src/mashbox/bshj.py:1-16), little endian:

    0   4    magic b"BSHJ"             28  4   flags (bit 0: tensors packed back to back in header order)
    4   2+2  major (1), minor (<= 1)   32  8   data_len
    8   8    JSON header bytes         40  8   header hash (0 = not set)
    16  8    data_offset (% align = 0) 48  16  reserved, zero
    24  4    align (>= 4096)           64  ..  JSON {"tensors": {name: {dtype, shape, offset, nbytes, layout}}, ...}

Tensors start at data_offset + offset. The file is parsed once into a `Header` and one `Record` per tensor, and every
problem found is reported together in one ValueError: a wrong magic or major version, a newer minor version, reserved
bytes that are not zero, a data section that is misaligned, overlaps the JSON header or runs past the end of the file,
and tensor records with an unknown dtype, a byte count that disagrees with their shape, a misaligned offset or bytes
past the data section (the checks of reference src/mashbox/bshj.py:33-53). A tensor is a zero-copy NumPy view of the
memory-mapped file; bfloat16 tensors are viewed as their uint16 bits (`torch_tensor` gives torch.bfloat16).

int8 per-row linears (reference src/mashbox/models/qwen3_8_27b/weights.py:31-118): `<name>.weight` int8 (out, in) plus
`<name>.weight_scale` float32 (out,), weight = q * s per output row. `int8_weight` moves one to the GPU as the
{"q", "s"} form mashbox_amd.int8.linear / embed take, or repacks it at load into the tiled planes the batched kernels
stream (packed=True); `int8_stack` fills one (L, out, in) + (L, out) buffer pair in place, layer by layer, for the
layer loop (weight l is {"q": q[l], "s": s[l]}).
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass

import numpy as np

FIXED = struct.Struct("<4sHHQQIIQQ16s")      # the 64-byte fixed header
MAX_MINOR = 1
DTYPES = {"bf16": np.dtype("<u2"), "f16": np.dtype("<f2"), "f32": np.dtype("<f4"), "f64": np.dtype("<f8"),
          "i8": np.dtype("i1"), "u8": np.dtype("u1"), "i16": np.dtype("<i2"), "u16": np.dtype("<u2"),
          "i32": np.dtype("<i4"), "u32": np.dtype("<u4"), "i64": np.dtype("<i8"), "u64": np.dtype("<u8")}


@dataclass(frozen=True)
class Header:
    """the fixed 64 bytes of a .bshj file"""
    magic: bytes
    major: int
    minor: int
    json_len: int
    data_offset: int
    align: int
    flags: int
    data_len: int
    header_hash: int
    reserved: bytes

    @classmethod
    def parse(cls, raw: bytes) -> "Header":
        return cls(*FIXED.unpack(raw))

    def problems(self, file_len: int) -> list:
        if self.magic != b"BSHJ" or self.major != 1:
            return [f"magic {self.magic!r} version {self.major}.{self.minor} is not BSHJ 1.x"]
        out = []
        if self.minor > MAX_MINOR:
            out.append(f"version 1.{self.minor} is newer than this reader (1.{MAX_MINOR})")
        if any(self.reserved):
            out.append("reserved header bytes are not zero")
        if self.align == 0 or self.data_offset % self.align:
            out.append(f"data offset {self.data_offset} is not a multiple of the alignment {self.align}")
        if self.data_offset < FIXED.size + self.json_len:
            out.append(f"data offset {self.data_offset} overlaps the {self.json_len}-byte JSON header")
        if self.data_offset + self.data_len > file_len:
            out.append(f"data section [{self.data_offset}, {self.data_offset + self.data_len}) runs past the "
                       f"{file_len}-byte file")
        return out


@dataclass(frozen=True)
class Record:
    """one tensor of the JSON header; offset is relative to the data section"""
    name: str
    dtype: str
    shape: tuple
    offset: int
    nbytes: int

    @property
    def np_dtype(self) -> np.dtype:
        return DTYPES[self.dtype]

    def problem(self, align: int, data_len: int):
        if self.dtype not in DTYPES:
            return f"tensor {self.name}: unknown dtype {self.dtype!r}"
        want = int(np.prod(self.shape, dtype=np.int64)) * self.np_dtype.itemsize
        if self.nbytes != want:
            return f"tensor {self.name}: {self.nbytes} bytes for shape {list(self.shape)} of {self.dtype} ({want})"
        if self.offset % align:
            return f"tensor {self.name}: offset {self.offset} is not a multiple of the alignment {align}"
        if self.offset + self.nbytes > data_len:
            return f"tensor {self.name}: bytes [{self.offset}, {self.offset + self.nbytes}) run past the data section"
        return None


class File:
    """an open .bshj file: meta(), tensors (name -> JSON record), records (name -> Record), array(name),
    torch_tensor(name, device), advise(name); a context manager"""

    def __init__(self, path: str):
        self.path = path
        self._fd = os.open(path, os.O_RDONLY)
        self._mm = None
        try:
            size = os.fstat(self._fd).st_size
            if size < FIXED.size:
                raise ValueError(f"{path}: {size} bytes, shorter than the {FIXED.size}-byte BSHJ header")
            self._mm = mmap.mmap(self._fd, 0, access=mmap.ACCESS_READ)
            self.fixed = Header.parse(self._mm[:FIXED.size])
            bad = self.fixed.problems(size)
            if not bad:
                text = bytes(self._mm[FIXED.size:FIXED.size + self.fixed.json_len]).decode("utf-8")
                self.header = json.loads(text)
                self.tensors = self.header["tensors"]
                self.records = {n: Record(n, t["dtype"], tuple(t["shape"]), int(t["offset"]), int(t["nbytes"]))
                                for n, t in self.tensors.items()}
                bad = [p for r in self.records.values() if (p := r.problem(self.fixed.align, self.fixed.data_len))]
            if bad:
                raise ValueError(f"{path}: not a readable BSHJ file: " + "; ".join(bad))
        except Exception:
            self.close()
            raise
        self.data_offset, self.align, self.data_len = self.fixed.data_offset, self.fixed.align, self.fixed.data_len

    def meta(self) -> dict:
        """the JSON header without its tensor table"""
        out = dict(self.header)
        out.pop("tensors", None)
        return out

    def array(self, name: str) -> np.ndarray:
        """zero-copy view of a tensor (bfloat16 as uint16 bits)"""
        r = self.records[name]
        start = self.data_offset + r.offset
        return np.frombuffer(self._mm, dtype=r.np_dtype, count=r.nbytes // r.np_dtype.itemsize, offset=start).reshape(r.shape)

    def torch_tensor(self, name: str, device=None):
        """a tensor copied into a torch tensor (bfloat16 as torch.bfloat16), on `device` if given"""
        import torch
        x = torch.from_numpy(self.array(name).copy())                 # owns its bytes: the map may close
        if self.records[name].dtype == "bf16":
            x = x.view(torch.int16).view(torch.bfloat16)
        return x if device is None else x.to(device)

    def advise(self, name: str) -> None:
        """ask the kernel to read a tensor's bytes ahead (a cold page cache); a hint only, never an error"""
        r = self.records[name]
        if hasattr(os, "posix_fadvise"):
            try:
                os.posix_fadvise(self._fd, self.data_offset + r.offset, r.nbytes, os.POSIX_FADV_WILLNEED)
            except OSError:
                pass

    def close(self) -> None:
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:                                       # a view of a tensor is still alive: the map
                pass                                                  # stays until it goes
            self._mm = None
        if self._fd is not None:
            os.close(self._fd)
            self._fd = None

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


def _int8_shape(f: File, name: str) -> tuple:
    q, s = f.records.get(name), f.records.get(name + "_scale")
    if q is None or s is None or q.dtype != "i8" or s.dtype != "f32" or len(q.shape) != 2 or s.shape != q.shape[:1]:
        raise ValueError(f"{f.path}: {name} is not an int8 (out, in) weight with a float32 (out,) scale")
    return q.shape


def int8_weight(f: File, name: str, device="cuda", packed: bool = False):
    """`<name>` (ending in ".weight") -> {"q": int8 (out, in), "s": float32 (out,)} on the device, or with packed=True
    its load-time repack into tiled planes (mashbox_amd.int8.Int8Planes)"""
    import torch
    _int8_shape(f, name)
    f.advise(name)
    q = torch.from_numpy(f.array(name).copy()).to(device)
    s = torch.from_numpy(f.array(name + "_scale").copy()).to(device)
    if packed:
        from . import int8
        return int8.repack(q, s)
    return {"q": q, "s": s}


def int8_stack(f: File, names, device="cuda") -> dict:
    """the int8 weights `names` (one per layer, same shape) -> {"q": (L, out, in), "s": (L, out)}, each buffer
    allocated once on the device and filled in place layer by layer"""
    import torch
    names = list(names)
    shapes = {_int8_shape(f, n) for n in names}
    if len(shapes) != 1:
        raise ValueError(f"{f.path}: a stack needs one shape, got {sorted(shapes)}")
    (out, inp), = shapes
    q = torch.empty((len(names), out, inp), dtype=torch.int8, device=device)
    s = torch.empty((len(names), out), dtype=torch.float32, device=device)
    for i, n in enumerate(names):
        f.advise(n)
        q[i].copy_(torch.from_numpy(f.array(n).copy()))
        s[i].copy_(torch.from_numpy(f.array(n + "_scale").copy()))
    return {"q": q, "s": s}


__all__ = ["File", "Header", "Record", "FIXED", "DTYPES", "prefix", "quantised", "int8_weight", "int8_stack"]
