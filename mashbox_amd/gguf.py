"""GGUF container reader: header, metadata and tensor directory parsed in place from an mmap (no copy of tensor bytes).

Serves the loader side of the quantized-linear path: a tensor's blocks come out as a (..., rows, row_bytes) uint8 view,
ready for mashbox_amd.kernels.repack_host / repack. Mirrors the reference's reader contract
(reference src/mashbox/gguf/reader.py:30-46, 49-87: File(path).tensors[name].rows(), dims reversed so that a weight is
(rows = out, cols = in), little-endian files only) with its own parser of the GGUF v2/v3 layout instead of gguf-py:

    magic "GGUF", u32 version, u64 tensor count, u64 metadata count
    metadata: (string key, u32 value type, value) ...        strings are u64 length + UTF-8 bytes
    tensor infos: (string name, u32 n_dims, u64 dims[n_dims] innermost first, u32 ggml type, u64 offset) ...
    tensor data: from the first multiple of general.alignment (default 32) after the directory; offsets are relative

A model split into shards (`<name>-00001-of-0000N.gguf`, reference src/mashbox/gguf/reader.py:14,49-65) is read as one:
opening any shard opens all N, their tensors together and each metadata key from the first shard that holds it; a
missing shard is an error naming it.
"""
from __future__ import annotations

import mmap
import os
import re
import struct

import numpy as np

# ggml type id -> (name, values per block, bytes per block) for the types whose row bytes this reader computes
# (reference src/mashbox/ops/reference.py:22-29)
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 16: ("IQ2_XXS", 256, 66),
    17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50), 20: ("IQ4_NL", 32, 18),
    21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136), 29: ("IQ1_M", 256, 56),
    30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66), 39: ("MXFP4", 32, 17), 40: ("NVFP4", 64, 36),
}

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_STRING, _ARRAY = 8, 9
MAGIC = b"GGUF"


class GGUFError(ValueError):
    """the file is not a GGUF container this reader can parse"""


class Tensor:
    """one tensor of a GGUF file: its ggml type, shape (outermost first: (rows, cols) for a weight) and raw bytes"""

    def __init__(self, name: str, t: int, shape: tuple, raw: np.ndarray):
        self.name, self.type, self.shape, self.raw = name, int(t), tuple(int(v) for v in shape), raw

    @property
    def type_name(self) -> str:
        return GGML_TYPES.get(self.type, (f"type{self.type}",))[0]

    @property
    def nbytes(self) -> int:
        return int(self.raw.size)

    def rows(self) -> np.ndarray:
        """raw bytes as (..., rows, row_bytes) uint8 (2-D and larger), (row_bytes,) for 1-D (reader.py:40-43)"""
        _, bs, ts = GGML_TYPES[self.type]
        rb = self.shape[-1] // bs * ts
        return self.raw.reshape(self.shape[:-1] + (rb,))

    def __repr__(self):
        return f"Tensor({self.name}, {self.type_name}, {self.shape})"


class _Cursor:
    def __init__(self, buf, pos=0):
        self.buf, self.pos = buf, pos

    def take(self, fmt: str):
        n = struct.calcsize(fmt)
        if self.pos + n > len(self.buf):
            raise GGUFError("truncated GGUF header")
        v = struct.unpack_from(fmt, self.buf, self.pos)[0]
        self.pos += n
        return v

    def string(self) -> str:
        n = self.take("<Q")
        if n > len(self.buf) - self.pos:
            raise GGUFError("truncated GGUF string")
        s = bytes(self.buf[self.pos:self.pos + n]).decode("utf-8", errors="replace")
        self.pos += n
        return s

    def value(self, vt: int):
        if vt in _SCALAR:
            return self.take(_SCALAR[vt])
        if vt == _STRING:
            return self.string()
        if vt == _ARRAY:
            it, n = self.take("<I"), self.take("<Q")
            if it in _SCALAR and it != 7:
                dt = np.dtype(_SCALAR[it])
                if self.pos + n * dt.itemsize > len(self.buf):
                    raise GGUFError("truncated GGUF array")
                a = np.frombuffer(self.buf, dtype=dt, count=n, offset=self.pos)
                self.pos += n * dt.itemsize
                return a
            return [self.value(it) for _ in range(n)]
        raise GGUFError(f"unknown GGUF metadata value type {vt}")


SPLIT = re.compile(r"-(\d{5})-of-(\d{5})\.gguf$")


def shard_paths(path: str) -> list:
    """every shard of the model `path` belongs to (itself when it is not a split file); GGUFError when one is missing"""
    m = SPLIT.search(path)
    if not m:
        return [path]
    count = int(m.group(2))
    paths = [f"{path[:m.start()]}-{i:05d}-of-{count:05d}.gguf" for i in range(1, count + 1)]
    missing = [os.path.basename(p) for p in paths if not os.path.exists(p)]
    if missing:
        raise GGUFError(f"{os.path.basename(path)} is shard {int(m.group(1))} of {count}; missing: {', '.join(missing)}")
    return paths


class File:
    """A GGUF model, one file or all the shards of a split one: .meta (key -> value), .tensors (name -> Tensor over the
    mmaps; bytes are never copied), .paths, .size"""

    def __init__(self, path: str):
        self.path = path
        self.paths = shard_paths(path)
        self._maps = []
        self.meta, self.tensors = {}, {}
        try:
            for p in self.paths:
                meta, tensors = self._read(p)
                for k, v in meta.items():
                    self.meta.setdefault(k, v)
                dup = set(tensors) & set(self.tensors)
                if dup:
                    raise GGUFError(f"{os.path.basename(p)}: tensor {sorted(dup)[0]} is also in an earlier shard")
                self.tensors.update(tensors)
        except Exception:
            self.close()
            raise
        self.size = sum(os.path.getsize(p) for p in self.paths)

    def _read(self, path: str):
        """one file -> (metadata, tensors)"""
        with open(path, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self._maps.append(mm)
        buf = memoryview(mm)
        c = _Cursor(buf)
        if len(buf) < 24 or bytes(buf[:4]) != MAGIC:
            raise GGUFError(f"{os.path.basename(path)} is not a GGUF file (magic {bytes(buf[:4])!r})")
        c.pos = 4
        self.version = c.take("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"{os.path.basename(path)}: GGUF version {self.version} (big-endian or unknown); "
                            "only little-endian v2/v3 files are read")
        nt, nkv = c.take("<Q"), c.take("<Q")
        meta = {}
        for _ in range(nkv):
            k = c.string()
            meta[k] = c.value(c.take("<I"))
        infos = []
        for _ in range(nt):
            name = c.string()
            nd = c.take("<I")
            dims = [c.take("<Q") for _ in range(nd)]
            t, off = c.take("<I"), c.take("<Q")
            infos.append((name, dims, t, off))
        align = int(meta.get("general.alignment", 32))
        start = (c.pos + align - 1) // align * align
        data = np.frombuffer(mm, dtype=np.uint8)
        tensors = {}
        for name, dims, t, off in infos:
            if t not in GGML_TYPES:
                raise GGUFError(f"{name}: unknown ggml type {t}")
            _, bs, ts = GGML_TYPES[t]
            shape = tuple(reversed(dims))                       # outermost first: (rows, cols) for a weight
            if shape[-1] % bs:
                raise GGUFError(f"{name}: {shape[-1]} values per row is not a multiple of {bs}")
            n = int(np.prod(shape, dtype=np.int64)) // bs * ts
            a = start + off
            if a + n > data.size:
                raise GGUFError(f"{name}: tensor bytes run past the end of the file")
            tensors[name] = Tensor(name, t, shape, data[a:a + n])
        return meta, tensors

    def get(self, key: str, default=None):
        return self.meta.get(key, default)

    def keys(self) -> list:
        return list(self.meta)

    @property
    def arch(self):
        return self.meta.get("general.architecture")

    def census(self):
        """-> ({type name: {"type", "tensors", "bytes"}} largest first, total tensor bytes)"""
        out, total = {}, 0
        for t in self.tensors.values():
            e = out.setdefault(t.type_name, {"type": t.type, "tensors": 0, "bytes": 0})
            e["tensors"] += 1
            e["bytes"] += t.nbytes
            total += t.nbytes
        return dict(sorted(out.items(), key=lambda kv: -kv[1]["bytes"])), total

    def close(self):
        self.tensors = {}
        for mm in self._maps:
            try:
                mm.close()
            except BufferError:
                pass        # a caller still holds a view; the map closes with the last one
        self._maps = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
