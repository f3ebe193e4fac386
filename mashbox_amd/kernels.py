"""mashbox's kernel-package surface, served by the MI355X kernels of libmbq.so.

mashbox's ops boundary imports a kernel package by module name (reference src/mashbox/ops/__init__.py:273-311,
env MASHBOX_GGUF_KERNELS) and uses this surface (reference src/mashbox/ops/__init__.py:11-34):

    TYPES                                    ggml type ids with kernel planes: Q4_0 (2), Q8_0 (8), Q4_K (12), Q5_K (13),
                                             Q6_K (14)
    repack_host(t, raw, shape) -> planes     host NumPy blocks (..., rows, row_bytes) -> planes (host, then .to(dev))
    repack(t, raw, shape, stacked=False)     device blocks (torch uint8 on the GPU) -> planes on the GPU
    matmul(x, planes, layer=None) -> y       x (..., cols) @ W.T as float32 (..., rows); layer= reads one weight of a
                                             stack in place (an int, or a 0-d int32 device tensor read by the kernel)
    dequant(planes) -> float32 (..., rows, cols), bit for bit the reference dequantization
    plane_bytes(t, shape) -> int             device bytes of one (rows, cols) weight's planes
    kq_covers(t, shape) -> bool              the shapes the kernels run
    picks_layer = True                       matmul takes layer=

Arrays are torch tensors (PyTorch-ROCm holds device memory and streams); every call is ordered on torch's current
stream. Errors raise (mashbox's boundary catches them and sends the weight to its exact path, loudly:
reference src/mashbox/ops/__init__.py:441-459); nothing here computes on the host.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import INT8, OUT_BF16, OUT_F32, Q4_0, Q40T, Q4_K, Q4KT, Q5_K, Q5KT, Q6_K, Q6KT, Q8_0, Q8T, check, lib

# the types the reference's kernel package gives planes (reference src/mashbox/ops/bundle.py:39)
TYPES = frozenset({Q4_0, Q8_0, Q4_K, Q5_K, Q6_K})
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q4KT: "Q4_K tiled", Q8T: "Q8_0 tiled",
         Q5KT: "Q5_K tiled", Q6KT: "Q6_K tiled", Q40T: "Q4_0 tiled"}
# values and bytes per block (reference ops/reference.py:22-29)
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
# ggml types whose blocks also repack into 16-row tiles (repack(..., tiled=True)), and the plane type they take: every
# wave-wide weight load of a 16-row MFMA tile is one contiguous KiB (the layout for decode batches of several rows)
TILED = {Q4_0: Q40T, Q4_K: Q4KT, Q8_0: Q8T, Q5_K: Q5KT, Q6_K: Q6KT}
picks_layer = True
version = "0.1.0"


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def row_bytes(t: int, cols: int) -> int:
    return check(lib().mbq_row_bytes(int(t), int(cols)), f"row_bytes({t}, {cols})")


def plane_bytes(t: int, shape) -> int:
    """device bytes of one (rows, cols) weight's planes (reference src/mashbox/ops/__init__.py:24,374-378)"""
    rows, cols = (int(v) for v in tuple(shape)[-2:])
    return check(lib().mbq_plane_bytes(int(t), rows, cols), f"plane_bytes({t}, {tuple(shape)})")


def kq_covers(t: int, shape) -> bool:
    """True when the kernels run a (rows, cols) weight of type t (reference src/mashbox/ops/__init__.py:359-363)"""
    if int(t) not in TYPES:
        return False
    if len(tuple(shape)) < 2:
        return True
    rows, cols = (int(v) for v in tuple(shape)[-2:])
    return bool(lib().mbq_covers(int(t), rows, cols))


# weight layouts repack can produce: the row-major planes, the 16-row tiles of TILED[t], or both (tiles, with the
# row-major planes of the same weights beside them for single-row calls)
LAYOUTS = ("rowmajor", "tiles", "both")


class Planes:
    """The kernel planes of one (rows, cols) weight or a stack of them: `buf` is a flat uint8 tensor of
    prod(lead) * plane_bytes bytes (host or device), weight i of the stack at byte i * plane_bytes. `alt`, when set, is
    the row-major planes of the same weights (layout "both"): matmul runs single-row calls on it (the decode GEMV) and
    everything else on these planes."""

    def __init__(self, buf: torch.Tensor, t: int, n: int, k: int, lead=(), alt: "Planes | None" = None):
        self.buf, self.t, self.N, self.K, self.lead = buf, int(t), int(n), int(k), tuple(int(v) for v in lead)
        self.stride = plane_bytes(self.t, (self.N, self.K))
        self.alt = alt

    @property
    def count(self) -> int:
        c = 1
        for v in self.lead:
            c *= v
        return c

    @property
    def nbytes(self) -> int:
        """bytes the planes take (both layouts' with `alt`)"""
        return self.buf.numel() + (self.alt.nbytes if self.alt is not None else 0)

    def to(self, device) -> "Planes":
        return Planes(self.buf.to(device), self.t, self.N, self.K, self.lead,
                      None if self.alt is None else self.alt.to(device))

    def __getitem__(self, i) -> "Planes":
        """one weight (or sub-stack) of a stack along the first stacked axis: a view, no copy"""
        if not self.lead:
            raise IndexError("planes of one weight have no stacked axis")
        inner = 1
        for v in self.lead[1:]:
            inner *= v
        i = int(i)
        if not -self.lead[0] <= i < self.lead[0]:
            raise IndexError(i)
        i %= self.lead[0]
        size = inner * self.stride
        return Planes(self.buf[i * size:(i + 1) * size], self.t, self.N, self.K, self.lead[1:],
                      None if self.alt is None else self.alt[i])

    def __repr__(self):
        extra = " + row-major" if self.alt is not None else ""
        return f"Planes({NAMES.get(self.t, self.t)}{extra}, lead={self.lead}, ({self.N}, {self.K}), {self.buf.device})"


def _check_raw(t: int, raw_shape, shape):
    t = int(t)
    if t not in TYPES:
        raise NotImplementedError(f"ggml type {t} has no kernel planes (TYPES = {sorted(TYPES)})")
    rows, cols = (int(v) for v in tuple(shape)[-2:])
    rb = row_bytes(t, cols)
    if tuple(raw_shape[-2:]) != (rows, rb):
        raise ValueError(f"raw {tuple(raw_shape)} is not (..., {rows}, {rb}) for {NAMES[t]} ({rows}, {cols})")
    return t, rows, cols, tuple(int(v) for v in raw_shape[:-2])


def _layout_of(t: int, tiled: bool, layout) -> str:
    """the layout of a repack call: `layout` when given (one of LAYOUTS), else tiles when tiled=True"""
    if layout is None:
        return "tiles" if tiled else "rowmajor"
    if layout not in LAYOUTS:
        raise ValueError(f"layout {layout!r} is not one of {LAYOUTS}")
    if layout != "rowmajor" and int(t) not in TILED:
        raise NotImplementedError(f"{NAMES.get(int(t), t)} has no tiled planes (tiled: {[NAMES[v] for v in TILED]})")
    return layout


def _plane_type(t: int, tiled: bool) -> int:
    if not tiled:
        return t
    if t not in TILED:
        raise NotImplementedError(f"{NAMES.get(t, t)} has no tiled planes (tiled: {[NAMES[v] for v in TILED]})")
    return TILED[t]


def repack_host(t: int, raw, shape, threads: int = 0, tiled: bool = False, layout=None) -> Planes:
    """host blocks (..., rows, row_bytes) uint8 -> host planes, on the host's cores (C++ threads)
    (reference src/mashbox/ops/__init__.py:22-23,473-474); tiled=True (or layout="tiles"): the 16-row tiles of TILED[t];
    layout="both": the tiles with the row-major planes as `alt`"""
    lay = _layout_of(t, tiled, layout)
    if lay == "both":
        p = repack_host(t, raw, shape, threads, layout="tiles")
        p.alt = repack_host(t, raw, shape, threads)
        return p
    tiled = lay == "tiles"
    raw = np.ascontiguousarray(np.asarray(raw), dtype=np.uint8)
    t, rows, cols, lead = _check_raw(t, raw.shape, shape)
    t = _plane_type(t, tiled)
    pb = plane_bytes(t, (rows, cols))
    count = int(np.prod(lead, dtype=np.int64)) if lead else 1
    out = torch.empty(count * pb, dtype=torch.uint8)
    flat = raw.reshape(count, rows * raw.shape[-1])
    for i in range(count):
        dst = out[i * pb:(i + 1) * pb]
        check(lib().mbq_repack_host(t, flat[i].ctypes.data_as(ctypes.c_void_p), rows, cols,
                                    ctypes.c_void_p(dst.data_ptr()), pb, int(threads)), "repack_host")
    return Planes(out, t, rows, cols, lead)


def repack(t: int, raw: torch.Tensor, shape, stacked: bool = False, tiled: bool = False, layout=None) -> Planes:
    """device blocks (..., rows, row_bytes) uint8 (a torch tensor on the GPU) -> device planes, by the GPU
    (reference src/mashbox/ops/__init__.py:16,475-485). `stacked` is accepted for the surface; leading axes are a stack.
    tiled=True (or layout="tiles"): the 16-row tiles of TILED[t]; layout="both": the tiles with the row-major planes as
    `alt`."""
    lay = _layout_of(t, tiled, layout)
    if not raw.is_cuda:
        return repack_host(t, raw.numpy(), shape, layout=lay).to(torch.device("cuda", torch.cuda.current_device()))
    if lay == "both":
        p = repack(t, raw, shape, stacked, layout="tiles")
        p.alt = repack(t, raw, shape, stacked)
        return p
    tiled = lay == "tiles"
    raw = raw.contiguous()
    t, rows, cols, lead = _check_raw(t, tuple(raw.shape), shape)
    t = _plane_type(t, tiled)
    pb = plane_bytes(t, (rows, cols))
    count = int(np.prod(lead, dtype=np.int64)) if lead else 1
    out = torch.empty(count * pb, dtype=torch.uint8, device=raw.device)
    flat = raw.reshape(count, -1)
    for i in range(count):
        check(lib().mbq_repack_dev(t, _ptr(flat[i]), rows, cols, ctypes.c_void_p(out.data_ptr() + i * pb), _stream()),
              "repack")
    return Planes(out, t, rows, cols, lead)


def _layer_args(p: Planes, layer):
    """-> (planes for the call, host layer, device layer tensor or None, nlayers)"""
    if layer is None:
        if p.lead:
            raise ValueError(f"{p}: a stack needs layer= (or index it first)")
        return p, 0, None, 1
    if len(p.lead) != 1:
        raise ValueError(f"{p}: layer= needs planes stacked on exactly one axis")
    if isinstance(layer, torch.Tensor):
        if layer.numel() != 1:
            raise ValueError("layer must be a scalar")
        if layer.is_cuda:
            lt = layer.reshape(()).to(torch.int32)
            return p, 0, lt, p.lead[0]
        layer = int(layer.item())
    return p, int(layer), None, p.lead[0]


def _out(y_shape, device, dtype):
    return torch.empty(y_shape, dtype=dtype, device=device)


def matmul(x: torch.Tensor, p: Planes, layer=None, out_dtype=torch.float32) -> torch.Tensor:
    """x (..., cols) @ W.T -> (..., rows) float32 (or bfloat16 with out_dtype), float32 accumulation.
    x is cast to bfloat16 first (the call contract of reference src/mashbox/ops/bundle.py:559-598); no rows gives an
    empty result without a launch. layer= reads weight `layer` of a one-axis stack in place."""
    if not p.buf.is_cuda:
        raise ValueError(f"{p} is on the host: move the planes to the GPU (planes.to('cuda'))")
    if p.alt is not None and x.numel() == x.shape[-1]:
        p = p.alt                                     # one activation row: the row-major planes' decode GEMV
    p, lh, ld, nl = _layer_args(p, layer)
    lead = tuple(x.shape[:-1])
    if x.shape[-1] != p.K:
        raise ValueError(f"x has {x.shape[-1]} columns, the weight {p.K}")
    m = 1
    for v in lead:
        m *= int(v)
    y = _out(lead + (p.N,), p.buf.device, out_dtype)
    if m == 0:
        return y.zero_()
    x2 = x.reshape(m, p.K).to(device=p.buf.device, dtype=torch.bfloat16).contiguous()
    od = OUT_BF16 if out_dtype == torch.bfloat16 else OUT_F32
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"out_dtype {out_dtype}")
    check(lib().mbq_matmul(p.t, _ptr(p.buf), lh, None if ld is None else _ptr(ld), nl, _ptr(x2), m, p.N, p.K, _ptr(y),
                           od, _stream()), f"matmul {p}")
    return y


def dequant(p: Planes, layer=None) -> torch.Tensor:
    """planes -> float32 (lead..., rows, cols) on the device, bit for bit the reference dequantization
    (reference src/mashbox/ops/__init__.py:20,691-705)"""
    if not p.buf.is_cuda:
        raise ValueError(f"{p} is on the host: move the planes to the GPU (planes.to('cuda'))")
    if layer is not None:
        p, lh, ld, nl = _layer_args(p, layer)
        w = torch.empty((p.N, p.K), dtype=torch.float32, device=p.buf.device)
        check(lib().mbq_dequant(p.t, _ptr(p.buf), lh, None if ld is None else _ptr(ld), nl, p.N, p.K, _ptr(w), _stream()),
              f"dequant {p}")
        return w
    w = torch.empty((p.count, p.N, p.K), dtype=torch.float32, device=p.buf.device)
    for i in range(p.count):
        check(lib().mbq_dequant(p.t, _ptr(p.buf), i, None, p.count, p.N, p.K, _ptr(w[i]), _stream()), f"dequant {p}")
    return w.reshape(p.lead + (p.N, p.K))


def take_rows(p: Planes, ids, layer=None) -> torch.Tensor:
    """rows `ids` (any int shape; below zero counts from the end, then clamped, as jax.numpy indexes) of the weight as
    float32 (*ids.shape, cols), dequantizing only those rows: bit for bit dequant(p)[ids]"""
    if not p.buf.is_cuda:
        raise ValueError(f"{p} is on the host: move the planes to the GPU (planes.to('cuda'))")
    ids = torch.as_tensor(ids, device=p.buf.device)
    idx = ids.reshape(-1).to(torch.int32).contiguous()
    if layer is None and p.lead:
        raise ValueError(f"{p}: a stack needs layer= (or index it first)")
    q, lh, ld, nl = (p, 0, None, 1) if layer is None else _layer_args(p, layer)
    w = torch.empty((idx.numel(), p.K), dtype=torch.float32, device=p.buf.device)
    check(lib().mbq_dequant_rows(p.t, _ptr(q.buf), lh, None if ld is None else _ptr(ld), nl, p.N, p.K, _ptr(idx),
                                 idx.numel(), _ptr(w), _stream()), f"take_rows {p}")
    return w.reshape(tuple(ids.shape) + (p.K,))


__all__ = ["TYPES", "TILED", "LAYOUTS", "take_rows", "Planes", "repack_host", "repack", "matmul", "dequant", "plane_bytes", "kq_covers",
           "picks_layer", "row_bytes", "INT8", "Q4KT", "Q8T", "Q5KT", "Q6KT", "Q40T"]
