"""int8 per-output-channel linear and embedding rows on the MI355X kernels.

linear: restates the contract of reference src/mashbox/models/qwen3_8_27b/model.py:72-82 for w = {"q": int8 (out, in),
"s": float32 (out,)}: y = (x @ bf16(q).T with float32 accumulation) * s, rounded to x's dtype; with pj, pj receives the
float32 y * s before the rounding. Activations are bfloat16 (the model's activation dtype); other dtypes raise.
The weights run as the reference holds them (the dict), or repacked once at load (repack / repack_host -> Int8Planes:
16-row tiles whose MFMA operand tile of 16 rows x 64 bytes is one contiguous KiB, the layout the batched kernels
stream at full rate), with identical results.

embed: reference model.py:132-139 for an int8 table E = {"q": int8 (N, D), "s": float32 (N,)}: the rows of toks as
f32(q) * s, rounded to bfloat16 (pj receives the float32 rows first); token ids index as jax.numpy does (negative ids
count from the end, ids past either end are clamped).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import I8T, OUT_BF16, OUT_F32, check, lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class Int8Planes:
    """int8 per-output-channel weights repacked once at load into 16-row tiles (libmbq's MBQ_I8T planes): `buf` is a
    flat uint8 tensor of count * plane_bytes bytes (host or device) holding one (N, K) weight, or a stack of them along
    `lead` (weight i at byte i * plane_bytes)"""

    def __init__(self, buf: torch.Tensor, n: int, k: int, lead=()):
        self.buf, self.N, self.K, self.lead = buf, int(n), int(k), tuple(int(v) for v in lead)
        self.stride = check(lib().mbq_plane_bytes(I8T, self.N, self.K), "int8 plane_bytes")

    @property
    def count(self) -> int:
        c = 1
        for v in self.lead:
            c *= v
        return c

    def to(self, device) -> "Int8Planes":
        return Int8Planes(self.buf.to(device), self.N, self.K, self.lead)

    def __getitem__(self, i) -> "Int8Planes":
        """one weight of a stack along its first axis: a view, no copy"""
        if not self.lead:
            raise IndexError("planes of one weight have no stacked axis")
        i = int(i)
        if not -self.lead[0] <= i < self.lead[0]:
            raise IndexError(i)
        i %= self.lead[0]
        size = (self.count // self.lead[0]) * self.stride
        return Int8Planes(self.buf[i * size:(i + 1) * size], self.N, self.K, self.lead[1:])

    def __repr__(self):
        return f"Int8Planes(lead={self.lead}, ({self.N}, {self.K}), {self.buf.device})"


def plane_bytes(n: int, k: int) -> int:
    return check(lib().mbq_plane_bytes(I8T, int(n), int(k)), "int8 plane_bytes")


def repack_host(q, s, threads: int = 0) -> Int8Planes:
    """host int8 q (..., N, K) and float32 s (..., N) -> host planes, on the host's cores (leading axes: a stack)"""
    q = np.ascontiguousarray(np.asarray(q), dtype=np.int8)
    s = np.ascontiguousarray(np.asarray(s), dtype=np.float32)
    n, k = q.shape[-2:]
    lead = q.shape[:-2]
    if s.shape != lead + (n,):
        raise ValueError(f"scales {s.shape} do not match quants {q.shape}")
    pb = plane_bytes(n, k)
    count = int(np.prod(lead, dtype=np.int64)) if lead else 1
    out = torch.empty(count * pb, dtype=torch.uint8)
    qf, sf = q.reshape(count, n, k), s.reshape(count, n)
    for i in range(count):
        check(lib().mbq_int8_repack_host(qf[i].ctypes.data_as(ctypes.c_void_p), sf[i].ctypes.data_as(ctypes.c_void_p),
                                         n, k, ctypes.c_void_p(out.data_ptr() + i * pb), pb, int(threads)),
              "int8 repack_host")
    return Int8Planes(out, n, k, lead)


def repack(q: torch.Tensor, s: torch.Tensor) -> Int8Planes:
    """device int8 q (..., N, K) and float32 s (..., N) -> device planes, by the GPU (leading axes: a stack)"""
    if not q.is_cuda:
        return repack_host(q.numpy(), s.numpy()).to(torch.device("cuda", torch.cuda.current_device()))
    if q.dtype != torch.int8:
        raise TypeError(f"q must be int8, got {q.dtype}")
    q = q.contiguous()
    s = s.to(device=q.device, dtype=torch.float32).contiguous()
    n, k = q.shape[-2:]
    lead = tuple(q.shape[:-2])
    if tuple(s.shape) != lead + (n,):
        raise ValueError(f"scales {tuple(s.shape)} do not match quants {tuple(q.shape)}")
    pb = plane_bytes(n, k)
    count = q.numel() // (n * k)
    out = torch.empty(count * pb, dtype=torch.uint8, device=q.device)
    qf, sf = q.reshape(count, n, k), s.reshape(count, n)
    for i in range(count):
        check(lib().mbq_int8_repack_dev(ctypes.c_void_p(qf[i].data_ptr()), ctypes.c_void_p(sf[i].data_ptr()), n, k,
                                        ctypes.c_void_p(out.data_ptr() + i * pb), _stream()), "int8 repack")
    return Int8Planes(out, n, k, lead)


def _planes_linear(x: torch.Tensor, p: Int8Planes, layer, f32: bool) -> torch.Tensor:
    if not p.buf.is_cuda:
        raise ValueError(f"{p} is on the host: move the planes to the GPU (planes.to('cuda'))")
    if x.shape[-1] != p.K:
        raise ValueError(f"x has {x.shape[-1]} columns, the weight {p.K}")
    lh, ld, nl = 0, None, 1
    if layer is None:
        if p.lead:
            raise ValueError(f"{p}: a stack needs layer= (or index it first)")
    else:
        if len(p.lead) != 1:
            raise ValueError(f"{p}: layer= needs planes stacked on exactly one axis")
        nl = p.lead[0]
        if isinstance(layer, torch.Tensor) and layer.is_cuda:
            ld = layer.reshape(()).to(torch.int32)
        else:
            lh = int(layer)
    lead = tuple(x.shape[:-1])
    m = 1
    for v in lead:
        m *= int(v)
    y = torch.empty(lead + (p.N,), dtype=torch.float32 if f32 else torch.bfloat16, device=p.buf.device)
    if m == 0:
        return y.zero_()
    x2 = x.reshape(m, p.K).to(p.buf.device).contiguous()
    check(lib().mbq_matmul(I8T, ctypes.c_void_p(p.buf.data_ptr()), lh, None if ld is None else ctypes.c_void_p(ld.data_ptr()),
                           nl, ctypes.c_void_p(x2.data_ptr()), m, p.N, p.K, ctypes.c_void_p(y.data_ptr()),
                           OUT_F32 if f32 else OUT_BF16, _stream()), f"int8 linear {p}")
    return y


def linear(x: torch.Tensor, w, pj=None, layer=None) -> torch.Tensor:
    """x (..., in) bfloat16 @ w -> (..., out) in x's dtype (reference src/mashbox/models/qwen3_8_27b/model.py:72-82).
    w: the reference's form {'q': int8 (out, in), 's': float32 (out,)} on the GPU, or its load-time repack Int8Planes
    (layer= reads one weight of a one-axis stack in place: an int, or a 0-d int32 device tensor read by the kernel)"""
    if x.dtype != torch.bfloat16:
        raise TypeError(f"int8 linear runs bfloat16 activations, got {x.dtype}")
    if isinstance(w, Int8Planes):
        y = _planes_linear(x, w, layer, pj is not None)
        return y if pj is None else pj(y).to(x.dtype)
    if not isinstance(w, dict):
        raise TypeError("linear takes the int8 form {'q': int8 (out, in), 's': float32 (out,)} or Int8Planes")
    if layer is not None:
        raise ValueError("layer= needs Int8Planes (a repacked stack)")
    q, s = w["q"], w["s"]
    if q.dtype != torch.int8 or q.dim() != 2 or not q.is_cuda:
        raise TypeError("w['q'] must be a 2-D int8 tensor on the GPU")
    n, k = q.shape
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} columns, q {k}")
    s = s.to(device=q.device, dtype=torch.float32).contiguous()
    if s.shape != (n,):
        raise ValueError(f"w['s'] must be ({n},), got {tuple(s.shape)}")
    q = q.contiguous()
    lead = tuple(x.shape[:-1])
    m = 1
    for v in lead:
        m *= int(v)
    f32 = pj is not None
    y = torch.empty(lead + (n,), dtype=torch.float32 if f32 else torch.bfloat16, device=q.device)
    if m == 0:
        y.zero_()
    else:
        x2 = x.reshape(m, k).to(q.device).contiguous()
        check(lib().mbq_int8_linear(ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(s.data_ptr()),
                                    ctypes.c_void_p(x2.data_ptr()), m, n, k, ctypes.c_void_p(y.data_ptr()),
                                    OUT_F32 if f32 else OUT_BF16, _stream()), "int8 linear")
    if pj is not None:
        return pj(y).to(x.dtype)
    return y


def embed(E, toks: torch.Tensor, pj=None) -> torch.Tensor:
    """embedding rows of toks (any shape) -> (*toks.shape, D) bfloat16 (reference model.py:132-139). E: the int8 table
    {"q", "s"} on the GPU (the gather kernel of libmbq.so), or a plain (N, D) table."""
    if not isinstance(E, dict):
        n = E.shape[0]
        idx = toks.to(device=E.device, dtype=torch.int64)
        idx = torch.where(idx < 0, idx + n, idx).clamp(0, n - 1)
        return E[idx] if pj is None else pj(E[idx].float()).to(torch.bfloat16)
    q, s = E["q"], E["s"]
    if q.dtype != torch.int8 or q.dim() != 2 or not q.is_cuda:
        raise TypeError("E['q'] must be a 2-D int8 tensor on the GPU")
    n, d = q.shape
    s = s.to(device=q.device, dtype=torch.float32).contiguous()
    if s.shape != (n,):
        raise ValueError(f"E['s'] must be ({n},), got {tuple(s.shape)}")
    if toks.dtype.is_floating_point or toks.dtype == torch.bool:
        raise TypeError(f"token ids must be integers, got {toks.dtype}")
    q = q.contiguous()
    t = toks.to(device=q.device, dtype=torch.int32).contiguous()
    y = torch.empty(tuple(toks.shape) + (d,), dtype=torch.float32 if pj is not None else torch.bfloat16, device=q.device)
    if t.numel():
        check(lib().mbq_int8_embed(ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(s.data_ptr()), n, d,
                                   ctypes.c_void_p(t.data_ptr()), t.numel(), ctypes.c_void_p(y.data_ptr()),
                                   OUT_F32 if pj is not None else OUT_BF16, _stream()), "int8 embed")
    return y if pj is None else pj(y).to(torch.bfloat16)
