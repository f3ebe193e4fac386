"""int8 per-output-channel linear and embedding rows on the MI355X kernels.

linear: restates the contract of reference src/mashbox/models/qwen3_8_27b/model.py:72-82 for w = {"q": int8 (out, in),
"s": float32 (out,)}: y = (x @ bf16(q).T with float32 accumulation) * s, rounded to x's dtype; with pj, pj receives the
float32 y * s before the rounding. Activations are bfloat16 (the model's activation dtype); other dtypes raise.

embed: reference model.py:132-139 for an int8 table E = {"q": int8 (N, D), "s": float32 (N,)}: the rows of toks as
f32(q) * s, rounded to bfloat16 (pj receives the float32 rows first); token ids index as jax.numpy does (negative ids
count from the end, ids past either end are clamped).
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import OUT_BF16, OUT_F32, check, lib


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def linear(x: torch.Tensor, w, pj=None) -> torch.Tensor:
    """x (..., in) bfloat16 @ w -> (..., out) in x's dtype (reference src/mashbox/models/qwen3_8_27b/model.py:72-82)"""
    if not isinstance(w, dict):
        raise TypeError("linear takes the int8 form {'q': int8 (out, in), 's': float32 (out,)}")
    q, s = w["q"], w["s"]
    if x.dtype != torch.bfloat16:
        raise TypeError(f"int8 linear runs bfloat16 activations, got {x.dtype}")
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
