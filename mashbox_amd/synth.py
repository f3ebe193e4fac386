"""Seeded synthetic GGUF / int8 weights and bf16 activations, generated on the GPU (for the bench's large workloads).

Value ranges are those of the five BASELINE configs: fp16 block scales d (and Q4_K dmin) ~ U(1e-3, 1e-2), Q8_0 / int8
quants uniform in [-127, 127], Q4_K six-bit scales and mins uniform in [0, 63] packed as the Q4_K scale bytes hold
them (reference src/mashbox/ops/reference.py:132-139), four-bit quants uniform in [0, 15], int8 per-row scales
~ U(1e-3, 1e-2), activations ~ N(0, 1) rounded to bfloat16. The bytes are the file's block layout (Q8_0 34 B per 32
values, Q4_K 144 B per 256), ready for repack.
"""
from __future__ import annotations

import torch


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def _uniform_f16_bytes(g, shape, lo, hi, device):
    v = torch.rand(shape, generator=g, device=device, dtype=torch.float32) * (hi - lo) + lo
    return v.to(torch.float16).view(torch.uint8).reshape(shape[:-1] + (shape[-1] * 2,))


def acts(m: int, k: int, seed: int = 0, device="cuda") -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randn((m, k), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)


def q8_0_raw(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2) -> torch.Tensor:
    """(n, k/32*34) uint8 Q8_0 blocks"""
    g = _gen(seed, device)
    nb = k // 32
    d = _uniform_f16_bytes(g, (n, nb, 1), lo, hi, device)                       # (n, nb, 2)
    q = torch.randint(-127, 128, (n, nb, 32), generator=g, device=device, dtype=torch.int8).view(torch.uint8)
    return torch.cat([d, q], dim=-1).reshape(n, nb * 34)


def q4_k_raw(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2) -> torch.Tensor:
    """(n, k/256*144) uint8 Q4_K super-blocks"""
    g = _gen(seed, device)
    nb = k // 256
    d = _uniform_f16_bytes(g, (n, nb, 1), lo, hi, device)
    dmin = _uniform_f16_bytes(g, (n, nb, 1), lo, hi, device)
    sc = torch.randint(0, 64, (n, nb, 8), generator=g, device=device, dtype=torch.int32)
    mn = torch.randint(0, 64, (n, nb, 8), generator=g, device=device, dtype=torch.int32)
    s = torch.empty((n, nb, 12), dtype=torch.int32, device=device)
    s[..., 0:4] = (sc[..., 0:4] & 0x3F) | ((sc[..., 4:8] >> 4) << 6)
    s[..., 4:8] = (mn[..., 0:4] & 0x3F) | ((mn[..., 4:8] >> 4) << 6)
    s[..., 8:12] = (sc[..., 4:8] & 0x0F) | ((mn[..., 4:8] & 0x0F) << 4)
    q = torch.randint(0, 16, (n, nb, 4, 2, 32), generator=g, device=device, dtype=torch.int32)
    qs = (q[:, :, :, 0, :] | (q[:, :, :, 1, :] << 4)).reshape(n, nb, 128)
    return torch.cat([d, dmin, s.to(torch.uint8), qs.to(torch.uint8)], dim=-1).reshape(n, nb * 144)


def int8_weights(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2):
    g = _gen(seed, device)
    q = torch.randint(-127, 128, (n, k), generator=g, device=device, dtype=torch.int8)
    s = torch.rand((n,), generator=g, device=device, dtype=torch.float32) * (hi - lo) + lo
    return q, s


# (ggml type or "int8", activation rows M, [(name, N, K), ...])
LAYER_27B = [("q", 6144, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 6144),
             ("gate", 17408, 5120), ("up", 17408, 5120), ("down", 5120, 17408)]
CONFIGS = {
    1: ("int8", 1, [("w", 4096, 4096)]),
    2: (8, 1, [("w", 17408, 5120)]),
    3: (12, 1, [("w", 5120, 17408)]),
    4: ("int8", 64, LAYER_27B),
    5: (12, 2048, LAYER_27B),
}
