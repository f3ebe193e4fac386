"""Seeded synthetic GGUF / int8 weights and bf16 activations, generated on the GPU (for the bench's large workloads).

Value ranges are those of the five BASELINE configs: fp16 block scales d (and Q4_K dmin) ~ U(1e-3, 1e-2), Q8_0 / int8
quants uniform in [-127, 127], Q4_K six-bit scales and mins uniform in [0, 63] packed as the Q4_K scale bytes hold
them (reference src/mashbox/ops/reference.py:132-139), four-bit quants uniform in [0, 15], int8 per-row scales
~ U(1e-3, 1e-2), activations ~ N(0, 1) rounded to bfloat16; Q6_K (the reference's Q6_K output-head shape, not a
BASELINE config): d ~ U(1e-3, 1e-2) / 64, int8 sub-block scales uniform in [-127, 127], six-bit quants uniform in
[0, 63]; Q4_0: d ~ U(1e-3, 1e-2), four-bit quants uniform in [0, 15]. The bytes are the file's block layout (Q4_0
18 B and Q8_0 34 B per 32 values, Q4_K 144 B and Q6_K 210 B per 256), ready for repack.
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


def q4_0_raw(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2) -> torch.Tensor:
    """(n, k/32*18) uint8 Q4_0 blocks: d, then value i in the low nibble of byte i, value 16 + i in its high nibble
    (reference src/mashbox/ops/reference.py:66-70)"""
    g = _gen(seed, device)
    nb = k // 32
    d = _uniform_f16_bytes(g, (n, nb, 1), lo, hi, device)
    q = torch.randint(0, 16, (n, nb, 2, 16), generator=g, device=device, dtype=torch.int32)
    qs = (q[:, :, 0] | (q[:, :, 1] << 4)).to(torch.uint8)
    return torch.cat([d, qs], dim=-1).reshape(n, nb * 18)


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


def q5_k_raw(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2) -> torch.Tensor:
    """(n, k/256*176) uint8 Q5_K super-blocks: the Q4_K header (d, dmin, 12 packed 6-bit scales and mins), 32 bytes of
    high bits, 128 bytes of low nibbles, both uniform random bytes (5-bit quants uniform in [0, 31])"""
    g = _gen(seed, device)
    nb = k // 256
    head = q4_k_raw(n, k, seed=seed, device=device, lo=lo, hi=hi).reshape(n, nb, 144)[:, :, :16]
    bits = torch.randint(0, 256, (n, nb, 160), generator=g, device=device, dtype=torch.int32).to(torch.uint8)
    return torch.cat([head, bits], dim=-1).reshape(n, nb * 176)


def q6_k_raw(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2) -> torch.Tensor:
    """(n, k/256*210) uint8 Q6_K super-blocks: ql (low nibbles), qh (2-bit highs), 16 int8 scales, fp16 d
    (reference src/mashbox/ops/reference.py:164-173: value 128g + 32r + i takes nibble r // 2 of ql[64g + 32 (r % 2) + i]
    and bits 2r, 2r + 1 of qh[32g + i])"""
    g = _gen(seed, device)
    nb = k // 256
    q = torch.randint(0, 64, (n, nb, 2, 4, 32), generator=g, device=device, dtype=torch.int32)
    ql = torch.cat([(q[:, :, :, j] & 15) | ((q[:, :, :, 2 + j] & 15) << 4) for j in range(2)], dim=-1)   # (n, nb, 2, 64)
    qh = sum((q[:, :, :, r] >> 4) << (2 * r) for r in range(4))                                         # (n, nb, 2, 32)
    del q
    sc = torch.randint(-127, 128, (n, nb, 16), generator=g, device=device, dtype=torch.int8).view(torch.uint8)
    d = _uniform_f16_bytes(g, (n, nb, 1), lo / 64, hi / 64, device)
    return torch.cat([ql.reshape(n, nb, 128).to(torch.uint8), qh.reshape(n, nb, 64).to(torch.uint8), sc, d],
                     dim=-1).reshape(n, nb * 210)


def q2_k_raw(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2) -> torch.Tensor:
    """(n, k/256*84) uint8 Q2_K super-blocks: 16 scale bytes (4-bit scale, 4-bit min, each uniform in [0, 15]), 64 bytes
    of 2-bit quants (uniform bytes), fp16 d and dmin ~ U(lo, hi) (reference src/mashbox/ops/reference.py:106-114)"""
    g = _gen(seed, device)
    nb = k // 256
    body = torch.randint(0, 256, (n, nb, 80), generator=g, device=device, dtype=torch.int32).to(torch.uint8)
    d = _uniform_f16_bytes(g, (n, nb, 1), lo, hi, device)
    dmin = _uniform_f16_bytes(g, (n, nb, 1), lo, hi, device)
    return torch.cat([body, d, dmin], dim=-1).reshape(n, nb * 84)


def int8_weights(n: int, k: int, seed: int = 0, device="cuda", lo=1e-3, hi=1e-2):
    g = _gen(seed, device)
    q = torch.randint(-127, 128, (n, k), generator=g, device=device, dtype=torch.int8)
    s = torch.rand((n,), generator=g, device=device, dtype=torch.float32) * (hi - lo) + lo
    return q, s


# (ggml type or "int8", activation rows M, [(name, N, K), ...])
LAYER_27B = [("q", 6144, 5120), ("k", 1024, 5120), ("v", 1024, 5120), ("o", 5120, 6144),
             ("gate", 17408, 5120), ("up", 17408, 5120), ("down", 5120, 17408)]
# the layer with q, k, v stacked by rows into one weight and gate, up into another (they share their input)
LAYER_27B_STACKED = [("qkv", 8192, 5120), ("o", 5120, 6144), ("gate_up", 34816, 5120), ("down", 5120, 17408)]
CONFIGS = {
    1: ("int8", 1, [("w", 4096, 4096)]),
    2: (8, 1, [("w", 17408, 5120)]),
    3: (12, 1, [("w", 5120, 17408)]),
    4: ("int8", 64, LAYER_27B),
    5: (12, 2048, LAYER_27B),
}
# the reference's largest published per-call number: a Q6_K output head, 151936 x 2560, one activation row
# (reference CORE-CHANGES.md:73, 369.8 us on TPU v6e-1); the 9728 x 2560 rows below: CORE-CHANGES.md:84
# batched decode over one 27B-class layer at the reference engine's row buckets 4 and 16 (runtime/engine.py:424-428):
# Q4_K, Q8_0, Q5_K, Q6_K and int8 weights, each repacked into 16-row tiles (as config 4 takes int8)
EXTRA = {"q6k_head": (14, 1, [("w", 151936, 2560)]),
         "m4_q4k": (12, 4, LAYER_27B), "m16_q4k": (12, 16, LAYER_27B), "m4_q8": (8, 4, LAYER_27B), "m16_q8": (8, 16, LAYER_27B),
         "m4_q5k": (13, 4, LAYER_27B), "m16_q5k": (13, 16, LAYER_27B),
         "m4_q6k": (14, 4, LAYER_27B), "m16_q6k": (14, 16, LAYER_27B),
         "m4_int8": ("int8", 4, LAYER_27B), "m16_int8": ("int8", 16, LAYER_27B),
         # single-row decode of the same layer: row-major planes (decode GEMV) and the same weights as 16-row tiles
         "m1_q4k": (12, 1, LAYER_27B), "m1_q4k_tiles": (12, 1, LAYER_27B),
         # config 5's prefill on the row-major planes (config 5 itself loads the weights as 16-row tiles)
         "c5_rm": (12, 2048, LAYER_27B),
         # the same layer with the projections that share an input stacked by rows at load (ops.stack_rows): q|k|v and
         # gate|up, four launches instead of seven (Q4_K as 16-row tiles, ops.prepare's default; int8 as config 4)
         "m1_q4k_stacked": (12, 1, LAYER_27B_STACKED), "m4_q4k_stacked": (12, 4, LAYER_27B_STACKED),
         "m16_q4k_stacked": (12, 16, LAYER_27B_STACKED), "c4_stacked": ("int8", 64, LAYER_27B_STACKED),
         # a prefill chunk of the reference engine's default size (runtime/engine.py:168: chunk=512), Q4_K tiles
         "p512_q4k": (12, 512, LAYER_27B),
         # the reference's other published per-call numbers (CORE-CHANGES.md:84, kernel package 0.1.13, one row):
         # Q4_K 9728 x 2560 on the kernels (row-major planes, the decode GEMV) and Q2_K 9728 x 2560, a type without
         # kernel planes here, on the exact path's fused product (mbq_matmul_raw over the file's blocks)
         "q4k_9728": (12, 1, [("w", 9728, 2560)]), "q2k_9728": (10, 1, [("w", 9728, 2560)])}
REF_TPU_US = {"q6k_head": 369.8, "q4k_9728": 22.6, "q2k_9728": 25.5}
