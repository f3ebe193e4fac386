"""ctypes binding of libmbq.so (C ABI: include/mbq.h). Loading fails loudly: there is no fallback path here."""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("MBQ_LIB", os.path.join(HERE, "libmbq.so"))

Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, INT8, I8T = 2, 8, 12, 13, 14, -8, -9
Q8T, Q40T, Q4KT, Q5KT, Q6KT = -10, -11, -12, -13, -14   # the GGUF types' planes in 16-row tiles (MBQ_Q8T, ...)
OUT_F32, OUT_BF16 = 0, 1

# every symbol include/mbq.h declares, with its ctypes signature
_c = ctypes
_SIGS = {
    "mbq_version": (_c.c_int, []),
    "mbq_last_error": (_c.c_char_p, []),
    "mbq_has_type": (_c.c_int, [_c.c_int]),
    "mbq_has_raw_type": (_c.c_int, [_c.c_int]),
    "mbq_row_bytes": (_c.c_int64, [_c.c_int, _c.c_int64]),
    "mbq_covers": (_c.c_int, [_c.c_int, _c.c_int64, _c.c_int64]),
    "mbq_plane_bytes": (_c.c_int64, [_c.c_int, _c.c_int64, _c.c_int64]),
    "mbq_repack_host": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_size_t, _c.c_int]),
    "mbq_unpack_host": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_size_t]),
    "mbq_repack_dev": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_void_p]),
    "mbq_matmul": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int64,
                              _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_int, _c.c_void_p]),
    "mbq_matmul_noalloc": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int64,
                                      _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_int, _c.c_void_p]),
    "mbq_dequant": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                               _c.c_void_p, _c.c_void_p]),
    "mbq_dequant_rows": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                                    _c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_void_p]),
    "mbq_dequant_raw": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_void_p]),
    "mbq_matmul_raw": (_c.c_int, [_c.c_int, _c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_int,
                                  _c.c_void_p]),
    "mbq_int8_embed": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_int64, _c.c_void_p,
                                  _c.c_int, _c.c_void_p]),
    "mbq_int8_repack_host": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_size_t,
                                        _c.c_int]),
    "mbq_int8_repack_dev": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_void_p]),
    "mbq_int8_unpack_host": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_int64, _c.c_void_p, _c.c_void_p]),
    "mbq_int8_linear": (_c.c_int, [_c.c_void_p, _c.c_void_p, _c.c_void_p, _c.c_int64, _c.c_int64, _c.c_int64,
                                   _c.c_void_p, _c.c_int, _c.c_void_p]),
    "mbq_gemm_plan": (_c.c_int, [_c.c_int, _c.c_int64, _c.c_int64, _c.c_int64, _c.POINTER(_c.c_int),
                                 _c.POINTER(_c.c_int), _c.POINTER(_c.c_int), _c.POINTER(_c.c_int)]),
    "mbq_force_gemm_plan": (_c.c_int, [_c.c_int, _c.c_int, _c.c_int, _c.c_int]),
    "mbq_probe_read": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_void_p]),
    "mbq_probe_mfma": (_c.c_int, [_c.c_int, _c.c_void_p, _c.POINTER(_c.c_int64), _c.c_void_p]),
    "mbq_probe_bf16": (_c.c_int, [_c.c_void_p, _c.c_void_p]),
}


# GEMM kernels of gemm_plan / force_gemm_plan (MBQ_KERNEL_* of include/mbq.h)
KERNEL_AUTO = KERNEL_GEMV = 0
KERNEL_STREAM, KERNEL_TILES, KERNEL_KGROUP = 1, 2, 3
KERNEL_NAMES = {KERNEL_GEMV: "gemv", KERNEL_STREAM: "stream", KERNEL_TILES: "tiles", KERNEL_KGROUP: "kgroup"}


def gemm_plan(t: int, m: int, n: int, k: int):
    """-> (kernel, tile rows, tile cols, K splits) the library would use; (0, 0, 0, 0) = decode GEMV"""
    kn, bm, bn, sp = _c.c_int(), _c.c_int(), _c.c_int(), _c.c_int()
    check(lib().mbq_gemm_plan(int(t), int(m), int(n), int(k), _c.byref(kn), _c.byref(bm), _c.byref(bn), _c.byref(sp)),
          "gemm_plan")
    return kn.value, bm.value, bn.value, sp.value


def force_gemm_plan(kernel: int = KERNEL_AUTO, bm: int = 0, bn: int = 0, splits: int = 0):
    """force every later GEMM (M > 4) of the process to one kernel, bm x bn tiles and `splits` K ranges;
    force_gemm_plan() = automatic"""
    check(lib().mbq_force_gemm_plan(int(kernel), int(bm), int(bn), int(splits)), "force_gemm_plan")


def plan_str(t: int, m: int, n: int, k: int) -> str:
    """the plan as text, e.g. 'tiles 256x192/1'"""
    kn, bm, bn, sp = gemm_plan(t, m, n, k)
    return "gemv" if kn == KERNEL_GEMV else f"{KERNEL_NAMES[kn]} {bm}x{bn}/{sp}"

_lock = threading.Lock()
_lib = None


class MbqError(RuntimeError):
    """a libmbq.so entry point returned an error code"""


def lib() -> ctypes.CDLL:
    """the loaded libmbq.so; raises OSError when it is missing (build it with mashbox_amd.build)"""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise OSError(f"{LIB_PATH} is missing: build it with `python -m mashbox_amd.build`")
                L = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in _SIGS.items():
                    f = getattr(L, name)
                    f.restype, f.argtypes = res, args
                _lib = L
    return _lib


def check(rc: int, what: str) -> int:
    if rc < 0:
        msg = lib().mbq_last_error().decode(errors="replace")
        raise MbqError(f"{what}: {msg} (code {rc})")
    return rc
