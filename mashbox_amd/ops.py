"""mashbox's weight-ops boundary for the quantized-linear path, on the MI355X kernel package (mashbox_amd.kernels).

The caller side of the kernel-package surface, restated on PyTorch-ROCm so that the fast path and its fallback rules run
end to end on one MI355X (reference src/mashbox/ops/__init__.py; names, arguments and error behaviour follow it):

    load_kernels(log=None, module=None) -> types     import the kernel package (env MASHBOX_GGUF_KERNELS; "off" = none)
                                                      (reference :273-311)
    weight_path(t, shape, kernel_types=None)         "kq" | "exact" (:342-363)
    device_nbytes(t, shape, nbytes, kernel_types)    device bytes of one tensor on its path (:366-379)
    prepare(raw, t, shape, use_kernel=True)          Packed (kernel planes) | Raw (the file's blocks) (:412-467): the
                                                      first weight of each (type, shape) runs the kernel once on one row
                                                      (the preflight, :488-495); a failing repack or preflight sends that
                                                      weight and every later one of its (type, shape) to the exact path,
                                                      with one warning
    qmatmul(x, h) -> x @ W.T in x's dtype            float32 accumulation (:594-632); Packed, At (a layer of a stack read
                                                      in place) and Raw handles
    dequant(h), take_rows(h, ids)                    float32 weights / rows, exact (:513-548)
    contract_check(t, raw, shape) -> (ok, bad)       dequant(repack(raw)) == reference dequant(raw), bit for bit (:691-705)
    kernel_picks_layer(), scan_split(ws), scan_join  layer stacks held whole and read in place by the kernel (:635-688)

The exact path stays on the GPU: the file's blocks are rebuilt to float32 by libmbq's raw dequant (bit for bit the
reference dequantization), exact_chunk_rows rows at a time (at most 2**24 values, reference :555-571), and multiplied by
a float32 GEMM, as the reference rebuilds float32 weights and runs a float32 HIGHEST dot. Nothing here runs on the host's
CPU; without libmbq.so every call raises.

The fast paths' forced-failure switch is the reference's: MASHBOX_FAULT=force:kernels-package (the package does not
load) and force:quant-kernel (the kq repack fails), reference src/mashbox/runtime/faults.py:14-16,57-61.
"""
from __future__ import annotations

import ctypes
import importlib
import inspect
import os
import sys

import numpy as np
import torch

from . import _lib

KERNEL_MODULE = "mashbox_amd.kernels"
EXACT_CHUNK = 1 << 24                 # float32 values the exact path rebuilds per step (reference ops/__init__.py:555)
PREFLIGHT_DTYPE = torch.bfloat16      # the preflight's input dtype: the forward's activation dtype
FORCE = ("kernels-package", "quant-kernel")

# ggml type id -> (name, values per block, bytes per block) of the types this path reads (reference ops/reference.py:22-29)
TYPES = {2: ("Q4_0", 32, 18), 8: ("Q8_0", 32, 34), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210)}

_KERNELS = {"module": None, "types": frozenset(), "name": None, "error": None}
_KQ_RAN: dict = {}       # (type, shape) -> True when the kq preflight ran, else why it failed
_KQ_LAYER: dict = {}     # (type, shape) -> True when the layer= preflight ran on a stack, else why it failed


def warn(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def forced(name: str) -> bool:
    """True when MASHBOX_FAULT holds force:<name> (the fallback tests' switch)"""
    if name not in FORCE:
        raise ValueError(f"forced: unknown force name {name!r} (one of {FORCE})")
    parts = [p.strip() for p in os.environ.get("MASHBOX_FAULT", "").split(",")]
    return f"force:{name}" in parts


def type_name(t: int) -> str:
    return TYPES[t][0] if t in TYPES else f"type {t}"


def row_bytes(t: int, cols: int) -> int:
    _, bs, ts = TYPES[t]
    if cols % bs:
        raise ValueError(f"{type_name(t)}: a row of {cols} values is not a multiple of the block size {bs}")
    return cols // bs * ts


def exact_chunk_rows(rows: int, cols: int, limit: int | None = None) -> int:
    """rows per rebuild step of the exact path: the largest divisor of rows with rows * cols <= limit (all rows when the
    weight is that small; 1 row when one row is already over it). Reference src/mashbox/ops/__init__.py:558-571."""
    limit = EXACT_CHUNK if limit is None else limit
    if rows * cols <= limit:
        return rows
    best = 1
    for d in range(1, int(rows ** 0.5) + 1):
        if rows % d == 0:
            for c in (d, rows // d):
                if c * cols <= limit and c > best:
                    best = c
    return best


# --------------------------------------------------------------------------------------------------------- handles
class Raw:
    """Exact-path handle: the file's blocks as stored, (..., rows, row_bytes) uint8 on the GPU, plus type and shape"""

    def __init__(self, raw: torch.Tensor, t: int, shape):
        self.raw, self.t, self.shape = raw, int(t), tuple(int(s) for s in shape)

    def __repr__(self):
        return f"Raw({type_name(self.t)}, {self.shape})"


class Packed:
    """Kernel handle: the kernel package's planes (opaque here), plus type and logical shape"""

    def __init__(self, packed, t: int, shape):
        self.packed, self.t, self.shape = packed, int(t), tuple(int(s) for s in shape)

    def __repr__(self):
        return f"Packed({type_name(self.t)}, {self.shape})"


class At:
    """One layer of a Packed layer stack, for a kernel that reads the layer in place (matmul's layer=)"""

    def __init__(self, packed, layer, t: int, shape):
        self.packed, self.layer, self.t, self.shape = packed, layer, int(t), tuple(int(s) for s in shape)

    def __repr__(self):
        return f"At({type_name(self.t)}, {self.shape})"


def route(h) -> str:
    """'kernel' for kernel planes, else 'reference' (the exact path rebuilds the weights at every call)"""
    return "kernel" if isinstance(h, (Packed, At)) else "reference"


# --------------------------------------------------------------------------------------------------- the package
def load_kernels(log=None, module=None) -> frozenset:
    """Import the kernel package (env MASHBOX_GGUF_KERNELS names another module; "off" disables) -> the ggml types its kq
    planes run. An import failure leaves TYPES empty: every weight runs on the exact path. Starts the preflights over."""
    module = module or os.environ.get("MASHBOX_GGUF_KERNELS", KERNEL_MODULE)
    _KERNELS.update(module=None, types=frozenset(), name=None, error=None)
    _KQ_RAN.clear()
    _KQ_LAYER.clear()
    if module in ("", "off", "none"):
        return _KERNELS["types"]
    try:
        if forced("kernels-package"):
            raise RuntimeError("MASHBOX_FAULT=force:kernels-package")
        m = importlib.import_module(module)
        _KERNELS.update(module=m, types=frozenset(int(t) for t in getattr(m, "TYPES", ())), name=module)
    except Exception as e:                       # a broken package must not stop the exact path
        _KERNELS["error"] = f"{type(e).__name__}: {e}"
        if log:
            log(f"mashbox: kernel package {module} did not load ({_KERNELS['error']}); every type runs on the exact path")
    return _KERNELS["types"]


def kernel_types() -> frozenset:
    return _KERNELS["types"]


def _kq_covers(t: int, shape) -> bool:
    f = getattr(_KERNELS["module"], "kq_covers", None)
    return f is None or len(tuple(shape)) < 2 or bool(f(int(t), tuple(int(v) for v in tuple(shape)[-2:])))


def weight_path(t: int, shape=(), kernel_types=None) -> str:
    """-> "kq" | "exact": the path a weight of ggml type t and shape (rows, cols) takes (kernel_types limits the kernel
    types; frozenset() = the exact path for everything)"""
    t = int(t)
    allowed = _KERNELS["types"] if kernel_types is None else frozenset(int(v) for v in kernel_types)
    return "kq" if t in allowed and t in _KERNELS["types"] and _kq_covers(t, shape) else "exact"


def device_nbytes(t: int, shape, nbytes: int, kernel_types=None) -> int:
    """device bytes of one tensor (..., rows, cols) whose file blocks take nbytes, on its path: the kq planes (once per
    matrix of a stack) or the blocks as stored"""
    mod = _KERNELS["module"]
    if weight_path(t, shape, kernel_types) == "kq" and hasattr(mod, "plane_bytes"):
        lead = 1
        for v in tuple(shape)[:-2]:
            lead *= int(v)
        return lead * int(mod.plane_bytes(int(t), tuple(int(v) for v in tuple(shape)[-2:])))
    return int(nbytes)


def kernel_picks_layer() -> bool:
    mod = _KERNELS["module"]
    if getattr(mod, "picks_layer", None) is not None:
        return bool(mod.picks_layer)
    mm = getattr(mod, "matmul", None)
    try:
        return mm is not None and "layer" in inspect.signature(mm).parameters
    except (TypeError, ValueError):
        return False


# ---------------------------------------------------------------------------------------------------- prepare
def _device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def prepare(raw, t: int, shape, use_kernel: bool = True):
    """raw: host (NumPy) or device (torch) uint8 (rows, row_bytes), or with leading axes (a stack of same-shape tensors);
    shape is one tensor's (rows, cols) -> Packed or Raw handle on the GPU. On kq, the first weight of each (type, shape)
    also runs the kernel once (the preflight); if the repack or the preflight raises, this weight and every later one of
    that type and shape load on the exact path, with one warning naming the type, the shape and the error."""
    t = int(t)
    if t not in TYPES:
        raise NotImplementedError(f"ggml type {t} has no reader on this path (types {sorted(TYPES)})")
    path = weight_path(t, shape, None if use_kernel else frozenset())
    key = (t, tuple(int(s) for s in shape))
    if path == "kq" and _KQ_RAN.get(key, True) is True:
        try:
            h = _kq_planes(raw, t, shape)
            lead = len(tuple(raw.shape)) - 2
            if key not in _KQ_RAN:
                _kq_preflight(h, lead)
                _KQ_RAN[key] = True
            if lead == 1 and len(key[1]) == 2 and key not in _KQ_LAYER and kernel_picks_layer():
                _kq_layer_preflight(h, key)
            return h
        except Exception as e:                   # a fast path must never stop the load: fall back, loudly
            _KQ_RAN[key] = f"{type(e).__name__}: {e}"
            warn(f"mashbox: kq planes for {type_name(t)} {key[1]} failed ({_KQ_RAN[key]}); weights of this type and "
                 f"shape run on the exact path")
    dev = _device()
    r = raw if isinstance(raw, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(raw, np.uint8)))
    return Raw(r.to(dev).contiguous(), t, shape)


def _kq_planes(raw, t: int, shape) -> Packed:
    mod = _KERNELS["module"]
    if forced("quant-kernel"):
        raise RuntimeError("forced by MASHBOX_FAULT=force:quant-kernel")
    if not isinstance(raw, torch.Tensor) and hasattr(mod, "repack_host"):
        return Packed(mod.repack_host(t, np.asarray(raw), tuple(shape)).to(_device()), t, shape)
    r = raw if isinstance(raw, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(raw, np.uint8)))
    return Packed(mod.repack(t, r.to(_device()), tuple(shape), stacked=r.dim() > 2), t, shape)


def _kq_preflight(h: Packed, lead: int) -> None:
    """the kernel once on one tensor of h (index 0 of each stacked axis) with one row of input in the forward's dtype;
    it waits for the result, so a kernel that fails while it runs raises here"""
    planes = h.packed
    for _ in range(lead):
        planes = planes[0]
    x = torch.ones((1, h.shape[-1]), dtype=PREFLIGHT_DTYPE, device=_device())
    _KERNELS["module"].matmul(x, planes)
    torch.cuda.synchronize()


def _kq_layer_preflight(h: Packed, key) -> None:
    """matmul with layer= on a whole layer stack, once per (type, shape), with a device layer index; if it raises,
    stacks of this type and shape are sliced per layer instead (scan_split), with one warning"""
    try:
        x = torch.ones((1, h.shape[-1]), dtype=PREFLIGHT_DTYPE, device=_device())
        _KERNELS["module"].matmul(x, h.packed, layer=torch.zeros((), dtype=torch.int32, device=_device()))
        torch.cuda.synchronize()
        _KQ_LAYER[key] = True
    except Exception as e:
        _KQ_LAYER[key] = f"{type(e).__name__}: {e}"
        warn(f"mashbox: kq layer= for {type_name(key[0])} {key[1]} failed ({_KQ_LAYER[key]}); stacks of this type and "
             f"shape are sliced per layer before the kernel")


# ---------------------------------------------------------------------------------------------------- the exact path
def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _raw_dequant(raw2: torch.Tensor, t: int, rows: int, cols: int) -> torch.Tensor:
    """(rows, row_bytes) uint8 on the GPU -> float32 (rows, cols), bit for bit the reference dequantization"""
    w = torch.empty((rows, cols), dtype=torch.float32, device=raw2.device)
    _lib.check(_lib.lib().mbq_dequant_raw(int(t), ctypes.c_void_p(raw2.data_ptr()), rows, cols,
                                          ctypes.c_void_p(w.data_ptr()), _stream()), "dequant_raw")
    return w


def _mat(h: Raw) -> torch.Tensor:
    rows, cols = h.shape[-2], h.shape[-1]
    return h.raw.reshape(tuple(h.raw.shape[:-2]) + (rows, row_bytes(h.t, cols))) if h.raw.dim() >= 2 else \
        h.raw.reshape(rows, row_bytes(h.t, cols))


def _exact(x: torch.Tensor, h: Raw) -> torch.Tensor:
    """x (..., cols) @ W.T in float32: the weights rebuilt a chunk of exact_chunk_rows rows at a time (reference
    ops/__init__.py:574-576, 624-632)"""
    rows, cols = h.shape[-2], h.shape[-1]
    raw2 = _mat(h).reshape(rows, -1).contiguous()
    x32 = x.to(device=raw2.device, dtype=torch.float32)
    rc = exact_chunk_rows(rows, cols)
    out = torch.empty(tuple(x.shape[:-1]) + (rows,), dtype=torch.float32, device=raw2.device)
    for a in range(0, rows, rc):
        w = _raw_dequant(raw2[a:a + rc], h.t, rc, cols)
        out[..., a:a + rc] = torch.matmul(x32, w.t())
    return out


def qmatmul(x: torch.Tensor, h) -> torch.Tensor:
    """x (..., cols) @ W.T -> (..., rows): float32 accumulation, result in x's dtype (reference ops/__init__.py:594-632)"""
    if isinstance(h, Packed):
        return _KERNELS["module"].matmul(x, h.packed).to(x.dtype)
    if isinstance(h, At):
        return _KERNELS["module"].matmul(x, h.packed, layer=h.layer).to(x.dtype)
    if isinstance(h, Raw):
        if h.raw.dim() > 2:
            raise ValueError(f"{h}: a stack is multiplied one layer at a time (index the stack)")
        return _exact(x, h).to(x.dtype)
    raise TypeError(f"qmatmul: not a weight handle: {h!r}")


def dequant(h) -> torch.Tensor:
    """handle -> float32 weights (..., rows, cols), exact"""
    if isinstance(h, Packed):
        return _KERNELS["module"].dequant(h.packed)
    if isinstance(h, At):
        return _KERNELS["module"].dequant(h.packed, layer=h.layer)
    rows, cols = h.shape[-2], h.shape[-1]
    m = _mat(h)
    lead = tuple(m.shape[:-2])
    flat = m.reshape(-1, row_bytes(h.t, cols)).contiguous()
    return _raw_dequant(flat, h.t, flat.shape[0], cols).reshape(lead + (rows, cols))


def take_rows(h, ids) -> torch.Tensor:
    """rows `ids` of the weights as float32 (embedding lookup), exact; a negative id counts from the end"""
    rows = h.shape[-2]
    ids = torch.as_tensor(ids, device=_device()).long()
    ids = torch.where(ids < 0, ids + rows, ids)
    if isinstance(h, Raw):
        m = _mat(h).reshape(rows, -1)
        sel = m[ids.reshape(-1)].contiguous()
        w = _raw_dequant(sel, h.t, sel.shape[0], h.shape[-1])
        return w.reshape(tuple(ids.shape) + (h.shape[-1],))
    return dequant(h)[ids]


def contract_check(t: int, raw, shape):
    """dequant(repack(raw)) == the reference dequantization (the device raw dequant), bit for bit -> (ok, mismatching
    values); None when the kernel package does not cover type t. NaN must be NaN bit for bit (uint32 compare)."""
    mod = _KERNELS["module"]
    if int(t) not in _KERNELS["types"]:
        return None
    r = raw if isinstance(raw, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(raw, np.uint8)))
    r = r.to(_device()).contiguous()
    rows, cols = int(shape[-2]), int(shape[-1])
    ref = _raw_dequant(r.reshape(rows, -1), int(t), rows, cols)
    got = mod.dequant(mod.repack(int(t), r, tuple(shape))).reshape(rows, cols)
    bad = int((ref.view(torch.int32) != got.view(torch.int32)).sum().item())
    return bad == 0, bad


# ------------------------------------------------------------------------------------------------ layer stacks
def _held(v) -> bool:
    """a Packed stack of one (rows, cols) weight per layer whose (type, shape) passed the layer= preflight"""
    return isinstance(v, Packed) and len(v.shape) == 2 and _KQ_LAYER.get((v.t, v.shape)) is True


def _tree_map(f, tree):
    if isinstance(tree, dict):
        return {k: _tree_map(f, v) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        return type(tree)(_tree_map(f, v) for v in tree)
    return f(tree)


def scan_split(ws):
    """a tree of weights stacked over layers -> (held, xs): when the kernel reads a layer in place, each Packed stack that
    passed the layer= preflight is held whole (xs has None there) and the loop body multiplies by it at its layer
    (scan_join); other leaves are sliced per layer as before. With nothing held: (None, ws)."""
    picks = kernel_picks_layer()
    hits = []
    _tree_map(lambda v: hits.append(picks and _held(v)), ws)
    if not any(hits):
        return None, ws
    return (_tree_map(lambda v: v if picks and _held(v) else None, ws),
            _tree_map(lambda v: None if picks and _held(v) else v, ws))


def scan_join(held, w, layer):
    """inside the loop body: the layer's weights = w with each held stack as At(stack, layer)"""
    if held is None:
        return w
    if isinstance(held, dict):
        return {k: scan_join(held[k], w[k] if w is not None else None, layer) for k in held}
    if isinstance(held, (list, tuple)):
        return type(held)(scan_join(h, w[i] if w is not None else None, layer) for i, h in enumerate(held))
    if isinstance(held, Packed):
        return At(held.packed, layer, held.t, held.shape)
    return w


def slice_layer(h, i: int):
    """layer i of a stacked handle (what a scan slice gives)"""
    if isinstance(h, Packed):
        return Packed(h.packed[i], h.t, h.shape)
    if isinstance(h, Raw):
        return Raw(h.raw[i], h.t, h.shape)
    raise TypeError(f"slice_layer: {h!r}")
