"""mashbox's weight-ops boundary for the quantized-linear path, on PyTorch-ROCm and the MI355X kernel package.

This is the caller side of the kernel-package surface (reference src/mashbox/ops/__init__.py), built around torch and
libmbq's C ABI. The names, arguments, fallback rules and warning texts are the reference's interface, so that its
loaders and tests drive this module unchanged:

    load_kernels(log=None, module=None) -> types     import the kernel package named by env MASHBOX_GGUF_KERNELS
                                                      ("off" = none; reference :273-311)
    weight_path(t, shape, kernel_types=None)         "kq" | "exact" (:342-363)
    device_nbytes(t, shape, nbytes, kernel_types)    device bytes of one tensor on its path (:366-379)
    prepare(raw, t, shape, use_kernel=True)          Packed (kernel planes) | Raw (the file's blocks) (:412-467)
    stack_mixed(layers, shape)                       one role whose block types differ by layer -> Mixed (the callers'
                                                      construction, reference gguf/archs/dense.py:206-218)
    stack_rows(parts) -> (raw, t, sizes)             weights that share an input stacked by rows into one weight (one
                                                      launch per call; reference model.py:374 keeps q, k, v this way)
    qmatmul(x, h) -> x @ W.T in x's dtype            float32 accumulation (:594-632)
    dequant(h), take_rows(h, ids)                    float32 weights / rows, exact (:513-548)
    contract_check(t, raw, shape) -> (ok, bad)       dequant(repack(raw)) == reference dequant(raw) (:691-705)
    kernel_picks_layer(), scan_split, scan_join      stacks held whole and read in place by the kernel (:635-688)

Handles: Raw (the file's blocks), Packed (kernel planes, one weight or a stack), At (one layer of a held stack),
Mixed (per-type stacks of one role with per-layer `which` / `sub`) and Pick (one layer of a Mixed inside the layer
loop). A Pick whose index lives on the device is dispatched without a host sync: each type's kernel reads its stack at
`sub` where `which` selects that type (anywhere else the index lies outside the stack: the kernel reads nothing and
writes NaN) and the result is selected on the device.

The first weight of each (type, shape) on the kernel path runs the kernel once on one row (the preflight); if the
repack or the preflight raises, that weight and every later one of its (type, shape) load on the exact path, with one
warning. The exact path stays on the GPU: the file's blocks are rebuilt to float32 by libmbq's raw dequant (bit for bit
the reference dequantization), exact_chunk_rows rows at a time, and multiplied by a float32 GEMM. Nothing here computes
on the host's CPU; without libmbq.so every call raises. The forced-failure switch is the reference's MASHBOX_FAULT
(force:kernels-package, force:quant-kernel; reference src/mashbox/runtime/faults.py:14-16,57-61).

Weight layout (no counterpart in the reference, whose kernel package has one): weights of the types the kernel package
can tile (its TILED map: every GGUF type it serves) load as its 16-row tiles, the layout its K-group kernel runs at
2-64 activation rows, its tile GEMV at one row, and its prefill GEMM runs fastest on (MI355X, a 27B-class Q4_K layer:
4 rows 87 us against 122 us on row-major planes, 16 rows 98 against 137, 2048 rows 1339 against 1398); at one row the
row-major planes' decode GEMV is still a little faster (64-67 against 68-74 us). Env MBQ_LAYOUT picks another:
"rowmajor", or "both" (the tiles plus the row-major planes of the same weights, twice the bytes: every batch size gets
its faster kernel).
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

# the ggml types this path reads: id -> (name, values per block, bytes per block) (reference ops/reference.py:22-29).
# The kernel package gives planes to the first five; every type here runs on the exact path (mbq_dequant_raw). The
# reference's seven other types (IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M) decode through code books that
# gguf-py ships (reference ops/reference.py:243-252); this build does not carry them.
TYPES = {2: ("Q4_0", 32, 18), 8: ("Q8_0", 32, 34), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
         0: ("F32", 1, 4), 1: ("F16", 1, 2), 30: ("BF16", 1, 2), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
         7: ("Q5_1", 32, 24), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110), 20: ("IQ4_NL", 32, 18),
         23: ("IQ4_XS", 256, 136), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66), 39: ("MXFP4", 32, 17),
         40: ("NVFP4", 64, 36)}
CODEBOOK_TYPES = {16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S", 21: "IQ3_S", 22: "IQ2_S", 29: "IQ1_M"}


def warn(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def forced(name: str) -> bool:
    """True when env MASHBOX_FAULT (a comma-separated list) holds force:<name>"""
    if name not in FORCE:
        raise ValueError(f"forced: unknown force name {name!r} (one of {FORCE})")
    return f"force:{name}" in {p.strip() for p in os.environ.get("MASHBOX_FAULT", "").split(",")}


def type_name(t: int) -> str:
    return TYPES[t][0] if t in TYPES else f"type {t}"


def row_bytes(t: int, cols: int) -> int:
    name, per_block, block_bytes = TYPES[t]
    blocks, rest = divmod(cols, per_block)
    if rest:
        raise ValueError(f"{name}: a row of {cols} values is not a multiple of the block size {per_block}")
    return blocks * block_bytes


def exact_chunk_rows(rows: int, cols: int, limit: int | None = None) -> int:
    """rows per rebuild step of the exact path: the largest divisor of rows whose rows * cols stay within the limit (all
    rows when the weight fits; 1 when a single row is over it). Reference src/mashbox/ops/__init__.py:558-571."""
    limit = EXACT_CHUNK if limit is None else limit
    fit = limit // cols if cols > 0 else rows
    if rows <= fit:
        return rows
    divisors = set()
    i = 1
    while i * i <= rows:
        if rows % i == 0:
            divisors.update((i, rows // i))
        i += 1
    return max([d for d in divisors if d <= fit], default=1)


# --------------------------------------------------------------------------------------------------------- handles
class _Handle:
    """a weight of ggml type t and logical shape (rows, cols) (a stack: leading axes first)"""
    __slots__ = ("t", "shape")

    def _init(self, t, shape):
        self.t = int(t)
        self.shape = tuple(int(v) for v in shape)

    def __repr__(self):
        return f"{type(self).__name__}({type_name(self.t)}, {self.shape})"


class Raw(_Handle):
    """exact path: the file's blocks as stored, (..., rows, row_bytes) uint8 on the GPU"""
    __slots__ = ("raw",)

    def __init__(self, raw: torch.Tensor, t: int, shape):
        self.raw = raw
        self._init(t, shape)


class Packed(_Handle):
    """kernel path: the kernel package's planes (opaque here) of one weight, or of a stack along leading axes"""
    __slots__ = ("packed",)

    def __init__(self, packed, t: int, shape):
        self.packed = packed
        self._init(t, shape)


class At(_Handle):
    """one layer of a held Packed stack, read in place by the kernel (matmul's layer=): an int or a device int32"""
    __slots__ = ("packed", "layer")

    def __init__(self, packed, layer, t: int, shape):
        self.packed, self.layer = packed, layer
        self._init(t, shape)


class Mixed(_Handle):
    """one role stacked over layers whose block types differ by layer: stacks[i] holds the layers of types[i] in order,
    and per layer which[l] names its stack and sub[l] its index there ((layers,) int32, device or host)"""
    __slots__ = ("stacks", "which", "sub", "types")

    def __init__(self, stacks, which, sub, types, shape):
        self.stacks, self.which, self.sub = tuple(stacks), which, sub
        self.types = tuple(int(t) for t in types)
        self._init(self.types[0], shape)

    def __repr__(self):
        return f"Mixed({', '.join(type_name(t) for t in self.types)}, {self.shape})"


class Pick(Mixed):
    """one layer of a Mixed inside the layer loop: the whole stacks and that layer's which / sub scalars"""
    __slots__ = ()

    def __repr__(self):
        return f"Pick({', '.join(type_name(t) for t in self.types)}, {self.shape})"


def route(h) -> str:
    """'kernel' for kernel planes, else 'reference' (the exact path rebuilds the weights at every call)"""
    return "kernel" if isinstance(h, (Packed, At)) else "reference"


# ----------------------------------------------------------------------------------------------------- the package
class _Package:
    """the loaded kernel package and what the loads learned about it: per (type, shape), True once the preflight ran or
    the reason it failed (preflight), and the same for layer= on a stack (layer_preflight). Item access reads the
    fields the reference's tests read (module, types, name, error)."""

    def __init__(self):
        self.reset()

    def reset(self):
        self.module = None
        self.types = frozenset()
        self.name = None
        self.error = None
        self.preflight = {}
        self.layer_preflight = {}
        self._out_dtype = None

    def __getitem__(self, key):
        if key not in ("module", "types", "name", "error"):
            raise KeyError(key)
        return getattr(self, key)

    def covers(self, t: int, shape) -> bool:
        test = getattr(self.module, "kq_covers", None)
        if test is None or len(tuple(shape)) < 2:
            return True
        return bool(test(int(t), tuple(int(v) for v in tuple(shape)[-2:])))

    def out_dtype(self) -> bool:
        """the package's matmul takes out_dtype= (a result written in the activation dtype by the kernel itself)"""
        if self._out_dtype is None:
            mm = getattr(self.module, "matmul", None)
            try:
                self._out_dtype = mm is not None and "out_dtype" in inspect.signature(mm).parameters
            except (TypeError, ValueError):
                self._out_dtype = False
        return self._out_dtype

    def picks_layer(self) -> bool:
        flag = getattr(self.module, "picks_layer", None)
        if flag is not None:
            return bool(flag)
        mm = getattr(self.module, "matmul", None)
        try:
            return mm is not None and "layer" in inspect.signature(mm).parameters
        except (TypeError, ValueError):
            return False


_KERNELS = _Package()


def kernel_package() -> dict:
    return {"module": _KERNELS.name, "types": sorted(_KERNELS.types), "error": _KERNELS.error}


def load_kernels(log=None, module=None) -> frozenset:
    """import the kernel package (env MASHBOX_GGUF_KERNELS names another module; "off" disables) -> the ggml types its
    planes run. A package that fails to import leaves no types: every weight runs on the exact path. Starts the
    preflights over."""
    module = module or os.environ.get("MASHBOX_GGUF_KERNELS", KERNEL_MODULE)
    _KERNELS.reset()
    if module in ("", "off", "none"):
        return _KERNELS.types
    try:
        if forced("kernels-package"):
            raise RuntimeError("MASHBOX_FAULT=force:kernels-package")
        mod = importlib.import_module(module)
    except Exception as e:                       # a broken package must not stop the exact path
        _KERNELS.error = f"{type(e).__name__}: {e}"
        if log:
            log(f"mashbox: kernel package {module} did not load ({_KERNELS.error}); every type runs on the exact path")
        return _KERNELS.types
    _KERNELS.module, _KERNELS.name = mod, module
    _KERNELS.types = frozenset(int(t) for t in getattr(mod, "TYPES", ()))
    return _KERNELS.types


def kernel_types() -> frozenset:
    return _KERNELS.types


def kernel_picks_layer() -> bool:
    return _KERNELS.picks_layer()


def weight_path(t: int, shape=(), kernel_types=None) -> str:
    """-> "kq" | "exact": the path a weight of ggml type t and shape (rows, cols) takes (kernel_types limits the kernel
    types; frozenset() = the exact path for everything)"""
    t = int(t)
    allowed = _KERNELS.types if kernel_types is None else frozenset(int(v) for v in kernel_types) & _KERNELS.types
    return "kq" if t in allowed and _KERNELS.covers(t, shape) else "exact"


def device_nbytes(t: int, shape, nbytes: int, kernel_types=None) -> int:
    """device bytes of one tensor (..., rows, cols) whose file blocks take nbytes, on its path: the planes of every
    matrix of a stack on the kernel path, the blocks as stored on the exact path"""
    size = getattr(_KERNELS.module, "plane_bytes", None)
    if size is None or weight_path(t, shape, kernel_types) != "kq":
        return int(nbytes)
    shape = tuple(int(v) for v in shape)
    lay = _layout(t)
    one = 0
    if lay in ("tiles", "both"):
        one += int(size(_KERNELS.module.TILED[int(t)], shape[-2:]))
    if lay in ("rowmajor", "both"):
        one += int(size(int(t), shape[-2:]))
    return int(np.prod(shape[:-2], dtype=np.int64)) * one


# ---------------------------------------------------------------------------------------------------------- prepare
def _device() -> torch.device:
    return torch.device("cuda", torch.cuda.current_device())


def _as_tensor(raw) -> torch.Tensor:
    return raw if isinstance(raw, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(np.asarray(raw, np.uint8)))


LAYOUTS = ("tiles", "rowmajor", "both")


def _layout(t: int) -> str:
    """the layout weights of type t load in: env MBQ_LAYOUT ("tiles" by default, "rowmajor" or "both") for a type the
    kernel package tiles (its TILED map), else "rowmajor" (the package's only planes)"""
    if int(t) not in getattr(_KERNELS.module, "TILED", {}):
        return "rowmajor"
    lay = os.environ.get("MBQ_LAYOUT", "tiles") or "tiles"
    if lay not in LAYOUTS:
        raise ValueError(f"MBQ_LAYOUT={lay!r} is not one of {LAYOUTS}")
    return lay


def _planes_of(raw, t: int, shape):
    """the kernel package's planes on the device: its host repack for host blocks when it has one, else its repack
    (in the layout _layout(t) names)"""
    mod = _KERNELS.module
    if forced("quant-kernel"):
        raise RuntimeError("forced by MASHBOX_FAULT=force:quant-kernel")
    lay = _layout(t)
    kw = {"layout": lay} if lay != "rowmajor" else {}
    if not isinstance(raw, torch.Tensor) and hasattr(mod, "repack_host"):
        return mod.repack_host(t, np.asarray(raw), tuple(shape), **kw).to(_device())
    r = _as_tensor(raw).to(_device())
    return mod.repack(t, r, tuple(shape), stacked=r.dim() > 2, **kw)


def _preflight(planes, rows_cols, lead: int) -> None:
    """the kernel once on the first weight (index 0 of each stacked axis), one row of input in the forward's dtype,
    waited for: a kernel that fails while it runs raises here"""
    for _ in range(lead):
        planes = planes[0]
    x = torch.ones((1, rows_cols[-1]), dtype=PREFLIGHT_DTYPE, device=_device())
    _KERNELS.module.matmul(x, planes)
    torch.cuda.synchronize()


def _layer_preflight(planes, key) -> None:
    """matmul with a device layer= on a whole stack, once per (type, shape); if it raises, stacks of that type and shape
    are sliced per layer before the kernel instead, with one warning"""
    try:
        x = torch.ones((1, key[1][-1]), dtype=PREFLIGHT_DTYPE, device=_device())
        _KERNELS.module.matmul(x, planes, layer=torch.zeros((), dtype=torch.int32, device=_device()))
        torch.cuda.synchronize()
        _KERNELS.layer_preflight[key] = True
    except Exception as e:
        _KERNELS.layer_preflight[key] = f"{type(e).__name__}: {e}"
        warn(f"mashbox: kq layer= for {type_name(key[0])} {key[1]} failed ({_KERNELS.layer_preflight[key]}); stacks "
             f"of this type and shape are sliced per layer before the kernel")


def prepare(raw, t: int, shape, use_kernel: bool = True):
    """raw: host (NumPy) or device (torch) uint8 (rows, row_bytes), or a stack of them along leading axes; shape is one
    tensor's (rows, cols) -> Packed or Raw on the GPU"""
    t = int(t)
    if t in CODEBOOK_TYPES:
        raise NotImplementedError(f"ggml type {CODEBOOK_TYPES[t]} decodes through gguf-py's code books, which this build "
                                  f"does not carry")
    if t not in TYPES:
        raise NotImplementedError(f"ggml type {t} has no reader on this path (types {sorted(TYPES)})")
    key = (t, tuple(int(s) for s in shape))
    earlier = _KERNELS.preflight.get(key, True)
    if weight_path(t, shape, None if use_kernel else frozenset()) == "kq" and earlier is True:
        lead = len(tuple(raw.shape)) - 2
        try:
            h = Packed(_planes_of(raw, t, shape), t, shape)
            if key not in _KERNELS.preflight:
                _preflight(h.packed, key[1], lead)
                _KERNELS.preflight[key] = True
            if lead == 1 and key not in _KERNELS.layer_preflight and _KERNELS.picks_layer():
                _layer_preflight(h.packed, key)
            return h
        except Exception as e:                   # the load goes on: this (type, shape) takes the exact path
            _KERNELS.preflight[key] = f"{type(e).__name__}: {e}"
            warn(f"mashbox: kq planes for {type_name(t)} {key[1]} failed ({_KERNELS.preflight[key]}); weights of this "
                 f"type and shape run on the exact path")
    return Raw(_as_tensor(raw).to(_device()).contiguous(), t, shape)


def stack_mixed(layers, shape, use_kernel: bool = True):
    """one role over layers: `layers` = [(raw blocks (rows, row_bytes), ggml type)] in layer order, all of logical
    shape (rows, cols). One type: its prepared stack. Several: a Mixed of one prepared stack per type (in order of
    first appearance) with which / sub as device int32 (layers,)"""
    types = [int(t) for _, t in layers]
    order = list(dict.fromkeys(types))
    if len(order) == 1:
        return prepare(np.stack([np.asarray(r) for r, _ in layers]), order[0], shape, use_kernel)
    which = [order.index(t) for t in types]
    sub = [which[:l].count(which[l]) for l in range(len(which))]
    stacks = [prepare(np.stack([np.asarray(r) for r, t in layers if t == u]), u, shape, use_kernel) for u in order]
    dev = _device()
    return Mixed(stacks, torch.tensor(which, dtype=torch.int32, device=dev), torch.tensor(sub, dtype=torch.int32, device=dev),
                 order, shape)


def stack_rows(parts):
    """weights that multiply one input (a layer's q, k and v; its gate and up) as one weight: `parts` =
    [(raw blocks (rows_i, row_bytes), ggml type)], all of one type and row length, host (NumPy) or device (torch) ->
    (raw (sum rows_i, row_bytes), type, sizes). prepare(raw, type, (sum(sizes), cols)) loads it as one weight, so a
    call runs the parts in one kernel launch, and torch.split(qmatmul(x, h), sizes, -1) gives each part's output as a
    view of the result. No output row mixes weight rows: each part's output is its own product, within the float32
    rounding of another plan. The reference keeps its linear-attention layers' q, k and v stacked by rows the same way
    (one weight w["qkv"], reference src/mashbox/models/qwen3_8_27b/model.py:374)."""
    if not parts:
        raise ValueError("stack_rows: no parts")
    types = {int(t) for _, t in parts}
    if len(types) != 1:
        raise ValueError(f"stack_rows: the parts' types differ ({sorted(type_name(t) for t in types)}); only weights of "
                         f"one type stack")
    t = types.pop()
    raws = [r for r, _ in parts]
    widths = {int(r.shape[-1]) for r in raws}
    if len(widths) != 1 or any(len(tuple(r.shape)) != 2 for r in raws):
        raise ValueError(f"stack_rows: every part must be (rows, row_bytes) of one row length, got "
                         f"{[tuple(r.shape) for r in raws]}")
    sizes = [int(r.shape[0]) for r in raws]
    if all(isinstance(r, torch.Tensor) for r in raws):
        return torch.cat([r.to(raws[0].device) for r in raws], 0), t, sizes
    return np.concatenate([r.cpu().numpy() if isinstance(r, torch.Tensor) else np.asarray(r, np.uint8) for r in raws], 0), t, sizes


# ------------------------------------------------------------------------------------------------- the exact path
def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _raw_dequant(raw2: torch.Tensor, t: int, rows: int, cols: int) -> torch.Tensor:
    """(rows, row_bytes) uint8 on the GPU -> float32 (rows, cols), bit for bit the reference dequantization"""
    w = torch.empty((rows, cols), dtype=torch.float32, device=raw2.device)
    _lib.check(_lib.lib().mbq_dequant_raw(int(t), ctypes.c_void_p(raw2.data_ptr()), rows, cols,
                                          ctypes.c_void_p(w.data_ptr()), _stream()), "dequant_raw")
    return w


def _blocks(h: Raw) -> torch.Tensor:
    """a Raw handle's blocks as (..., rows, row_bytes)"""
    rows, cols = h.shape[-2:]
    return h.raw.reshape(tuple(h.raw.shape[:-2]) + (rows, row_bytes(h.t, cols)))


RAW_GEMV_MAX_M = 8                    # activation rows mbq_matmul_raw takes


def _raw_gemv(x: torch.Tensor, h: "Raw") -> torch.Tensor | None:
    """the fused exact-path product for a bfloat16 x of 1-8 rows on a type without kernel planes (mbq_matmul_raw: each
    weight row rebuilt in registers and multiplied in float32, result rounded to bfloat16); None where it does not apply
    (other dtypes: the reference multiplies float32 x, not its bfloat16 rounding)"""
    rows, cols = h.shape[-2:]
    lead = tuple(x.shape[:-1])
    m = int(np.prod(lead, dtype=np.int64)) if lead else 1
    if (x.dtype != torch.bfloat16 or not 1 <= m <= RAW_GEMV_MAX_M or h.t in (2, 8, 12, 13, 14)
            or cols % max(32, TYPES[h.t][1])):
        return None                                  # (the kernel types' blocks, off the kernels: rebuild and GEMM)
    blocks = _blocks(h).reshape(rows, -1).contiguous()
    x2 = x.reshape(m, cols).to(blocks.device).contiguous()
    y = torch.empty((m, rows), dtype=torch.bfloat16, device=blocks.device)
    _lib.check(_lib.lib().mbq_matmul_raw(int(h.t), ctypes.c_void_p(blocks.data_ptr()), ctypes.c_void_p(x2.data_ptr()), m,
                                         rows, cols, ctypes.c_void_p(y.data_ptr()), 1, _stream()), "matmul_raw")
    return y.reshape(lead + (rows,))


def _exact_matmul(x: torch.Tensor, h: Raw) -> torch.Tensor:
    """x (..., cols) @ W.T in float32, the weight rebuilt exact_chunk_rows rows at a time (reference
    ops/__init__.py:574-576, 624-632: a float32 product of float32 x and the float32 weights)"""
    rows, cols = h.shape[-2:]
    blocks = _blocks(h).reshape(rows, -1).contiguous()
    x32 = x.to(device=blocks.device, dtype=torch.float32)
    step = exact_chunk_rows(rows, cols)
    pieces = [torch.matmul(x32, _raw_dequant(blocks[r:r + step], h.t, step, cols).t()) for r in range(0, rows, step)]
    return pieces[0] if len(pieces) == 1 else torch.cat(pieces, dim=-1)


# ------------------------------------------------------------------------------------------------- picking layers
def _held(v) -> bool:
    """a Packed stack of one (rows, cols) weight per layer whose (type, shape) passed the layer= preflight"""
    return isinstance(v, Packed) and len(v.shape) == 2 and _KERNELS.layer_preflight.get((v.t, v.shape)) is True


def _one(stack, sub):
    """layer `sub` of one type stack: At when the kernel reads the layer in place, else the stack indexed (host)"""
    if _held(stack) and _KERNELS.picks_layer():
        return At(stack.packed, sub, stack.t, stack.shape)
    i = int(sub.item()) if isinstance(sub, torch.Tensor) else int(sub)
    return slice_layer(stack, i)


def _on_pick(h: Pick, fn):
    """fn(handle of the picked layer). A host index takes one branch. A device index over stacks the kernel reads in
    place runs every branch with its stack index (outside the stack where `which` names another type: the kernel reads
    nothing and writes NaN) and selects on the device, with no host sync; other stacks read the index on the host."""
    which = h.which
    on_device = isinstance(which, torch.Tensor) and which.is_cuda
    if not on_device or len(h.stacks) == 1 or not all(_held(s) for s in h.stacks) or not _KERNELS.picks_layer():
        i = int(which.item()) if isinstance(which, torch.Tensor) else int(which)
        return fn(_one(h.stacks[i], h.sub))
    out = None
    for i, s in enumerate(h.stacks):
        idx = torch.where(which == i, h.sub, torch.full_like(h.sub, s.packed.lead[0])).to(torch.int32)
        y = fn(At(s.packed, idx, s.t, s.shape))
        out = y if out is None else torch.where(which == i, y, out)
    return out


# ----------------------------------------------------------------------------------------------------- the calls
def _kernel_matmul(x: torch.Tensor, planes, **kw) -> torch.Tensor:
    """the package's matmul with the result in x's dtype. A bfloat16 x gets a bfloat16 result written by the kernel
    (its float32 sums rounded to nearest even, the same bits as a float32 result cast afterwards) when the package takes
    out_dtype=; other dtypes, and packages without it, take the float32 result and a cast."""
    if x.dtype == torch.bfloat16 and _KERNELS.out_dtype():
        return _KERNELS.module.matmul(x, planes, out_dtype=torch.bfloat16, **kw)
    return _KERNELS.module.matmul(x, planes, **kw).to(x.dtype)


def qmatmul(x: torch.Tensor, h) -> torch.Tensor:
    """x (..., cols) @ W.T -> (..., rows): float32 accumulation, result in x's dtype (reference ops/__init__.py:594-632)"""
    if isinstance(h, Pick):
        return _on_pick(h, lambda one: qmatmul(x, one))
    if isinstance(h, At):
        return _kernel_matmul(x, h.packed, layer=h.layer)
    if isinstance(h, Packed):
        return _kernel_matmul(x, h.packed)
    if isinstance(h, Raw):
        if h.raw.dim() > 2:
            raise ValueError(f"{h}: a stack is multiplied one layer at a time (index the stack)")
        y = _raw_gemv(x, h)
        return y if y is not None else _exact_matmul(x, h).to(x.dtype)
    raise TypeError(f"qmatmul: not a weight handle: {h!r}")


def dequant(h) -> torch.Tensor:
    """handle -> float32 weights (..., rows, cols), exact"""
    if isinstance(h, Pick):
        return _on_pick(h, dequant)
    if isinstance(h, At):
        return _KERNELS.module.dequant(h.packed, layer=h.layer)
    if isinstance(h, Packed):
        return _KERNELS.module.dequant(h.packed)
    rows, cols = h.shape[-2:]
    blocks = _blocks(h)
    flat = blocks.reshape(-1, blocks.shape[-1]).contiguous()
    return _raw_dequant(flat, h.t, flat.shape[0], cols).reshape(tuple(blocks.shape[:-2]) + (rows, cols))


def take_rows(h, ids) -> torch.Tensor:
    """rows `ids` of the weights as float32 (an embedding lookup), exact; an id below zero counts from the end. Only the
    looked-up rows are rebuilt."""
    if isinstance(h, Pick):
        return _on_pick(h, lambda one: take_rows(one, ids))
    rows, cols = h.shape[-2:]
    ids = torch.as_tensor(ids, device=_device()).long()
    ids = torch.where(ids < 0, ids + rows, ids)
    gather = getattr(_KERNELS.module, "take_rows", None)
    if isinstance(h, (Packed, At)):
        layer = h.layer if isinstance(h, At) else None
        if gather is not None:
            return gather(h.packed, ids, layer=layer)
        return (dequant(h))[ids]
    blocks = _blocks(h).reshape(rows, -1)
    picked = blocks[ids.reshape(-1)].contiguous()
    if picked.shape[0] == 0:
        return torch.empty(tuple(ids.shape) + (cols,), dtype=torch.float32, device=blocks.device)
    return _raw_dequant(picked, h.t, picked.shape[0], cols).reshape(tuple(ids.shape) + (cols,))


def contract_check(t: int, raw, shape):
    """dequant(repack(raw)) == the reference dequantization (the device raw dequant), bit for bit -> (ok, mismatching
    values); None when the kernel package does not cover type t. NaN must be NaN bit for bit (uint32 compare)."""
    if int(t) not in _KERNELS.types:
        return None
    mod = _KERNELS.module
    r = _as_tensor(raw).to(_device()).contiguous()
    rows, cols = int(shape[-2]), int(shape[-1])
    want = _raw_dequant(r.reshape(rows, -1), int(t), rows, cols)
    got = mod.dequant(mod.repack(int(t), r, tuple(shape))).reshape(rows, cols)
    bad = int((want.view(torch.int32) != got.view(torch.int32)).sum().item())
    return bad == 0, bad


# ------------------------------------------------------------------------------------------------- layer stacks
def _walk(f, tree):
    if isinstance(tree, dict):
        return {k: _walk(f, v) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        return type(tree)(_walk(f, v) for v in tree)
    return f(tree)


def _whole(v) -> bool:
    """a leaf the layer loop keeps whole: a held Packed stack, or a Mixed (its stacks are picked per layer)"""
    return isinstance(v, Mixed) and not isinstance(v, Pick) or (_KERNELS.picks_layer() and _held(v))


def scan_split(ws):
    """a tree of weights stacked over layers -> (held, xs): leaves kept whole by the layer loop (held Packed stacks and
    Mixed roles) go to `held` (None in xs); the others stay in xs, sliced per layer as before. Nothing held: (None, ws)."""
    flags = []
    _walk(lambda v: flags.append(_whole(v)), ws)
    if not any(flags):
        return None, ws
    return _walk(lambda v: v if _whole(v) else None, ws), _walk(lambda v: None if _whole(v) else v, ws)


def scan_join(held, w, layer):
    """inside the loop body, at `layer` (an int or a device int32): w with each held leaf as that layer's handle (At of
    a held stack, Pick of a Mixed)"""
    if held is None:
        return w
    if isinstance(held, dict):
        return {k: scan_join(held[k], None if w is None else w[k], layer) for k in held}
    if isinstance(held, (list, tuple)):
        return type(held)(scan_join(v, None if w is None else w[i], layer) for i, v in enumerate(held))
    if isinstance(held, Mixed):
        return Pick(held.stacks, held.which[layer], held.sub[layer], held.types, held.shape)
    if isinstance(held, Packed):
        return At(held.packed, layer, held.t, held.shape)
    return w


def slice_layer(h, i: int):
    """layer i of a stacked handle (what a per-layer slice gives)"""
    if isinstance(h, Packed):
        return Packed(h.packed[i], h.t, h.shape)
    if isinstance(h, Raw):
        return Raw(h.raw[i], h.t, h.shape)
    if isinstance(h, Mixed):
        w = int(h.which[i].item()) if isinstance(h.which, torch.Tensor) else int(h.which[i])
        s = int(h.sub[i].item()) if isinstance(h.sub, torch.Tensor) else int(h.sub[i])
        return slice_layer(h.stacks[w], s)
    raise TypeError(f"slice_layer: {h!r}")
