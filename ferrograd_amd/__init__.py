"""ferrograd_amd — an MI355X-native execution path for ferrograd's realize pipeline.

The Python API mirrors the reference's public Rust API (src/tensor.rs,
src/nn.rs, src/optim.rs): lazy `Tensor` graphs that realise through the
C++ scheduler, the gfx950 lowering and the HIP device in
`libferrograd_amd.so` (C-ABI: include/ferrograd.h, include/ferrograd_hip.h).

Devices: "hip" (the MI355X) and "cpu" (only when the test oracle has been
loaded). Nothing here falls back to the CPU: if the native library is missing
the import of any op raises.
"""
from __future__ import annotations

import ctypes
import importlib
import os
from typing import Iterable, Sequence

import numpy as np

__all__ = ["Tensor", "Linear", "Sgd", "FerrogradError", "lib", "stats", "synchronize", "reset_init_seed",
           "debug_plan", "F32", "I32", "BOOL", "clear_caches"]

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libferrograd_amd.so")

F32, I32, BOOL = 0, 1, 2
_DEVICES = {"cpu": 0, "hip": 1}
_DTYPES = {"f32": F32, "float32": F32, "i32": I32, "int32": I32, "bool": BOOL}
_NP = {F32: np.float32, I32: np.int32, BOOL: np.bool_}

_lib = None


class FerrogradError(RuntimeError):
    """An error reported by the native library (the reference panics here)."""


# The hot Tensor methods live in the CPython extension `_fgc` (csrc/pymodule.c),
# which links the native library. Until it is built (python -m
# ferrograd_amd.build) the package imports, and lib() refuses to run.
try:
    # import_module, not `from . import`: a reload after the build must not
    # take the None this name held before the extension existed.
    _fgc = importlib.import_module("._fgc", __name__)
except ImportError as _fgc_missing:  # noqa: F841
    _fgc = None
else:
    _fgc.set_error_class(FerrogradError)


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH) or _fgc is None:
            raise FerrogradError(f"native library not built: {LIB_PATH} (run python -m ferrograd_amd.build)")
        l = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        _declare(l)
        _lib = l
    return _lib


def _declare(l: ctypes.CDLL) -> None:
    P = ctypes.c_void_p
    PP = ctypes.POINTER(ctypes.c_void_p)
    i64p = ctypes.POINTER(ctypes.c_int64)
    c_int, c_size = ctypes.c_int, ctypes.c_size_t
    sigs = {
        "fg_last_error": (ctypes.c_char_p, []),
        "fg_tensor_from_data": (c_int, [c_int, c_int, P, c_size, i64p, c_int, PP]),
        "fg_tensor_zeros": (c_int, [c_int, c_int, i64p, c_int, PP]),
        "fg_tensor_ones": (c_int, [c_int, c_int, i64p, c_int, PP]),
        "fg_tensor_free": (c_int, [P]),
        "fg_idx_images": (c_int, [ctypes.c_char_p, c_int, PP]),
        "fg_idx_labels": (c_int, [ctypes.c_char_p, P, c_size, ctypes.POINTER(c_size)]),
        "fg_tensor_unary": (c_int, [P, c_int, PP]),
        "fg_tensor_binary": (c_int, [P, P, c_int, PP]),
        "fg_tensor_reduce": (c_int, [P, c_int, i64p, c_int, PP]),
        "fg_tensor_movement": (c_int, [P, c_int, i64p, c_int, PP]),
        "fg_tensor_narrow": (c_int, [P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, PP]),
        "fg_tensor_log_softmax": (c_int, [P, ctypes.c_int64, PP]),
        "fg_tensor_assign": (c_int, [P, P]),
        "fg_tensor_replace": (c_int, [P, P]),
        "fg_tensor_realize_many": (c_int, [PP, c_int]),
        "fg_tensor_read": (c_int, [P, P, c_size]),
        "fg_tensor_write": (c_int, [P, P, c_size]),
        "fg_tensor_shape": (c_int, [P, i64p, ctypes.POINTER(c_int)]),
        "fg_tensor_info": (c_int, [P] + [ctypes.POINTER(c_int)] * 4),
        "fg_tensor_set_requires_grad": (c_int, [P, c_int]),
        "fg_tensor_same": (c_int, [P, P, ctypes.POINTER(c_int)]),
        "fg_tensor_data_ptr": (c_int, [P, PP, ctypes.POINTER(c_size)]),
        "fg_tensor_grad": (c_int, [P, PP]),
        "fg_tensor_backward": (c_int, [P]),
        "fg_tensor_gradient": (c_int, [P, PP, c_int, PP]),
        "fg_reset_init_seed": (c_int, [ctypes.c_uint64]),
        "fg_linear_new": (c_int, [c_int, ctypes.c_int64, ctypes.c_int64, c_int, PP]),
        "fg_linear_forward": (c_int, [P, P, PP]),
        "fg_linear_num_params": (c_int, [P, ctypes.POINTER(c_int)]),
        "fg_linear_param": (c_int, [P, c_int, PP]),
        "fg_linear_free": (c_int, [P]),
        "fg_sgd_new": (c_int, [PP, c_int, ctypes.c_float, PP]),
        "fg_sgd_zero_grad": (c_int, [P]),
        "fg_sgd_step": (c_int, [P]),
        "fg_mlp_train_steps": (c_int, [P, c_int, P, P, P, c_int, ctypes.POINTER(ctypes.c_float)]),
        "fg_mlp_train_batches": (c_int, [P, c_int, P, P, P, ctypes.c_int64, ctypes.c_int64, c_int,
                                         ctypes.POINTER(ctypes.c_float)]),
        "fg_sgd_free": (c_int, [P]),
        "fg_synchronize": (c_int, [c_int]),
        "fg_default_device": (c_int, [ctypes.POINTER(c_int)]),
        "fg_gpu_passes": (c_int, [ctypes.POINTER(c_int)] * 6),
        "fg_stats": (c_int, [ctypes.POINTER(ctypes.c_uint64)] * 3),
        "fg_graph_stats": (c_int, [ctypes.POINTER(ctypes.c_uint64)] * 2),
        "fg_step_capture_stats": (c_int, [ctypes.POINTER(ctypes.c_uint64)] * 2),
        "fg_clear_caches": (c_int, []),
        "fg_host_times": (c_int, [ctypes.POINTER(ctypes.c_uint64)]),
        "fg_plan_cache_enable": (c_int, [c_int]),
        "fg_plan_cache_stats": (c_int, [ctypes.POINTER(ctypes.c_uint64)] * 3),
        "fg_set_graph_min_launches": (c_int, [c_int, ctypes.POINTER(c_int)]),
        "fg_debug_plan": (c_int, [PP, c_int, c_int, c_int, ctypes.c_char_p, c_size, ctypes.POINTER(c_size)]),
    }
    for name, (res, args) in sigs.items():
        f = getattr(l, name)
        f.restype = res
        f.argtypes = args


def _check(rc: int) -> None:
    if rc != 0:
        raise FerrogradError(lib().fg_last_error().decode())


def _i64(xs: Iterable[int]):
    xs = [int(x) for x in xs]
    return (ctypes.c_int64 * max(1, len(xs)))(*xs), len(xs)


def _dev(device) -> int:
    """Device code of a name ("hip", "cpu"), a code, or None: the default
    device, which the DEVICE environment variable selects ("hip" unless set)."""
    if device is None:
        code = ctypes.c_int()
        _check(lib().fg_default_device(ctypes.byref(code)))
        return code.value
    if isinstance(device, int):
        return device
    try:
        return _DEVICES[device]
    except KeyError:
        raise FerrogradError(f"unknown device {device!r}") from None


def _dtype_code(dtype) -> int:
    if dtype is None:
        return F32
    if isinstance(dtype, int):
        return dtype
    if isinstance(dtype, str):
        return _DTYPES[dtype]
    dt = np.dtype(dtype)
    if dt == np.float32:
        return F32
    if dt == np.int32:
        return I32
    if dt == np.bool_:
        return BOOL
    raise FerrogradError(f"unsupported dtype {dtype!r}")


class Tensor(_fgc.TensorBase if _fgc is not None else object):
    """A lazily evaluated tensor (tensor.rs:95-97). Handles alias shared state.

    The handle (`_h`, an int) and the graph-building ops (unary, binary,
    reductions, movement, narrow, log_softmax, realize, assign, alias) come
    from the extension type; `Tensor(handle)` adopts a handle the C-ABI
    returned."""

    __slots__ = ()

    @staticmethod
    def _out(fn, *args) -> "Tensor":
        # One ctypes call that returns a new handle through its last argument.
        out = ctypes.c_void_p()
        if fn(*args, ctypes.byref(out)):
            raise FerrogradError(_lib.fg_last_error().decode())
        return _fgc.from_handle(Tensor, out.value)

    # ── construction (tensor.rs:260-312) ─────────────────────────────────
    @staticmethod
    def new(data, shape: Sequence[int] | None = None, device=None, dtype=None) -> "Tensor":
        """Tensor::new — copy host data into a new device buffer."""
        if dtype is None:
            # ndarrays keep int32/bool; everything else (lists, float64) is f32
            # unless it is a list of bools.
            if isinstance(data, np.ndarray) and data.dtype in (np.int32, np.bool_):
                dtype = data.dtype
            elif isinstance(data, (list, tuple)) and data and all(isinstance(x, bool) for x in data):
                dtype = np.bool_
            else:
                dtype = np.float32
        code = _dtype_code(dtype)
        arr = np.ascontiguousarray(np.asarray(data, dtype=_NP[code]))
        if shape is None:
            shape = arr.shape
        if code == BOOL:
            arr = arr.astype(np.uint8)
        s, n = _i64(shape)
        return Tensor._out(lib().fg_tensor_from_data, _dev(device), code, arr.ctypes.data_as(ctypes.c_void_p),
                           arr.nbytes, s, n)

    @staticmethod
    def zeros(shape: Sequence[int], device=None, dtype=None) -> "Tensor":
        s, n = _i64(shape)
        return Tensor._out(lib().fg_tensor_zeros, _dev(device), _dtype_code(dtype), s, n)

    @staticmethod
    def ones(shape: Sequence[int], device=None, dtype=None) -> "Tensor":
        s, n = _i64(shape)
        return Tensor._out(lib().fg_tensor_ones, _dev(device), _dtype_code(dtype), s, n)

    @staticmethod
    def full(shape: Sequence[int], value: float, device=None) -> "Tensor":
        return Tensor.new(np.full(int(np.prod(shape)) if len(shape) else 1, value, dtype=np.float32), shape, device)

    @staticmethod
    def scalar(value: float, device=None) -> "Tensor":
        return Tensor.new(np.array([value], dtype=np.float32), [1], device)

    # ── metadata ─────────────────────────────────────────────────────────
    def _info(self):
        d, dev, r, g = (ctypes.c_int(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int())
        _check(lib().fg_tensor_info(self._h, ctypes.byref(d), ctypes.byref(dev), ctypes.byref(r), ctypes.byref(g)))
        return d.value, dev.value, bool(r.value), bool(g.value)

    @property
    def shape(self) -> tuple:
        buf = (ctypes.c_int64 * 16)()
        nd = ctypes.c_int(16)
        _check(lib().fg_tensor_shape(self._h, buf, ctypes.byref(nd)))
        return tuple(buf[i] for i in range(nd.value))

    @property
    def dtype(self) -> int:
        return self._info()[0]

    @property
    def device(self) -> str:
        return {0: "cpu", 1: "hip"}[self._info()[1]]

    def numel(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    def ndim(self) -> int:
        return len(self.shape)

    def is_realized(self) -> bool:
        return self._info()[2]

    def requires_grad(self) -> bool:
        return self._info()[3]

    def with_requires_grad(self, requires_grad: bool = True) -> "Tensor":
        _check(lib().fg_tensor_set_requires_grad(self._h, int(requires_grad)))
        return self

    def data_ptr(self) -> tuple:
        """(device pointer, byte size) of a realised tensor's storage."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        _check(lib().fg_tensor_data_ptr(self._h, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def same(self, other: "Tensor") -> bool:
        s = ctypes.c_int()
        _check(lib().fg_tensor_same(self._h, other._h, ctypes.byref(s)))
        return bool(s.value)

    # ── ops (tensor.rs:442-778): neg, reciprocal, exp2, log2, sqrt, relu, exp,
    # log, contiguous, detach, add, mul, sub, matmul, cross_entropy, reshape,
    # permute, expand, narrow, sum, max, log_softmax, assign and realize are
    # the extension type's methods (csrc/pymodule.c).

    def replace(self, other: "Tensor") -> "Tensor":
        _check(lib().fg_tensor_replace(self._h, other._h))
        return self

    # ── realisation (tensor.rs:781-930) ──────────────────────────────────
    @staticmethod
    def realize_many(tensors: Sequence["Tensor"]) -> None:
        arr = (ctypes.c_void_p * max(1, len(tensors)))(*[t._h for t in tensors])
        _check(lib().fg_tensor_realize_many(arr, len(tensors)))

    def numpy(self) -> np.ndarray:
        code = self.dtype
        shape = self.shape
        n = int(np.prod(shape)) if shape else 1
        out = np.empty(n, dtype=np.uint8 if code == BOOL else _NP[code])
        _check(lib().fg_tensor_read(self._h, out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        if code == BOOL:
            out = out.astype(np.bool_)
        return out.reshape(shape)

    def write(self, data) -> "Tensor":
        """Device::copy_from_host into this realised tensor's buffer; the
        byte count must match (device.rs:294, cpu.rs:282-302)."""
        arr = np.ascontiguousarray(data)
        if self.dtype == BOOL:
            arr = arr.astype(np.uint8)
        _check(lib().fg_tensor_write(self._h, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes))
        return self

    def raw_bytes(self) -> bytes:
        """The realised buffer's bytes (bool as 0/1 bytes)."""
        code = self.dtype
        n = self.numel()
        size = n * (1 if code == BOOL else 4)
        out = np.empty(size, dtype=np.uint8)
        _check(lib().fg_tensor_read(self._h, out.ctypes.data_as(ctypes.c_void_p), size))
        return out.tobytes()

    def to_vec(self) -> list:
        """Tensor::to_vec — realise and return f32 data as a list."""
        if self.dtype != F32:
            raise FerrogradError("to_vec requires F32 tensor data")
        return self.numpy().reshape(-1).tolist()

    # ── autograd (tensor.rs:938-998) ─────────────────────────────────────
    def grad(self) -> "Tensor | None":
        out = ctypes.c_void_p()
        _check(lib().fg_tensor_grad(self._h, ctypes.byref(out)))
        return _fgc.from_handle(Tensor, out.value) if out.value else None

    def backward(self) -> None:
        _check(lib().fg_tensor_backward(self._h))

    def gradient(self, targets: Sequence["Tensor"]) -> list:
        n = len(targets)
        ins = (ctypes.c_void_p * max(1, n))(*[t._h for t in targets])
        outs = (ctypes.c_void_p * max(1, n))()
        _check(lib().fg_tensor_gradient(self._h, ins, n, outs))
        return [_fgc.from_handle(Tensor, outs[i]) for i in range(n)]

    def __repr__(self) -> str:
        try:
            return f"Tensor(shape={list(self.shape)}, device={self.device}, requires_grad={self.requires_grad()})"
        except FerrogradError:
            return "Tensor(<invalid>)"


class Linear:
    """nn::Linear (nn.rs:67-104): weight [out, in], Kaiming-normal seeded init, zero bias."""

    def __init__(self, in_features: int, out_features: int, device=None, bias: bool = True):
        h = ctypes.c_void_p()
        _check(lib().fg_linear_new(_dev(device), in_features, out_features, int(bias), ctypes.byref(h)))
        self._h = h
        n = ctypes.c_int()
        _check(lib().fg_linear_num_params(h, ctypes.byref(n)))
        ps = [Tensor._out(lib().fg_linear_param, h, i) for i in range(n.value)]
        self.weight = ps[0]
        self.bias = ps[1] if len(ps) > 1 else None

    def forward(self, x: Tensor) -> Tensor:
        return Tensor._out(_lib.fg_linear_forward, self._h, x._h)

    __call__ = forward

    def parameters(self) -> list:
        return [self.weight] + ([self.bias] if self.bias is not None else [])

    def __del__(self):
        if _lib is not None and getattr(self, "_h", None):
            _lib.fg_linear_free(self._h)
            self._h = None


class Sgd:
    """optim::Sgd (optim.rs:16-71)."""

    def __init__(self, params: Sequence[Tensor], lr: float):
        arr = (ctypes.c_void_p * max(1, len(params)))(*[p._h for p in params])
        h = ctypes.c_void_p()
        _check(lib().fg_sgd_new(arr, len(params), ctypes.c_float(lr), ctypes.byref(h)))
        self._h = h

    def zero_grad(self) -> None:
        _check(lib().fg_sgd_zero_grad(self._h))

    def step(self) -> None:
        _check(lib().fg_sgd_step(self._h))

    def __del__(self):
        if _lib is not None and getattr(self, "_h", None):
            _lib.fg_sgd_free(self._h)
            self._h = None


def train_steps_native(layers: Sequence[Linear], opt: Sgd, x: Tensor, targets: Tensor, steps: int) -> list:
    """fg_mlp_train_steps: `steps` iterations of examples/mnist.rs:84-101's loop
    body (forward with ReLU between layers, cross-entropy, zero_grad,
    backward, SGD step, loss read back) run from native code; the losses."""
    arr = (ctypes.c_void_p * max(1, len(layers)))(*[l._h.value for l in layers])
    out = (ctypes.c_float * max(1, steps))()
    _check(lib().fg_mlp_train_steps(arr, len(layers), opt._h, x._h, targets._h, int(steps), out))
    return [float(out[i]) for i in range(steps)]


def train_batches_native(layers: Sequence[Linear], opt: Sgd, images: Tensor, targets: Tensor, batch_size: int,
                         steps: int, first_batch: int = 0) -> list:
    """fg_mlp_train_batches: the same loop over resident `images` and
    `targets`, step i on rows narrow(0, s, batch_size) with s = ((first_batch
    + i) mod (rows // batch_size)) * batch_size (examples/mnist.rs:84-87);
    the losses."""
    arr = (ctypes.c_void_p * max(1, len(layers)))(*[l._h.value for l in layers])
    out = (ctypes.c_float * max(1, steps))()
    _check(lib().fg_mlp_train_batches(arr, len(layers), opt._h, images._h, targets._h, int(batch_size),
                                      int(first_batch), int(steps), out))
    return [float(out[i]) for i in range(steps)]


def reset_init_seed(seed: int = 42) -> None:
    """Reset the Kaiming init LCG (nn.rs:12-14) to `seed`."""
    _check(lib().fg_reset_init_seed(seed))


def synchronize(device=None) -> None:
    _check(lib().fg_synchronize(_dev(device)))


def default_device() -> str:
    """The device used where a program names none: DEVICE=hip (default) or
    DEVICE=cpu (the test oracle's device). The reference's tensor::cpu()
    (tensor.rs:1122-1127) with the choice moved to the environment."""
    return {v: k for k, v in _DEVICES.items()}[_dev(None)]


def gpu_passes() -> dict:
    """The HIP path's optional passes as OPT selected them for this process
    (reference grammar, src/optimize/mod.rs:85-112; names symbolic, mfma,
    narrow, fuse, block, batch)."""
    v = [ctypes.c_int() for _ in range(6)]
    _check(lib().fg_gpu_passes(*[ctypes.byref(x) for x in v]))
    return dict(zip(("symbolic", "mfma", "narrow", "fuse", "block", "batch"), (bool(x.value) for x in v)))


def stats() -> dict:
    k, p, h = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    lib().fg_stats(ctypes.byref(k), ctypes.byref(p), ctypes.byref(h))
    t = (ctypes.c_uint64 * 5)()
    lib().fg_host_times(t)
    names = ("schedule", "lower", "launch", "apply_map", "backward")
    g, u = ctypes.c_uint64(), ctypes.c_uint64()
    lib().fg_graph_stats(ctypes.byref(g), ctypes.byref(u))
    sc, sr = ctypes.c_uint64(), ctypes.c_uint64()
    lib().fg_step_capture_stats(ctypes.byref(sc), ctypes.byref(sr))
    return {"kernels_launched": k.value, "programs_compiled": p.value, "lowering_cache_hits": h.value,
            "graph_replays": g.value, "graph_updated_launches": u.value,
            "steps_captured": sc.value, "steps_replayed": sr.value,
            "host_ms": {n: t[i] / 1e6 for i, n in enumerate(names)}}


def clear_caches() -> None:
    _check(lib().fg_clear_caches())


def plan_cache(enabled: bool) -> None:
    """Turn realisation-plan replay on or off (off also drops recorded plans)."""
    _check(lib().fg_plan_cache_enable(int(enabled)))


def graph_min_launches(n: int) -> int:
    """Record replayed plans of at least `n` launches (n >= 2) as HIP graphs,
    shorter ones launching one by one; n = 0 (the default unless
    FG_HIP_GRAPHS=1) launches every plan one by one. Returns the previous
    threshold."""
    prev = ctypes.c_int()
    _check(lib().fg_set_graph_min_launches(int(n), ctypes.byref(prev)))
    return prev.value


def plan_stats() -> dict:
    h, m, e = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    _check(lib().fg_plan_cache_stats(ctypes.byref(h), ctypes.byref(m), ctypes.byref(e)))
    return {"hits": h.value, "misses": m.value, "entries": e.value}


def debug_plan(roots: Sequence[Tensor], fuse: bool = False, render_hip: bool = False) -> dict:
    """Schedule `roots` without running them; optionally render HIP kernels."""
    import json
    arr = (ctypes.c_void_p * max(1, len(roots)))(*[t._h for t in roots])
    need = ctypes.c_size_t()
    _check(lib().fg_debug_plan(arr, len(roots), int(fuse), int(render_hip), None, 0, ctypes.byref(need)))
    buf = ctypes.create_string_buffer(need.value + 1)
    _check(lib().fg_debug_plan(arr, len(roots), int(fuse), int(render_hip), buf, need.value + 1, ctypes.byref(need)))
    return json.loads(buf.value.decode())
