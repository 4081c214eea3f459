"""ctypes binding of the device C-ABI (include/ferrograd_hip.h).

This is the layer a Rust `HipDevice` would bind; tests use it to exercise the
backend directly, the benchmark uses its events for kernel timing.
"""
from __future__ import annotations

import ctypes

from . import lib

FG_ARG_PTR, FG_ARG_I32, FG_ARG_F32, FG_ARG_BOOL = 0, 1, 2, 3
FG_OK, FG_ERR_HIP, FG_ERR_COMPILE, FG_ERR_SYMBOL, FG_ERR_ARGS, FG_ERR_INVALID = range(6)
FG_NOALLOC_SCRATCH_BYTES = 64 << 20  # include/ferrograd_hip.h


class _Val(ctypes.Union):
    _fields_ = [("p", ctypes.c_void_p), ("i", ctypes.c_int32), ("f", ctypes.c_float), ("b", ctypes.c_uint8)]


class Arg(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("reserved", ctypes.c_int32), ("v", _Val)]

    @staticmethod
    def ptr(p):
        a = Arg()
        a.kind = FG_ARG_PTR
        a.v.p = p
        return a

    @staticmethod
    def i32(x):
        a = Arg()
        a.kind = FG_ARG_I32
        a.v.i = x
        return a

    @staticmethod
    def f32(x):
        a = Arg()
        a.kind = FG_ARG_F32
        a.v.f = x
        return a

    @staticmethod
    def boolean(x):
        a = Arg()
        a.kind = FG_ARG_BOOL
        a.v.b = 1 if x else 0
        return a


_declared = False


def api() -> ctypes.CDLL:
    global _declared
    l = lib()
    if not _declared:
        P, PP = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        c_int, c_size = ctypes.c_int, ctypes.c_size_t
        uint3 = ctypes.c_uint * 3
        sigs = {
            "fg_hip_init": (c_int, [c_int, PP]),
            "fg_hip_destroy": (c_int, [P]),
            "fg_hip_alloc": (c_int, [P, c_size, c_int, PP]),
            "fg_hip_alloc_hint": (c_int, [P, c_size, c_int, P, PP]),
            "fg_hip_free": (c_int, [P, P]),
            "fg_hip_trim": (c_int, [P]),
            "fg_hip_copy_h2d": (c_int, [P, P, P, c_size]),
            "fg_hip_copy_d2h": (c_int, [P, P, P, c_size]),
            "fg_hip_copy_d2d": (c_int, [P, P, P, c_size]),
            "fg_hip_compile": (c_int, [P, ctypes.c_char_p, ctypes.c_char_p, c_int, PP]),
            "fg_hip_program_free": (c_int, [P]),
            "fg_hip_program_num_args": (c_int, [P]),
            "fg_hip_launch": (c_int, [P, P, ctypes.POINTER(Arg), c_int, uint3, uint3, ctypes.c_uint]),
            "fg_hip_sync": (c_int, [P]),
            "fg_hip_graph_create": (c_int, [P, c_int, PP, ctypes.POINTER(ctypes.c_uint), ctypes.POINTER(ctypes.c_uint),
                                            ctypes.POINTER(ctypes.c_uint), ctypes.POINTER(c_int), ctypes.POINTER(Arg),
                                            PP]),
            "fg_hip_graph_launch": (c_int, [P, P, ctypes.POINTER(Arg), ctypes.POINTER(c_int)]),
            "fg_hip_graph_free": (c_int, [P]),
            "fg_hip_event_record": (c_int, [P, c_int]),
            "fg_hip_event_elapsed_ms": (c_int, [P, c_int, c_int, ctypes.POINTER(ctypes.c_float)]),
            "fg_hip_device_info": (c_int, [P, ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.POINTER(c_size),
                                           ctypes.c_char_p, c_size]),
            "fg_hip_profile_enable": (c_int, [P, c_int]),
            "fg_hip_profile_read": (c_int, [P, ctypes.c_char_p, c_size, ctypes.POINTER(c_size)]),
            "fg_device_context": (c_int, [c_int, PP]),
            "fg_hip_last_error": (ctypes.c_char_p, []),
            "fg_hip_render": (c_int, [ctypes.c_char_p, PP]),
            "fg_hip_rendered_info": (c_int, [P, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_char_p),
                                             ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.POINTER(c_size)]),
            "fg_hip_rendered_param": (c_int, [P, c_int, ctypes.POINTER(c_int)]),
            "fg_hip_rendered_launch": (c_int, [P, c_int, ctypes.POINTER(ctypes.c_char_p), uint3, uint3,
                                               ctypes.POINTER(ctypes.c_uint)]),
            "fg_hip_rendered_free": (c_int, [P]),
            "fg_hip_kernel_load": (c_int, [P, P, PP]),
            "fg_hip_kernel_run": (c_int, [P, P, ctypes.POINTER(Arg), c_int]),
            "fg_hip_kernel_free": (c_int, [P]),
            "fg_hip_kernel_run_noalloc": (c_int, [P, P, ctypes.POINTER(Arg), c_int]),
            "fg_hip_code_object_path": (ctypes.c_char_p, [ctypes.c_char_p]),
        }
        for name, (res, args) in sigs.items():
            f = getattr(l, name)
            f.restype = res
            f.argtypes = args
        _declared = True
    return l


def last_error() -> str:
    return api().fg_hip_last_error().decode()


class HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def check(rc: int) -> None:
    if rc != FG_OK:
        raise HipError(rc, last_error())


class Context:
    """An fg_ctx (device + stream)."""

    def __init__(self, ordinal: int = 0, handle: int | None = None):
        self.h = ctypes.c_void_p()
        if handle is not None:
            self.h = ctypes.c_void_p(handle)
        else:
            check(api().fg_hip_init(ordinal, ctypes.byref(self.h)))

    @staticmethod
    def of_device() -> "Context":
        """The HIP device's own context: the stream realised kernels run on."""
        h = ctypes.c_void_p()
        rc = api().fg_device_context(1, ctypes.byref(h))
        if rc != 0:
            from . import FerrogradError

            raise FerrogradError(api().fg_last_error().decode())
        return Context(handle=h.value)

    def profile(self, on: bool) -> None:
        check(api().fg_hip_profile_enable(self.h, int(on)))

    def profile_read(self) -> list:
        import json

        need = ctypes.c_size_t()
        check(api().fg_hip_profile_read(self.h, None, 0, ctypes.byref(need)))
        buf = ctypes.create_string_buffer(need.value + 1)
        check(api().fg_hip_profile_read(self.h, buf, need.value + 1, ctypes.byref(need)))
        return json.loads(buf.value.decode())

    def alloc(self, nbytes: int, zero: bool = True) -> int:
        p = ctypes.c_void_p()
        check(api().fg_hip_alloc(self.h, nbytes, int(zero), ctypes.byref(p)))
        return p.value

    def alloc_hint(self, nbytes: int, hint: int, zero: bool = False) -> int:
        """fg_hip_alloc_hint: the cached free block `hint` when it is free and
        of this size, else any block."""
        p = ctypes.c_void_p()
        check(api().fg_hip_alloc_hint(self.h, nbytes, int(zero), hint, ctypes.byref(p)))
        return p.value

    def free(self, p: int) -> None:
        check(api().fg_hip_free(self.h, p))

    def h2d(self, dst: int, arr) -> None:
        check(api().fg_hip_copy_h2d(self.h, dst, arr.ctypes.data, arr.nbytes))

    def d2h(self, arr, src: int) -> None:
        check(api().fg_hip_copy_d2h(self.h, arr.ctypes.data, src, arr.nbytes))

    def compile(self, source: str, name: str, num_args: int) -> int:
        p = ctypes.c_void_p()
        check(api().fg_hip_compile(self.h, source.encode(), name.encode(), num_args, ctypes.byref(p)))
        return p.value

    def launch(self, prog: int, args, grid=(1, 1, 1), block=(64, 1, 1), lds: int = 0) -> None:
        arr = (Arg * max(1, len(args)))(*args)
        g = (ctypes.c_uint * 3)(*grid)
        b = (ctypes.c_uint * 3)(*block)
        check(api().fg_hip_launch(self.h, prog, arr, len(args), g, b, lds))

    def sync(self) -> None:
        check(api().fg_hip_sync(self.h))

    def graph_create(self, launches) -> int:
        """Record launches [(prog, args, grid, block, lds), ...] as one HIP
        graph (fg_hip_graph_create); returns the graph handle."""
        n = len(launches)
        progs = (ctypes.c_void_p * n)(*[l[0] for l in launches])
        grids = (ctypes.c_uint * (3 * n))(*[g for l in launches for g in l[2]])
        blocks = (ctypes.c_uint * (3 * n))(*[b for l in launches for b in l[3]])
        lds = (ctypes.c_uint * n)(*[l[4] for l in launches])
        nargs = (ctypes.c_int * n)(*[len(l[1]) for l in launches])
        flat = [a for l in launches for a in l[1]]
        args = (Arg * max(1, len(flat)))(*flat)
        g = ctypes.c_void_p()
        check(api().fg_hip_graph_create(self.h, n, progs, grids, blocks, lds, nargs, args, ctypes.byref(g)))
        return g.value

    def graph_launch(self, graph: int, args) -> int:
        """Launch a recorded graph with every launch's arguments (concatenated);
        returns how many launches had to be updated."""
        arr = (Arg * max(1, len(args)))(*args)
        updated = ctypes.c_int()
        check(api().fg_hip_graph_launch(self.h, graph, arr, ctypes.byref(updated)))
        return updated.value

    def graph_free(self, graph: int) -> None:
        check(api().fg_hip_graph_free(graph))

    def record(self, slot: int) -> None:
        check(api().fg_hip_event_record(self.h, slot))

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        check(api().fg_hip_event_elapsed_ms(self.h, a, b, ctypes.byref(ms)))
        return ms.value

    def info(self) -> dict:
        cu, clk, lds = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
        arch = ctypes.create_string_buffer(64)
        check(api().fg_hip_device_info(self.h, ctypes.byref(cu), ctypes.byref(clk), ctypes.byref(lds), arch, 64))
        return {"cu_count": cu.value, "clock_khz": clk.value, "lds_per_block": lds.value, "arch": arch.value.decode()}


class Rendered:
    """fg_hip_render: one rangeified kernel (its fg-kernel text) rendered for
    gfx950, with its launch passes, parameter kinds and scratch size."""

    def __init__(self, kernel_text: str):
        h = ctypes.c_void_p()
        check(api().fg_hip_render(kernel_text.encode(), ctypes.byref(h)))
        self.h = h
        src, kind = ctypes.c_char_p(), ctypes.c_char_p()
        npar, nl, scratch = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
        check(api().fg_hip_rendered_info(h, ctypes.byref(src), ctypes.byref(kind), ctypes.byref(npar),
                                         ctypes.byref(nl), ctypes.byref(scratch)))
        self.source, self.kind, self.scratch_bytes = src.value.decode(), kind.value.decode(), scratch.value
        self.params = []
        for i in range(npar.value):
            k = ctypes.c_int()
            check(api().fg_hip_rendered_param(h, i, ctypes.byref(k)))
            self.params.append(k.value)
        self.launches = []
        for i in range(nl.value):
            f, g, b, lds = ctypes.c_char_p(), (ctypes.c_uint * 3)(), (ctypes.c_uint * 3)(), ctypes.c_uint()
            check(api().fg_hip_rendered_launch(h, i, ctypes.byref(f), g, b, ctypes.byref(lds)))
            self.launches.append({"func": f.value.decode(), "grid": tuple(g), "block": tuple(b), "lds": lds.value})

    def __del__(self):
        if getattr(self, "h", None):
            api().fg_hip_rendered_free(self.h)
            self.h = None


class Kernel:
    """A rendered kernel loaded on a context (fg_hip_kernel_load)."""

    def __init__(self, ctx: "Context", rendered: Rendered):
        h = ctypes.c_void_p()
        check(api().fg_hip_kernel_load(ctx.h, rendered.h, ctypes.byref(h)))
        self.h, self.ctx, self.rendered = h, ctx, rendered

    def run(self, args) -> None:
        """fg_hip_kernel_run: every pass, with the library's scratch."""
        arr = (Arg * max(1, len(args)))(*args)
        check(api().fg_hip_kernel_run(self.ctx.h, self.h, arr, len(args)))

    def run_noalloc(self, args) -> None:
        """fg_hip_kernel_run_noalloc: every pass, with the library's static
        per-GPU scratch; allocates nothing."""
        arr = (Arg * max(1, len(args)))(*args)
        check(api().fg_hip_kernel_run_noalloc(self.ctx.h, self.h, arr, len(args)))

    def __del__(self):
        if getattr(self, "h", None):
            api().fg_hip_kernel_free(self.h)
            self.h = None


def code_object_path(source: str) -> str:
    """Where fg_hip_compile caches the code object of `source`."""
    return api().fg_hip_code_object_path(source.encode()).decode()
