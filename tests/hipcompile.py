"""Compile rendered HIP kernels for gfx950 without a GPU, each within a time
limit: fg_hip_compile with a NULL context runs hiprtc and caches the code
object, nothing more. The compiles run in child processes (spawned, so no
HIP state is inherited) against fresh code-object and compiler caches, so
every source is really compiled, and a compile that does not finish fails the caller
instead of stalling it."""
from __future__ import annotations

import multiprocessing as mp
import os
import re
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _init(cache_dir: str) -> None:
    import sys

    os.environ["FG_KERNEL_CACHE"] = cache_dir
    # hiprtc's compiler library keeps a cache of its own (comgr): point it at
    # the same fresh directory, so no source is answered from an earlier run.
    os.environ["AMD_COMGR_CACHE_DIR"] = os.path.join(cache_dir, "comgr")
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)


def _compile(item):
    import ctypes
    import time

    from ferrograd_amd.hip import api

    source, func = item
    t0 = time.perf_counter()
    out = ctypes.c_void_p()
    rc = api().fg_hip_compile(None, source.encode(), func.encode(), 0, ctypes.byref(out))
    err = api().fg_hip_last_error().decode() if rc else ""
    return func, rc, err, time.perf_counter() - t0


def kernel_functions(source: str) -> list[str]:
    """The __global__ functions a rendered source defines."""
    return re.findall(r"extern \"C\" __global__ void __launch_bounds__\(\d+\) (\w+)\(", source)


def compile_sources(sources: dict[str, str], limit_s: float, workers: int = 8) -> list[tuple[str, float]]:
    """Compile every (source -> name) pair, `workers` at a time; every source
    must compile, and all of them within `limit_s` seconds in all. Returns
    (function, seconds) per source, slowest first."""
    items = []
    for src, name in sources.items():
        fns = kernel_functions(src)
        items.append((src, fns[0] if fns else name))
    ctx = mp.get_context("spawn")
    with tempfile.TemporaryDirectory() as cache:
        pool = ctx.Pool(min(workers, max(1, len(items))), initializer=_init, initargs=(cache,))
        try:
            res = pool.map_async(_compile, items, chunksize=1).get(timeout=limit_s)
        except mp.TimeoutError:
            raise AssertionError(f"compiling {len(items)} kernels did not finish within {limit_s} s") from None
        finally:
            pool.terminate()
            pool.join()
    bad = [(f, e) for f, rc, e, _ in res if rc]
    assert not bad, bad[:3]
    return sorted(((f, t) for f, _, _, t in res), key=lambda x: -x[1])
