"""fg_hip_kernel_run_noalloc (include/ferrograd_hip.h) against
fg_hip_kernel_run, through the C-ABI: the same rendered kernels, with the
library's static per-GPU scratch instead of scratch it allocates. Two calls
in a row, the second on a smaller problem, so the second runs over what the
first left in the static scratch; results bit for bit equal to
fg_hip_kernel_run's (the same kernels in the same deterministic order) and
within 1e-4 of sum|terms| of float64. A kernel needing more scratch than the
static array holds is refused before anything runs."""
from __future__ import annotations

import re

import numpy as np
import pytest

from conftest import rel_err_bound

pytestmark = pytest.mark.gpu


def dw_kernel(fg, B, M, N, seed):
    """The split-K weight-gradient product dW = gᵀ·h ([M, N], K = B) as one
    rendered kernel, with its host inputs."""
    from ferrograd_amd.hip import Rendered

    r = np.random.default_rng(seed)
    g = (r.standard_normal((B, M)) / B).astype(np.float32)
    h = r.uniform(0, 1, (B, N)).astype(np.float32)
    tg, th = fg.Tensor.new(g, [B, M], "hip"), fg.Tensor.new(h, [B, N], "hip")
    w = fg.Tensor.new(np.ones((M, N), np.float32), [M, N], "hip").with_requires_grad(True)
    (dw,) = th.matmul(w.permute([1, 0])).mul(tg).sum([0, 1]).gradient([w])
    (item,) = fg.debug_plan([dw], fuse=True, render_hip=True)["items"]
    return Rendered(item["kernel"]), item["kernel"], g, h


def run_both(ctx, fg, rendered, text, g, h, M, N):
    from ferrograd_amd.hip import Arg, Kernel

    k = Kernel(ctx, rendered)
    sizes = {int(m.group(1)): int(m.group(2)) for m in re.finditer(r"ParamBuffer \w+ param:(\d+):(\d+)", text)}
    by_size = {g.size: g, h.size: h}
    assert g.size != h.size and sizes[0] == M * N and len(sizes) == 3
    ins = []
    for slot in (1, 2):
        a = by_size[sizes[slot]]
        p = ctx.alloc(a.nbytes, zero=False)
        ctx.h2d(p, a)
        ins.append(p)
    outs = {}
    for mode in ("noalloc", "run"):
        out = ctx.alloc(M * N * 4, zero=False)
        args = [Arg.ptr(out)] + [Arg.ptr(p) for p in ins]
        (k.run_noalloc if mode == "noalloc" else k.run)(args)
        host = np.empty(M * N, np.float32)
        ctx.d2h(host, out)
        ctx.free(out)
        outs[mode] = host.reshape(M, N)
    for p in ins:
        ctx.free(p)
    return outs


def test_noalloc_matches_kernel_run_on_two_calls(fg, hip):
    from ferrograd_amd.hip import FG_NOALLOC_SCRATCH_BYTES, Context

    ctx = Context.of_device()
    results = []
    # First call: 32 MiB of split-K partials; second: a smaller problem
    # (8 MiB), run over the first call's leftovers.
    for (B, M, N, seed) in ((8192, 512, 256, 1), (4096, 256, 128, 2)):
        r, text, g, h = dw_kernel(fg, B, M, N, seed)
        assert 0 < r.scratch_bytes <= FG_NOALLOC_SCRATCH_BYTES and len(r.launches) == 2
        outs = run_both(ctx, fg, r, text, g, h, M, N)
        assert np.array_equal(outs["noalloc"].view(np.uint32), outs["run"].view(np.uint32))
        g64, h64 = g.astype(np.float64), h.astype(np.float64)
        assert rel_err_bound(outs["noalloc"], g64.T @ h64, np.abs(g64).T @ np.abs(h64), 1e-4) <= 1.0
        results.append(r.scratch_bytes)
    assert results[1] < results[0]


def test_noalloc_refuses_a_kernel_beyond_its_scratch(fg, hip):
    from ferrograd_amd.hip import FG_NOALLOC_SCRATCH_BYTES, Arg, Context, HipError, Kernel

    ctx = Context.of_device()
    r, text, g, h = dw_kernel(fg, 8192, 2560, 2560, 3)  # 4 K splits of a 2560x2560 output: 125 MiB
    assert r.scratch_bytes > FG_NOALLOC_SCRATCH_BYTES
    k = Kernel(ctx, r)
    p = ctx.alloc(4)
    with pytest.raises(HipError, match="more than the 67108864 the library holds per GPU"):
        k.run_noalloc([Arg.ptr(p)] * 3)
    ctx.sync()
    ctx.free(p)
