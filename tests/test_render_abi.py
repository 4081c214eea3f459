"""The Renderer half of the device boundary (include/ferrograd_hip.h):
fg_hip_render takes a rangeified kernel as text and returns the gfx950
source, launch passes, parameter kinds and scratch size; fg_hip_kernel_load /
fg_hip_kernel_run compile and run it. This is what a Rust `Renderer` +
`Device` pair (codegen.rs:17-20, device.rs:275-332) binds.

CPU tests: the text round trip reproduces the product's own rendering for
every kernel of the benchmark programs, malformed text fails with a message
naming the line, rendered sources compile for gfx950. GPU tests: rendered
kernels, among them split-K GEMMs and split column reductions with library
scratch, run through the C-ABI and match the CPU oracle to the path's
tolerances; argument errors are reported before anything runs; a damaged
cached code object is compiled again."""
from __future__ import annotations

import os
import re
import subprocess
import sys

import numpy as np
import pytest

from conftest import rel_err_bound, seeded


HOST = {"x": (64, 96), "w": (48, 96), "b": (48,), "a": (1000,), "bb": (1000,), "c": (1000,), "tall": (8192, 64),
        "g": (8192, 128), "h": (8192, 96), "gs": (2048, 128), "hs": (2048, 80)}


def host_arrays():
    r = seeded(3)
    return {k: (r.uniform(-1, 1, s) if k in ("a", "bb", "c") else r.standard_normal(s)).astype(np.float32)
            for k, s in HOST.items()}


def programs(fg, dev):
    """Lazy roots of small versions of the benchmark programs, plus a split
    column reduction and a split-K weight-gradient GEMM (kernels with
    scratch), each one kernel when fused; and the host inputs in the
    kernel's slot order."""
    H = host_arrays()
    T = {k: fg.Tensor.new(v, list(v.shape), dev) for k, v in H.items()}
    s0, s1 = fg.Tensor.scalar(0.5, dev), fg.Tensor.scalar(1.0, dev)
    wg = fg.Tensor.new(np.zeros((128, 96), np.float32), [128, 96], dev).with_requires_grad(True)
    loss = T["h"].matmul(wg.permute([1, 0])).mul(T["g"]).sum([0, 1])
    (dw,) = loss.gradient([wg])  # dW = gᵀ·h, K = 8192: split over K
    ws = fg.Tensor.new(np.zeros((128, 80), np.float32), [128, 80], dev).with_requires_grad(True)
    loss_s = T["hs"].matmul(ws.permute([1, 0])).mul(T["gs"]).sum([0, 1])
    (dws,) = loss_s.gradient([ws])  # K = 2048: the one-pass small GEMM
    half, one = np.array([0.5], np.float32), np.array([1.0], np.float32)
    return {
        "c1": (T["x"].mul(s0).add(s1).relu().sum([1]), [H["x"], half, one]),
        "c2": (T["a"].mul(T["bb"]).add(T["c"]).relu(), [H["a"], H["bb"], H["c"]]),
        "c3": (T["x"].matmul(T["w"].permute([1, 0])).add(T["b"]), [H["x"], H["w"], H["b"]]),
        "colsum_split": (T["tall"].sum([0]), [H["tall"]]),
        "dw_split_k": (dw, None),  # inputs g and h, matched by size
        "dw_small": (dws, None),  # inputs gs and hs, matched by size
    }


def plan(fg, root):
    return fg.debug_plan([root], fuse=True, render_hip=True)["items"]


def test_kernel_text_round_trip_reproduces_the_rendering(fg, cpu):
    from ferrograd_amd.hip import Rendered

    roots = programs(fg, cpu)
    # And every kernel of an MLP train step (forward, loss, backward, SGD).
    from ferrograd_amd.mlp import Mlp, synthetic_batch

    fg.reset_init_seed(42)
    m = Mlp((64, 48, 10), cpu)
    xs, ts = synthetic_batch(512, 64, 10, 1, 2)
    loss = m.forward(fg.Tensor.new(xs, list(xs.shape), cpu)).cross_entropy(fg.Tensor.new(ts, list(ts.shape), cpu))
    loss.backward()
    params = m.parameters()
    for p in params:
        p.assign(p.detach().sub(p.grad().mul(fg.Tensor.scalar(0.01, cpu))))
    items = [it for root, _ in roots.values() for it in plan(fg, root)]
    items += fg.debug_plan(params + [loss], fuse=True, render_hip=True)["items"]
    # A column sum too long for one workgroup: split into partials and a finishing pass.
    cols = fg.Tensor.new(np.ones((4096, 512), np.float32), [4096, 512], cpu)
    items += fg.debug_plan([cols.sum([0])], fuse=True, render_hip=True)["items"]
    # A product above the one-pass small-GEMM size with too few tiles for the
    # chip: split-K partials and a finishing pass.
    a = fg.Tensor.new(np.ones((2048, 2048), np.float32), [2048, 2048], cpu)
    w = fg.Tensor.new(np.ones((64, 2048), np.float32), [64, 2048], cpu)
    items += fg.debug_plan([a.matmul(w.permute([1, 0]))], fuse=True, render_hip=True)["items"]
    kinds = set()
    for it in items:
        r = Rendered(it["kernel"])
        assert r.source == it["source"] and r.kind == it["class"]
        assert r.launches[0]["grid"] == tuple(it["grid"]) or len(r.launches) > 1
        assert len(r.params) == len(it["inputs"]) + (1 if it["output"] is not None else 0)
        kinds.add((r.kind, len(r.launches), r.scratch_bytes > 0))
    assert ("gemm_mfma_f32", 2, True) in kinds and ("column_reduce", 2, True) in kinds
    assert {"elementwise", "row_reduce", "serial", "block"} <= {k[0] for k in kinds}


def test_parameter_kinds_follow_the_slots(fg, cpu):
    from ferrograd_amd.hip import FG_ARG_F32, FG_ARG_I32, FG_ARG_PTR, Rendered

    # narrow() starts become i32 kernel scalars (schedule.rs:217-239).
    x = fg.Tensor.new(np.ones((6, 4), np.float32), [6, 4], cpu)
    (it,) = plan(fg, x.narrow(0, 2, 3).add(x.narrow(0, 1, 3)))
    r = Rendered(it["kernel"])
    assert r.params[0] == FG_ARG_PTR and FG_ARG_I32 in r.params and FG_ARG_F32 not in r.params
    text = it["kernel"].replace("ParamScalar i32", "ParamScalar f32")
    assert FG_ARG_F32 in Rendered(text).params


@pytest.mark.parametrize("edit,message", [
    (lambda t: t.replace("fg-kernel 1", "fg-kernel 2"), "must start with"),
    (lambda t: t.replace("Reduce f32", "Fold f32", 1), "unknown op 'Fold'"),
    (lambda t: t.replace("range:2:REDUCE", "range:2:SIDEWAYS"), "unknown axis kind"),
    (lambda t: re.sub(r"Load f32 - \d+", "Load f32 - 999", t, count=1), "is not an earlier node"),
    (lambda t: t.replace("int:784", "int:78x4"), "bad integer"),
    (lambda t: "\n".join(t.splitlines()[:-1]), "must end with the kernel's Sink"),
])
def test_malformed_kernel_text_is_rejected_by_line(fg, cpu, edit, message):
    from ferrograd_amd.hip import HipError, Rendered

    x = fg.Tensor.new(np.ones((300, 784), np.float32), [300, 784], cpu)
    w = fg.Tensor.new(np.ones((128, 784), np.float32), [128, 784], cpu)
    text = plan(fg, x.matmul(w.permute([1, 0])))[0]["kernel"]
    assert edit(text) != text
    with pytest.raises(HipError, match=re.escape(message)):
        Rendered(edit(text))


def test_float_args_cross_exactly(fg, cpu):
    from ferrograd_amd.hip import Rendered

    # 0.1 is not a dyadic rational: the f64 bit pattern must survive.
    x = fg.Tensor.new(np.ones(16, np.float32), [16], cpu)
    (it,) = plan(fg, x.mul(fg.Tensor.scalar(0.1, cpu)).add(fg.Tensor.full([16], 1e-30, cpu)))
    assert Rendered(it["kernel"]).source == it["source"]
    text = "\n".join(l for l in it["kernel"].splitlines())
    assert "float:" not in text or re.search(r"float:[0-9a-f]{16}", text)


def test_rendered_sources_compile_for_gfx950(fg, cpu):
    from ferrograd_amd.hip import Rendered, api

    import ctypes

    for name, (root, _) in programs(fg, cpu).items():
        for it in plan(fg, root):
            r = Rendered(it["kernel"])
            for l in r.launches:
                out = ctypes.c_void_p()
                rc = api().fg_hip_compile(None, r.source.encode(), l["func"].encode(), len(r.params), ctypes.byref(out))
                assert rc == 0, (name, api().fg_hip_last_error().decode())


def test_a_second_process_finds_the_cached_code_object(fg, cpu, tmp_path):
    # The cache key is the source plus every option and the hiprtc version: a
    # second process compiling the same source reuses the file, a different
    # source gets another one.
    from ferrograd_amd.hip import Rendered, code_object_path

    (it,) = plan(fg, programs(fg, cpu)["c2"][0])
    src = Rendered(it["kernel"]).source
    env = dict(os.environ, FG_KERNEL_CACHE=str(tmp_path))
    script = ("import ctypes, sys; sys.path.insert(0, %r); from ferrograd_amd.hip import api, code_object_path; "
              "src = sys.stdin.read(); out = ctypes.c_void_p(); "
              "assert api().fg_hip_compile(None, src.encode(), b'x', 3, ctypes.byref(out)) == 0; "
              "print(code_object_path(src))") % os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    run = lambda: subprocess.run([sys.executable, "-c", script], input=src, env=env, capture_output=True,  # noqa: E731
                                 text=True, check=True).stdout.strip()
    p1 = run()
    assert os.path.dirname(p1) == str(tmp_path) and os.path.getsize(p1) > 0
    st = os.stat(p1)
    assert run() == p1
    assert os.stat(p1).st_mtime_ns == st.st_mtime_ns and os.stat(p1).st_ino == st.st_ino  # hit: not rewritten
    assert len(os.listdir(tmp_path)) == 1
    assert code_object_path(src) != code_object_path(src + "\n// another source")


# ── running rendered kernels through the C-ABI ─────────────────────────────

def run_rendered(ctx, text, inputs, out_numel):
    """Load and run one rendered allocating kernel: slot 0 is the output
    (`out_numel` floats), slots 1.. take `inputs` in order, or, when `inputs`
    is a dict, the array of the slot's ParamBuffer size."""
    from ferrograd_amd.hip import Arg, Kernel, Rendered

    r = Rendered(text)
    k = Kernel(ctx, r)
    sizes = {int(m.group(1)): int(m.group(2)) for m in re.finditer(r"ParamBuffer \w+ param:(\d+):(\d+)", text)}
    assert sizes[0] == out_numel and len(r.params) == len(sizes)
    out = ctx.alloc(out_numel * 4, zero=False)
    bufs, args = [out], [Arg.ptr(out)]
    for slot in range(1, len(r.params)):
        a = np.ascontiguousarray(inputs[sizes[slot]] if isinstance(inputs, dict) else inputs[slot - 1])
        assert a.size == sizes[slot]
        p = ctx.alloc(a.nbytes, zero=False)
        ctx.h2d(p, a)
        bufs.append(p)
        args.append(Arg.ptr(p))
    k.run(args)
    got = np.empty(out_numel, np.float32)
    ctx.d2h(got, out)
    for p in bufs:
        ctx.free(p)
    return got, r


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["c1", "c2", "c3", "colsum_split", "dw_split_k", "dw_small"])
def test_rendered_kernels_run_and_match_the_oracle(fg, cpu, hip, name):
    from ferrograd_amd.hip import Context

    H = host_arrays()
    root, inputs = programs(fg, cpu)[name]
    (it,) = plan(fg, root)
    want = root.numpy().reshape(-1)  # realised on the oracle
    if inputs is None:
        inputs = {H[k].size: H[k] for k in (("gs", "hs") if name == "dw_small" else ("g", "h"))}
    got, r = run_rendered(Context.of_device(), it["kernel"], inputs, want.size)
    if name == "c2":
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        return
    if name in ("colsum_split", "dw_split_k"):
        assert r.scratch_bytes > 0 and len(r.launches) == 2
    if name == "dw_small":
        assert r.scratch_bytes == 0 and len(r.launches) == 1 and "mfma_f32_16x16x4f32" in r.source
    # Reductions and products: 1e-4 of sum |terms| against the oracle.
    f64 = {k: v.astype(np.float64) for k, v in H.items()}
    scale = {
        "c1": lambda: np.maximum(f64["x"] * 0.5 + 1.0, 0).sum(1),
        "c3": lambda: np.abs(f64["x"]) @ np.abs(f64["w"]).T + np.abs(f64["b"]),
        "colsum_split": lambda: np.abs(f64["tall"]).sum(0),
        "dw_split_k": lambda: np.abs(f64["g"]).T @ np.abs(f64["h"]),
        "dw_small": lambda: np.abs(f64["gs"]).T @ np.abs(f64["hs"]),
    }[name]().reshape(-1)
    assert rel_err_bound(got, want, scale, 1e-4) <= 1.0


@pytest.mark.gpu
def test_kernel_run_rejects_bad_arguments_before_queueing(fg, cpu, hip):
    from ferrograd_amd.hip import Arg, Context, HipError, Kernel, Rendered

    ctx = Context.of_device()
    (it,) = plan(fg, programs(fg, cpu)["c2"][0])
    k = Kernel(ctx, Rendered(it["kernel"]))
    p = ctx.alloc(4000)
    with pytest.raises(HipError, match="takes 4 arguments, got 3"):
        k.run([Arg.ptr(p)] * 3)
    with pytest.raises(HipError, match="argument 2 must be a pointer, got f32"):
        k.run([Arg.ptr(p), Arg.ptr(p), Arg.f32(1.0), Arg.ptr(p)])
    with pytest.raises(HipError, match="argument 1 is a null pointer"):
        k.run([Arg.ptr(p), Arg.ptr(None), Arg.ptr(p), Arg.ptr(p)])
    ctx.sync()
    ctx.free(p)


@pytest.mark.gpu
def test_a_damaged_cached_code_object_is_compiled_again(fg, cpu, hip):
    # A foreign file at the cache path is replaced by a fresh compile when the
    # runtime rejects it, and the kernel then runs.
    from ferrograd_amd.hip import Context, Rendered, code_object_path

    root, inputs = programs(fg, cpu)["c2"]
    (it,) = plan(fg, root)
    path = code_object_path(Rendered(it["kernel"]).source)
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "wb") as f:
        f.write(b"\x7fELF this is not a code object")
    # A context of its own: the device's context may hold this source's
    # module loaded already, and would not read the file.
    got, _ = run_rendered(Context(0), it["kernel"], inputs, 1000)
    assert np.array_equal(got, root.numpy().reshape(-1))
    assert os.path.getsize(path) > 100
