"""Small kernels as one 1024-thread workgroup (the `block` class) and runs of
them batched into one launch (the `batch` pass).

A block kernel's body is a device function; alone it is launched as one
workgroup, in a batch several bodies run back to back behind workgroup
barriers. The values are the oracle's within the reduction tolerance
(1e-4·Σ|terms|; max and elementwise bit for bit), and a batched sequence
gives the same bits as the same kernels launched one by one.
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def plan(fg, roots):
    return fg.debug_plan(roots, fuse=True, render_hip=True)["items"]


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


# (name, builder over (device, arrays), arrays, expected base class)
CASES = {
    "row_sum_L128": (lambda fg, d, a: fg.Tensor.new(a[0], list(a[0].shape), d).sum([1]), [rnd((40, 128), 1)], "row_reduce"),
    "row_max_L64": (lambda fg, d, a: fg.Tensor.new(a[0], list(a[0].shape), d).max([1]), [rnd((100, 64), 2)], "row_reduce"),
    "row_sum_L1000_one_output": (lambda fg, d, a: fg.Tensor.new(a[0], list(a[0].shape), d).sum([0]),
                                 [rnd((1000,), 3)], "row_reduce"),
    "col_sum_T64": (lambda fg, d, a: fg.Tensor.new(a[0], list(a[0].shape), d).sum([0]), [rnd((300, 64), 4)], "column_reduce"),
    "col_sum_T1000": (lambda fg, d, a: fg.Tensor.new(a[0], list(a[0].shape), d).sum([0]), [rnd((64, 1000), 5)],
                      "column_reduce"),
    "col_sum_T10_relu_product": (lambda fg, d, a: fg.Tensor.new(a[0], list(a[0].shape), d).relu()
                                 .mul(fg.Tensor.new(a[1], list(a[1].shape), d)).sum([0]),
                                 [rnd((256, 10), 6), rnd((256, 10), 7)], "column_reduce"),
    "log_softmax_32x10": (lambda fg, d, a: fg.Tensor.new(a[0], list(a[0].shape), d).log_softmax(1), [rnd((32, 10), 8)],
                          None),
    "elementwise_1000": (lambda fg, d, a: fg.Tensor.new(a[0], [1000], d).mul(fg.Tensor.new(a[1], [1000], d)).relu(),
                         [rnd((1000,), 9), rnd((1000,), 10)], "elementwise"),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_small_kernels_plan_as_one_workgroup(fg, cpu, name):
    build, arrays, base = CASES[name]
    items = plan(fg, [build(fg, cpu, arrays)])
    assert all(it["class"] == "block" for it in items), [(it["class"], it["base_class"]) for it in items]
    assert all(it["grid"] == [1, 1, 1] and it["block"] == [1024, 1, 1] for it in items)
    if base:
        assert items[-1]["base_class"] == base
    assert all("_body(" in it["source"] and "__restrict__" not in it["source"].split("_body(")[1].split(")")[0]
               for it in items)


def test_kernels_past_the_workgroup_limits_keep_their_class(fg, cpu):
    # More than 4096 outputs, a reduction longer than 1024, or more than 2^16
    # terms folded in all (64 per thread): the ordinary multi-workgroup classes.
    big_out = fg.Tensor.new(np.ones((5000,), np.float32), [5000], cpu).relu()
    long_red = fg.Tensor.new(np.ones((8, 2048), np.float32), [8, 2048], cpu).sum([1])
    much_work = fg.Tensor.new(np.ones((512, 256), np.float32), [512, 256], cpu).sum([0])
    for t, cls in ((big_out, "elementwise"), (long_red, "row_reduce"), (much_work, "column_reduce")):
        (it,) = plan(fg, [t])
        assert it["class"] == cls and it["base_class"] == cls


def compile_all(src):
    import ctypes
    import re

    from ferrograd_amd.hip import api

    for fn in re.findall(r"extern \"C\" __global__ void __launch_bounds__\(\d+\) (\w+)\(", src):
        h = ctypes.c_void_p()
        assert api().fg_hip_compile(None, src.encode(), fn.encode(), 16, ctypes.byref(h)) == 0, api().fg_hip_last_error()


def test_block_sources_compile(fg, cpu):
    for name, (build, arrays, _) in CASES.items():
        for it in plan(fg, [build(fg, cpu, arrays)]):
            compile_all(it["source"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(CASES))
def test_block_kernels_match_the_oracle(fg, cpu, hip, name):
    build, arrays, _ = CASES[name]
    print(f"block case {name}", flush=True)
    got = build(fg, hip, arrays).numpy().astype(np.float64)
    want = build(fg, cpu, arrays).numpy().astype(np.float64)
    if name.startswith(("row_max", "elementwise")):
        assert np.array_equal(got, want)
        return
    a = arrays[0].astype(np.float64)
    if name == "col_sum_T10_relu_product":
        scale = (np.maximum(a, 0) * np.abs(arrays[1])).sum(0)
    elif name.startswith("col_sum") or name == "row_sum_L1000_one_output":
        scale = np.abs(a).sum(0)
    elif name.startswith("row_sum"):
        scale = np.abs(a).sum(1)
    else:  # log_softmax: max-shifted log of a 10-term sum of exponentials
        scale = np.abs(want) + np.log(np.exp(a - a.max(1, keepdims=True)).sum(1, keepdims=True)) + 1.0
    assert np.all(np.abs(got - want).reshape(-1) <= 1e-4 * np.asarray(scale).reshape(-1) + 1e-30)


# C4-sized train steps in a child process with the given OPT: losses and every
# parameter, the launches of one Python-driven step and of a native-loop step
# seen by the launch profiler.
STEPS_SCRIPT = r"""
import json, sys
import numpy as np
sys.path.insert(0, %r)
import ferrograd_amd as fg
from ferrograd_amd.hip import Context
from ferrograd_amd.mlp import Mlp, synthetic_batch, train_step, train_steps_native
fg.reset_init_seed(42)
model = Mlp((784, 128, 10), "hip")
opt = fg.Sgd(model.parameters(), 0.01)
xs, ts = synthetic_batch(256, 784, 10, 7, 8)
x = fg.Tensor.new(xs, list(xs.shape), "hip")
t = fg.Tensor.new(ts, list(ts.shape), "hip")
losses = [train_step(model, opt, x, t).to_vec()[0] for _ in range(4)]
ctx = Context.of_device()
ctx.profile_read()
ctx.profile(True)
losses += [train_step(model, opt, x, t).to_vec()[0]]
fg.synchronize()
ctx.profile(False)
launches = len(ctx.profile_read())
losses += train_steps_native(model, opt, x, t, 6)
def native_kernels(steps):
    fg.synchronize()
    ctx.profile_read()
    ctx.profile(True)
    out = train_steps_native(model, opt, x, t, steps)
    fg.synchronize()
    ctx.profile(False)
    return out, [p["kernel"] for p in ctx.profile_read()]
# A call's first steps launch outside the step capture; the difference of two
# calls counts captured steps alone.
l1, n1 = native_kernels(5)
l5, n5 = native_kernels(9)
losses += l1 + l5
native = n1 + n5
print(json.dumps({"passes": fg.gpu_passes(), "losses": losses, "launches": launches,
                  "native_launches": (len(n5) - len(n1)) / 4, "native_readback_kernels": native.count("fg_readback"),
                  "params": [p.numpy().tolist() for p in model.parameters()]}))
"""


def run_steps(opt, extra_env=None):
    env = {k: v for k, v in os.environ.items() if k != "OPT"}
    env.update(extra_env or {})
    if opt is not None:
        env["OPT"] = opt
    print(f"C4 steps with OPT={opt}", flush=True)
    p = subprocess.run([sys.executable, "-u", "-c", STEPS_SCRIPT % ROOT], env=env, capture_output=True, text=True,
                       timeout=110)
    assert p.returncode == 0, p.stderr[-3000:]
    return json.loads(p.stdout.strip().splitlines()[-1])


@pytest.mark.gpu
def test_batched_launches_give_the_same_bits_as_one_by_one(fg, hip):
    batched = run_steps(None)
    single = run_steps("symbolic,mfma,narrow,fuse,block")
    assert batched["passes"]["batch"] and not single["passes"]["batch"]
    assert batched["losses"] == single["losses"]
    for a, b in zip(batched["params"], single["params"]):
        assert np.array_equal(np.asarray(a, np.float32), np.asarray(b, np.float32))
    # The C4 update plan's class-axis kernels became one launch, b1's
    # gradient moved past dW2's (no shared buffer) to join b2's in another, and
    # the loss plan's four kernels one more: 7 launches fewer.
    assert batched["launches"] <= single["launches"] - 7, (batched["launches"], single["launches"])
    # In the native loop the loss read-back is the last stage of the step's
    # last batch, not a kernel of its own.
    assert batched["native_readback_kernels"] == 0 and single["native_readback_kernels"] > 0
    # Seven kernels per step (one-pass small GEMMs, two batches), the two
    # weight-gradient GEMMs (independent, the same workgroup size) as one
    # paired launch: six.
    assert batched["native_launches"] <= 6, batched["native_launches"]
    assert single["native_launches"] >= 7, single["native_launches"]


@pytest.mark.gpu
def test_direct_queue_gives_the_same_bits(fg, hip):
    # The native loop's captured steps dispatched as AQL packets into the
    # context's own HSA queue (the default) against hipModuleLaunchKernel
    # (FG_AQL=0): the same losses and parameters, bit for bit.
    aql = run_steps(None)
    hip_launches = run_steps(None, {"FG_AQL": "0"})
    assert aql["losses"] == hip_launches["losses"]
    for a, b in zip(aql["params"], hip_launches["params"]):
        assert np.array_equal(np.asarray(a, np.float32), np.asarray(b, np.float32))


@pytest.mark.gpu
def test_small_gemms_beside_a_batch_give_the_same_bits(fg, hip):
    # The C4 step's last launch runs the paired weight-gradient GEMMs beside
    # the batch of bias updates, the loss and its read-back (render_hbatch):
    # five launches per captured step, and the same losses and parameters,
    # bit for bit, as with the two launched apart.
    merged = run_steps(None)
    apart = run_steps(None, {"FG_HBATCH": "0"})
    assert merged["losses"] == apart["losses"]
    for a, b in zip(merged["params"], apart["params"]):
        assert np.array_equal(np.asarray(a, np.float32), np.asarray(b, np.float32))
    assert merged["native_readback_kernels"] == 0 and apart["native_readback_kernels"] == 0
    assert merged["native_launches"] <= 5 and apart["native_launches"] == merged["native_launches"] + 1, (
        merged["native_launches"], apart["native_launches"])


def test_reference_partition_small_kernels_compile_as_blocks(fg, cpu):
    # Without the schedule-time fusions the relu masks are materialised as
    # bool buffers: small ones become block kernels with a bool output.
    from ferrograd_amd.mlp import Mlp, synthetic_batch

    fg.reset_init_seed(42)
    m = Mlp((64, 32, 10), cpu)
    xs, ts = synthetic_batch(16, 64, 10, 1, 2)
    loss = m.forward(fg.Tensor.new(xs, list(xs.shape), cpu)).cross_entropy(fg.Tensor.new(ts, list(ts.shape), cpu))
    loss.backward()
    params = m.parameters()
    for p in params:
        p.assign(p.detach().sub(p.grad().mul(fg.Tensor.scalar(0.01, cpu))))
    items = fg.debug_plan(params + [loss], fuse=False, render_hip=True)["items"]
    blocks = [it for it in items if it["class"] == "block"]
    assert blocks and any("void " in it["source"] and "bool* data0" in it["source"] for it in blocks)
    for it in items:
        compile_all(it["source"])


def sixteen_roots(fg, dev, seed=11):
    """16 roots a*b + c*d + e over f32[8], each its own block kernel with 6
    arguments (output + five inputs): 96 arguments for a run of 16."""
    r = np.random.default_rng(seed)
    arrays = [[r.uniform(-1, 1, 8).astype(np.float32) for _ in range(5)] for _ in range(16)]
    roots = []
    for a, b, c, d, e in arrays:
        t = [fg.Tensor.new(v, [8], dev) for v in (a, b, c, d, e)]
        roots.append(t[0].mul(t[1]).add(t[2].mul(t[3])).add(t[4]))
    want = [(a * b + c * d) + e for a, b, c, d, e in arrays]  # float32, each op rounded once
    return roots, want


def test_batch_runs_stay_within_the_launch_argument_limit(fg, cpu):
    # A batch launch passes every stage's arguments, and a launch takes at
    # most 64 (FG_MAX_LAUNCH_ARGS): the 16 consecutive block kernels split
    # into runs of at most 10 six-argument kernels.
    roots, _ = sixteen_roots(fg, cpu)
    p = fg.debug_plan(roots, fuse=True, render_hip=True)
    items = p["items"]
    assert len(items) == 16 and all(it["class"] == "block" for it in items)
    nargs = [len(it["inputs"]) + 1 for it in items]
    assert nargs == [6] * 16
    runs = p["batches"]
    assert runs == [[0, 10], [10, 6]], runs
    for first, n in runs:
        assert sum(nargs[first:first + n]) <= 64


def test_batch_runs_split_after_sixteen_kernels(fg, cpu):
    # Two-argument kernels (relu of one input): the 16-stage cap splits a run
    # of 20 before the argument limit does.
    r = np.random.default_rng(12)
    roots = [fg.Tensor.new(r.uniform(-1, 1, 8).astype(np.float32), [8], cpu).relu() for _ in range(20)]
    p = fg.debug_plan(roots, fuse=True, render_hip=True)
    assert p["batches"] == [[0, 16], [16, 4]], p["batches"]


@pytest.mark.gpu
def test_sixteen_block_roots_replayed_twice(fg, hip):
    # The same 16-root plan realised three times: the first realise records
    # the plan, the second replays it with its kernels batched, the third
    # replays the recorded graph. Every result bit for bit against float32.
    print("sixteen block roots, replayed", flush=True)
    for rep in range(3):
        roots, want = sixteen_roots(fg, hip, seed=20 + rep)
        fg.Tensor.realize_many(roots)
        for t, w in zip(roots, want):
            assert np.array_equal(t.numpy().reshape(8), w), rep


def test_c4_batches_keep_stage_outputs_in_lds_and_compile(fg, cpu):
    # The C4 step's runs of block kernels as batches: every stage output of
    # the softmax run is one stage's full, not in-place, output, so all six
    # stay in LDS and reach their buffers after the last stage; the batch
    # kernels compile for gfx950.
    from hipcompile import compile_sources
    from ferrograd_amd.mlp import Mlp, synthetic_batch

    fg.reset_init_seed(42)
    m = Mlp((784, 128, 10), cpu)
    opt = fg.Sgd(m.parameters(), 0.01)
    xs, ts = synthetic_batch(256, 784, 10, 7, 8)
    x = fg.Tensor.new(xs, list(xs.shape), cpu)
    t = fg.Tensor.new(ts, list(ts.shape), cpu)
    loss = m.forward(x).cross_entropy(t)
    opt.zero_grad()
    loss.backward()
    opt.step()
    loss.to_vec()
    loss = m.forward(x).cross_entropy(t)
    opt.zero_grad()
    loss.backward()
    ps = m.parameters()
    for p in ps:
        p.assign(p.detach().sub(p.grad().mul(fg.Tensor.scalar(0.01, cpu))))
    plan = fg.debug_plan(ps + [loss], fuse=True, render_hip=True)
    bks = plan["batch_kernels"]
    assert len(bks) == len(plan["batches"]) >= 2
    first = bks[0]
    assert first["forwarded"] == plan["batches"][0][1] == 6
    src = first["source"]
    assert src.count("__shared__ __attribute__((aligned(16))) float fg_fwd") == 6
    assert src.count("] = fg_fwd") == 6  # each array copied to its buffer once, after the last stage
    compile_sources({b["source"]: b["name"] for b in bks}, limit_s=120)


def test_batch_forwarding_skips_in_place_and_partial_outputs(fg, cpu):
    # An in-place SGD-style update reads its destination: its output stays in
    # its buffer, and later stages read the buffer.
    r = np.random.default_rng(4)
    w = fg.Tensor.new(r.uniform(-1, 1, (8, 8)).astype(np.float32), [8, 8], cpu)
    g = fg.Tensor.new(r.uniform(-1, 1, (8, 8)).astype(np.float32), [8, 8], cpu)
    h = g.mul(g)
    w.assign(w.sub(h.mul(fg.Tensor.scalar(0.5, cpu))))
    plan = fg.debug_plan([h, w], fuse=True, render_hip=True)
    assert [it["class"] for it in plan["items"]] == ["block", "block"] and plan["batches"] == [[0, 2]]
    bk = plan["batch_kernels"][0]
    src = bk["source"][bk["source"].index('extern "C"'):]
    # h, a fresh full output, is forwarded and read by the update from LDS;
    # w's in-place update (its output is argument 2) writes its buffer.
    assert bk["forwarded"] == 1
    assert "_blk_body(fg_fwd0, a1);" in src and "_blk_body(a2, fg_fwd0, a4);" in src
    assert "a0[i] = fg_fwd0[i]" in src and "a2[i] =" not in src


def two_products(fg, dev, dependent=False, seed=21):
    """y1 = a·bᵀ and y2 = c·dᵀ (right operands given as transposed views, as
    Linear does, so each product is one GEMM kernel; K 96 for both, so both
    run two-wave workgroups); with `dependent`, y2 = y1·dᵀ instead."""
    r = np.random.default_rng(seed)
    shapes = ((64, 96), (48, 96), (64, 96), (64, 48 if dependent else 96))
    a, b, c, d = (r.uniform(-1, 1, s).astype(np.float32) for s in shapes)
    ta, tb, tc, td = (fg.Tensor.new(v, list(v.shape), dev) for v in (a, b, c, d))
    y1 = ta.matmul(tb.permute([1, 0]))
    y2 = (y1 if dependent else tc).matmul(td.permute([1, 0]))
    return (a, b.T, c, d.T), y1, y2


def test_independent_small_gemms_pair_into_one_launch(fg, cpu):
    # Two independent one-pass small GEMMs with the same workgroup size, next
    # to each other in a sequence: one launch whose first workgroups run the
    # first product's body and the rest the second's. Each body keeps its own
    # name (a regression: both once carried the unrenamed placeholder, and
    # the launch ran the first body twice, over the second's smaller buffers).
    from hipcompile import compile_sources

    _, y1, y2 = two_products(fg, cpu)
    p = fg.debug_plan([y1, y2], fuse=True, render_hip=True)
    items = p["items"]
    gemms = [i for i, it in enumerate(items) if it["class"] == "gemm_mfma_f32"]
    assert len(gemms) == 2 and gemms[1] == gemms[0] + 1
    assert [q["first"] for q in p["pairs"]] == [gemms[0]]
    pair = p["pairs"][0]
    src = pair["source"]
    n1, n2 = (items[i]["name"] for i in gemms)
    assert n1 != n2 and src.count(n1 + "_hb(") == 2 and src.count(n2 + "_hb(") == 2
    g1 = items[gemms[0]]["grid"][0]
    assert f"if (blockIdx.x < {g1}u) {n1}_hb(" in src and f"else {n2}_hb(" in src and f"blockIdx.x - {g1}u);" in src
    assert pair["grid"] == g1 + items[gemms[1]]["grid"][0]
    assert "FGKERNELNAME" not in src
    compile_sources({src: pair["name"]}, limit_s=120)


def test_dependent_gemms_do_not_pair(fg, cpu):
    _, y1, y2 = two_products(fg, cpu, dependent=True)
    p = fg.debug_plan([y1, y2], fuse=True, render_hip=True)
    assert p["pairs"] == []


@pytest.mark.gpu
def test_paired_small_gemms_on_hip(fg, cpu, hip):
    # The two products realised together four times (recorded, replayed with
    # the pair, then with graphs on recorded as a graph and replayed through
    # it), each time against the oracle within 1e-4 of sum|terms|.
    from conftest import graphs_on

    print("paired small gemms", flush=True)
    for rep in range(4):
        (a, b, c, d), y1, y2 = two_products(fg, hip, seed=30 + rep)
        with graphs_on(fg, 2 if rep >= 2 else 0):
            fg.Tensor.realize_many([y1, y2])
        for y, (l, r) in ((y1, (a, b)), (y2, (c, d))):
            want = l.astype(np.float64) @ r.astype(np.float64)
            scale = np.abs(l.astype(np.float64)) @ np.abs(r.astype(np.float64))
            got = y.numpy().astype(np.float64).reshape(want.shape)
            assert np.all(np.abs(got - want) <= 1e-4 * scale), rep


def test_batch_barriers_only_between_dependent_stages(fg, cpu):
    # C4's softmax batch: the fifth stage reads only an input of the batch,
    # so no barrier separates it from the fourth; every other stage reads its
    # predecessor's output. One more barrier precedes the copies to the
    # buffers.
    from ferrograd_amd.mlp import Mlp, synthetic_batch

    fg.reset_init_seed(42)
    m = Mlp((784, 128, 10), cpu)
    xs, ts = synthetic_batch(256, 784, 10, 7, 8)
    loss = m.forward(fg.Tensor.new(xs, list(xs.shape), cpu)).cross_entropy(fg.Tensor.new(ts, list(ts.shape), cpu))
    loss.backward()
    ps = m.parameters()
    for p in ps:
        p.assign(p.detach().sub(p.grad().mul(fg.Tensor.scalar(0.01, cpu))))
    plan = fg.debug_plan(ps + [loss], fuse=True, render_hip=True)
    src = plan["batch_kernels"][0]["source"]
    body = src[src.index('extern "C"'):]
    assert plan["batches"][0][1] == 6 and body.count("__syncthreads();") == 5


def test_batch_stages_sharing_a_body_keep_their_barriers(fg, cpu):
    # Sixteen roots of one structure: every stage is the same body function,
    # whose static LDS the next call would reuse, so even independent stages
    # stay behind barriers.
    roots, _ = sixteen_roots(fg, cpu)
    plan = fg.debug_plan(roots, fuse=True, render_hip=True)
    for (first, n), bk in zip(plan["batches"], plan["batch_kernels"]):
        body = bk["source"][bk["source"].index('extern "C"'):]
        assert body.count("__syncthreads();") == (n - 1) + (1 if bk["forwarded"] else 0)


def gemm_beside_blocks(fg, dev, seed=0, dependent=False):
    """A C4-sized one-pass small GEMM, y = a·bᵀ ([256, 784]·[128, 784]ᵀ), and
    two small reductions that become block kernels: of independent inputs,
    or (dependent) of y's first rows."""
    r = np.random.default_rng(seed)
    ah, bh = r.standard_normal((256, 784)).astype(np.float32), r.standard_normal((128, 784)).astype(np.float32)
    ch, dh = r.standard_normal((8, 16)).astype(np.float32), r.standard_normal((8, 16)).astype(np.float32)
    a, b = fg.Tensor.new(ah, [256, 784], dev), fg.Tensor.new(bh, [128, 784], dev)
    c, d = fg.Tensor.new(ch, [8, 16], dev), fg.Tensor.new(dh, [8, 16], dev)
    y = a.matmul(b.permute([1, 0]))
    if dependent:
        c = y.narrow(0, 0, 8).narrow(1, 0, 16)
    s1 = c.sum([1])
    s2 = d.mul(fg.Tensor.scalar(2.0, dev)).max([1])
    return (ah, bh, ch, dh), y, s1, s2


def test_small_gemm_runs_beside_an_independent_batch(fg, cpu):
    # A one-pass small GEMM next to a batch of block kernels it shares no
    # buffer with: one launch of 1024-thread workgroups, the first running
    # the batch and the others the GEMM's tiles, whose waves past the GEMM's
    # own 832 threads end at once.
    from hipcompile import compile_sources

    _, y, s1, s2 = gemm_beside_blocks(fg, cpu)
    p = fg.debug_plan([y, s1, s2], fuse=True, render_hip=True)
    items = p["items"]
    assert [it["class"] for it in items] == ["gemm_mfma_f32", "block", "block"]
    assert p["batches"] == [[1, 2]] and len(p["hbatches"]) == 1
    h = p["hbatches"][0]
    assert h["hb"] == [0] and h["batch"] == 0
    assert h["grid"] == 1 + items[0]["grid"][0]
    src = h["source"]
    gemm = items[0]["name"]
    assert "__launch_bounds__(1024)" in src and f"if (threadIdx.x < {items[0]['block'][0]}u) {gemm}_hb(" in src
    assert "if (blockIdx.x != 0u)" in src and src.count(gemm + "_hb(") == 2
    for it in items[1:]:
        assert it["name"] + "_body(" in src
    compile_sources({src: h["name"]}, limit_s=120)


def test_small_gemm_does_not_run_beside_a_batch_that_reads_it(fg, cpu):
    _, y, s1, s2 = gemm_beside_blocks(fg, cpu, dependent=True)
    p = fg.debug_plan([y, s1, s2], fuse=True, render_hip=True)
    assert p["hbatches"] == []


@pytest.mark.gpu
def test_small_gemm_beside_a_batch_on_hip(fg, hip):
    # Realised together four times (recorded, replayed as the merged launch,
    # then with graphs on recorded as a graph and replayed through it): the
    # product within 1e-4 of sum|terms| of float64, the sum likewise, and the
    # max bit for bit.
    from conftest import graphs_on

    print("small gemm beside a batch", flush=True)
    for rep in range(4):
        (ah, bh, ch, dh), y, s1, s2 = gemm_beside_blocks(fg, hip, seed=40 + rep)
        with graphs_on(fg, 2 if rep >= 2 else 0):
            fg.Tensor.realize_many([y, s1, s2])
        a64, b64 = ah.astype(np.float64), bh.astype(np.float64)
        got = y.numpy().astype(np.float64).reshape(256, 128)
        assert np.all(np.abs(got - a64 @ b64.T) <= 1e-4 * (np.abs(a64) @ np.abs(b64).T)), rep
        c64 = ch.astype(np.float64)
        assert np.all(np.abs(s1.numpy().reshape(8) - c64.sum(1)) <= 1e-4 * np.abs(c64).sum(1)), rep
        assert np.array_equal(s2.numpy().reshape(8), (dh * np.float32(2.0)).max(1)), rep
