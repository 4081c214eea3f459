"""Tensors with an axis of extent 0.

The reference's loop nests run no iteration over such an axis
(codegen/clang.rs:164-170 renders `for (int idxN = 0; idxN < 0; idxN++)`), so
an elementwise result is empty, a sum over the empty axis is its accumulator's
initial value 0.0 and a max is -INFINITY (devectorize.rs `init_value`), and a
product whose shared axis is empty is all zeros. The oracle is pinned against
those closed forms; on HIP, an output of no element renders as a launch that
does nothing, and a reduction over an empty range keeps its initial value, at
sizes that reach the multi-workgroup classes as well as the one-workgroup
block kernels."""
from __future__ import annotations

import numpy as np
import pytest

F = np.float32


def cases(fg):
    T = fg.Tensor
    z = lambda s, d: T.new(np.zeros(s, F), list(s), d)  # noqa: E731
    return {
        "add_0x4": (lambda d: z((0, 4), d).add(z((0, 4), d)), np.zeros((0, 4), F)),
        "sum_rows_4x0": (lambda d: z((4, 0), d).sum([1]), np.zeros((4, 1), F)),
        "max_rows_4x0": (lambda d: z((4, 0), d).max([1]), np.full((4, 1), -np.inf, F)),
        "sum_cols_0x4": (lambda d: z((0, 4), d).sum([0]), np.zeros((1, 4), F)),
        "add_0x5000": (lambda d: z((0, 5000), d).add(z((0, 5000), d)), np.zeros((0, 5000), F)),
        "sum_rows_0x5000": (lambda d: z((0, 5000), d).sum([1]), np.zeros((0, 1), F)),
        "sum_cols_5000x0": (lambda d: z((5000, 0), d).sum([0]), np.zeros((1, 0), F)),
        "sum_rows_8192x0": (lambda d: z((8192, 0), d).sum([1]), np.zeros((8192, 1), F)),
        "max_rows_8192x0": (lambda d: z((8192, 0), d).max([1]), np.full((8192, 1), -np.inf, F)),
        "matmul_k0_300": (lambda d: z((300, 0), d).matmul(z((0, 300), d)), np.zeros((300, 300), F)),
        "matmul_m0": (lambda d: z((0, 64), d).matmul(z((64, 64), d)), np.zeros((0, 64), F)),
    }


def run(fg, dev, name):
    build, want = cases(fg)[name]
    t = build(dev)
    return np.asarray(t.to_vec(), F), want


@pytest.mark.parametrize("name", sorted(cases(__import__("ferrograd_amd"))))
def test_empty_axes_on_the_oracle(fg, cpu, name):
    got, want = run(fg, cpu, name)
    assert got.shape == (want.size,) and np.array_equal(got, want.reshape(-1))


def test_empty_outputs_render_as_no_op_launches(fg, cpu):
    # No output element: a launch of one workgroup that does nothing, with
    # the kernel's parameters, whatever class the shape would otherwise take
    # (these would be column and row reductions and an elementwise kernel).
    from hipcompile import compile_sources

    sources = {}
    for name in ("add_0x5000", "sum_rows_0x5000", "sum_cols_5000x0", "matmul_m0"):
        t = cases(fg)[name][0](cpu)
        items = fg.debug_plan([t], fuse=True, render_hip=True)["items"]
        empty = [it for it in items if it["class"] == "empty"]
        assert empty and all(it["grid"] == [1, 1, 1] for it in empty), name
        for it in empty:
            assert it["source"].rstrip().endswith("{}"), name
            sources[it["source"]] = it["name"]
    compile_sources(sources, limit_s=120)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(cases(__import__("ferrograd_amd"))))
def test_empty_axes_on_hip_match_the_oracle(fg, cpu, hip, name):
    print(f"empty-axis case {name}", flush=True)
    want, _ = run(fg, cpu, name)
    got, _ = run(fg, hip, name)
    assert np.array_equal(got, want)


# Ragged shapes: extents that are not multiples of the 4-wide lanes, of the
# workgroup tiles or of the MFMA tiles, at sizes above the one-workgroup
# limits. Elementwise results and maxima are bit-exact against the oracle;
# sums and products are within 1e-4 of the sum of their terms' magnitudes.
RAGGED = {
    "add_67x131": ((67, 131), (67, 131), lambda x, y: x.add(y), lambda a, b: a + b, "exact"),
    "relu_mul_4099": ((4099,), (4099,), lambda x, y: x.mul(y).relu(), lambda a, b: np.maximum(a * b, 0), "exact"),
    "max_rows_67x4099": ((67, 4099), None, lambda x, y: x.max([1]), lambda a, b: a.max(1, keepdims=True), "exact"),
    "sum_rows_67x4099": ((67, 4099), None, lambda x, y: x.sum([1]), lambda a, b: a.sum(1, keepdims=True),
                         lambda a, b: np.abs(a).sum(1, keepdims=True)),
    "sum_cols_4099x67": ((4099, 67), None, lambda x, y: x.sum([0]), lambda a, b: a.sum(0, keepdims=True),
                         lambda a, b: np.abs(a).sum(0, keepdims=True)),
    "matmul_257x131x263": ((257, 131), (131, 263), lambda x, y: x.matmul(y), lambda a, b: a @ b,
                           lambda a, b: np.abs(a) @ np.abs(b)),
    "matmul_1031x517x33": ((1031, 517), (517, 33), lambda x, y: x.matmul(y), lambda a, b: a @ b,
                           lambda a, b: np.abs(a) @ np.abs(b)),
}


def ragged_run(fg, dev, name, seed=5):
    sa, sb, op, _, _ = RAGGED[name]
    r = np.random.default_rng(seed)
    a = r.uniform(-1, 1, sa).astype(F)
    b = r.uniform(-1, 1, sb).astype(F) if sb else None
    x = fg.Tensor.new(a, list(sa), dev)
    y = fg.Tensor.new(b, list(sb), dev) if sb else None
    return a, b, np.asarray(op(x, y).to_vec(), F)


@pytest.mark.parametrize("name", sorted(RAGGED))
def test_ragged_shapes_on_the_oracle(fg, cpu, name):
    a, b, got = ragged_run(fg, cpu, name)
    _, _, _, ref, tol = RAGGED[name]
    a64, b64 = a.astype(np.float64), (b.astype(np.float64) if b is not None else None)
    want = np.asarray(ref(a64, b64)).reshape(-1)
    if tol == "exact":
        assert np.array_equal(got, np.asarray(ref(a, b), F).reshape(-1))
    else:
        assert np.all(np.abs(got - want) <= 1e-4 * np.asarray(tol(a64, b64)).reshape(-1) + 1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(RAGGED))
def test_ragged_shapes_on_hip_match_the_oracle(fg, cpu, hip, name):
    print(f"ragged case {name}", flush=True)
    a, b, want = ragged_run(fg, cpu, name)
    _, _, got = ragged_run(fg, hip, name)
    tol = RAGGED[name][4]
    if tol == "exact":
        assert np.array_equal(got, want)
    else:
        a64, b64 = a.astype(np.float64), (b.astype(np.float64) if b is not None else None)
        scale = np.asarray(tol(a64, b64)).reshape(-1)
        assert np.all(np.abs(got.astype(np.float64) - want) <= 1e-4 * scale + 1e-30)


def narrowed_empty_sum(fg, dev):
    """A narrow() of a tensor with an extent-0 axis, summed over that axis and
    scaled: the narrow's start becomes a kernel parameter (schedule.rs:
    217-239) that the index arithmetic then drops (it multiplies the zero
    stride of the empty axis)."""
    x = fg.Tensor.new(np.zeros((5, 0), F), [5, 0], dev)
    y = fg.Tensor.new(np.arange(1, 5, dtype=F).reshape(4, 1), [4, 1], dev)
    return x.narrow(0, 1, 4).sum([1]).mul(y)


def test_a_parameter_the_body_drops_stays_in_the_signature(fg, cpu):
    # The kernel is launched with every scheduled argument in slot order, so
    # its HIP signature declares the dropped start too (an unused int).
    from hipcompile import compile_sources

    items = fg.debug_plan([narrowed_empty_sum(fg, cpu)], fuse=True, render_hip=True)["items"]
    assert len(items) == 1
    it = items[0]
    assert {"i32": 1} in it["inputs"]
    sig = next(l for l in it["source"].splitlines() if "__global__" in l)
    assert sig.count("data") == len(it["inputs"]) + 1 and "int data2" in sig, sig
    compile_sources({it["source"]: it["name"]}, limit_s=120)


@pytest.mark.gpu
def test_a_parameter_the_body_drops_on_hip(fg, hip):
    # Against the closed form (a sum over the empty axis is 0.0, times y):
    # the oracle, like the reference, keys its program cache by the lowered
    # kernel, which lost the parameter, so a cached twin with one argument
    # fewer can be handed this launch and fail its argument count.
    print("narrowed empty sum", flush=True)
    for _ in range(2):  # scheduled, then replayed
        got = narrowed_empty_sum(fg, hip).to_vec()
        assert np.array_equal(np.asarray(got, F), np.zeros(4, F))
