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
