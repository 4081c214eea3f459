"""Committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py): each is pinned to float64 arithmetic here, the
CPU oracle must reproduce it bit for bit, and the HIP path must match it to the
path's tolerances (bit-exact elementwise; 1e-4 * sum|terms| for reductions and
products)."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

from conftest import rel_err_bound

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden as mg  # noqa: E402
import f64ref  # noqa: E402  (tests/f64ref.py)

NAMES = ["w1", "b1", "w2", "b2"]


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz")) as z:  # allow_pickle=False (default)
        return {k: z[k] for k in z.files}


# ── fixtures against float64 ────────────────────────────────────────────────

def test_fixtures_match_float64():
    f = load("c1_64x64"); mg.check_c1(f, f["out"])
    f = load("c2_4096"); mg.check_c2(f, f["out"])
    f = load("c3_64"); mg.check_c3(f, f["out"])
    f = load("c4_step_b8")
    mg.check_c4(f, [f[n + "_0"] for n in NAMES], float(f["loss"][0]), [f[n + "_1"] for n in NAMES])


def test_float64_check_rejects_planted_mistakes():
    # A fixture with a dropped bias term or a transposed weight must fail the pin.
    f = load("c3_64")
    bad = (f["x"].astype(np.float64) @ f["w"].astype(np.float64).T).astype(np.float32)
    with pytest.raises(AssertionError):
        mg.check_c3(f, bad)
    bad = (f["x"].astype(np.float64) @ f["w"].astype(np.float64) + f["b"]).astype(np.float32)
    with pytest.raises(AssertionError):
        mg.check_c3(f, bad)
    g = load("c4_step_b8")
    p1 = [g[n + "_1"] for n in NAMES]
    p1[3] = p1[3] + 0.01 * 1e-2  # a bias update off by a small gradient-sized term
    with pytest.raises(AssertionError):
        mg.check_c4(g, [g[n + "_0"] for n in NAMES], float(g["loss"][0]), p1)


def loose_param_check(p0, p1_got, p1_want, grads):
    """The bound parameters were once held to: 1e-4 of |p| + lr (|g| + 1e-3)
    on p1 itself, which |p| dominates."""
    return all(mg.within(a, b, np.abs(p) + 0.01 * (np.abs(g) + 1e-3), 1e-4)
               for a, b, p, g in zip(p1_got, p1_want, p0, grads))


def planted_update(p0, grads, i, bad_grad):
    """Params after SGD with gradient i replaced by `bad_grad` (i = -1: none),
    rounded to f32 as the device's update kernel rounds them."""
    lr32 = np.float32(0.01)
    return [(p - lr32 * (bad_grad if j == i else g).astype(np.float32)).astype(np.float32)
            for j, (p, g) in enumerate(zip(p0, grads))]


def largest_weight_tile(p, T):
    """Top-left corner of the T x T tile of p whose smallest |p| is largest:
    where a bound proportional to |p| is loosest."""
    a = np.abs(p)
    corners = [(r, c) for r in range(0, a.shape[0] - T + 1, T) for c in range(0, a.shape[1] - T + 1, T)]
    return max(corners, key=lambda rc: a[rc[0]:rc[0] + T, rc[1]:rc[1] + T].min())


def forward_f64(x, t, p0):
    w1, b1, w2, b2 = (np.asarray(p, np.float64) for p in p0)
    hp = x @ w1.T + b1
    h = np.maximum(hp, 0)
    z = h @ w2.T + b2
    zs = z - z.max(1, keepdims=True)
    dz = (np.exp(zs) / np.exp(zs).sum(1, keepdims=True) - t) / x.shape[0]
    return h, dz


@pytest.mark.parametrize("plant", ["w2_transposed_tile", "w2_tile_off_0.5pct", "w1_tile_off_0.2pct",
                                   "w2_tile_lost_one_of_256_batch_terms"])
def test_effective_gradient_check_catches_what_the_parameter_bound_missed(plant):
    # Weight-gradient mistakes confined to one tile of dW, as a GEMM tile or
    # split-K partial would make them, placed where |p| is largest. Each
    # passes the bound parameters were once held to (1e-4 of |p| + lr(|g| +
    # 1e-3), on p1) and fails the effective-gradient check.
    if plant == "w2_tile_lost_one_of_256_batch_terms":
        # C4's shapes (B=256, 784 -> 128 -> 10), float64 throughout.
        r = np.random.default_rng(0)
        x, t = r.uniform(0, 1, (256, 784)), np.eye(10)[r.integers(0, 10, 256)]
        p0 = [(r.standard_normal((128, 784)) * np.sqrt(2 / 784)).astype(np.float32), np.zeros(128, np.float32),
              (r.standard_normal((10, 128)) * np.sqrt(2 / 128)).astype(np.float32), np.zeros(10, np.float32)]
    else:
        f = load("c4_step_b8")
        x, t = f["x"].astype(np.float64), f["t"].astype(np.float64)
        p0 = [f[n + "_0"] for n in NAMES]
    _, want, grads, scales = mg.mlp_step_f64(x, t, p0)
    i = 0 if plant.startswith("w1") else 2
    T = 2 if "transposed" in plant else 4
    r0, c0 = largest_weight_tile(p0[i], T)
    tile = (slice(r0, r0 + T), slice(c0, c0 + T))
    bad = grads[i].copy()
    if "transposed" in plant:
        bad[tile] = grads[i][tile].T
    elif "lost_one" in plant:
        h, dz = forward_f64(x, t, p0)
        bad[tile] = (dz[1:].T @ h[1:])[tile]
    else:
        bad[tile] *= 1.005 if "0.5pct" in plant else 1.002
    p1 = planted_update(p0, grads, i, bad)
    assert loose_param_check(p0, p1, want, grads), "the plant must pass the old parameter bound"
    worst = max(f64ref.sgd_effective_gradient_err(a, b, g, s) for a, b, g, s in zip(p0, p1, grads, scales))
    assert worst > 1.0
    # The update without a plant passes.
    assert max(f64ref.sgd_effective_gradient_err(a, b, g, s)
               for a, b, g, s in zip(p0, planted_update(p0, grads, -1, None), grads, scales)) <= 1.0


def test_f64ref_matches_the_golden_two_layer_restatement():
    # tests/f64ref.py (N layers, used by the GPU tests and bench.py) against
    # the fixture writer's own two-layer restatement: same loss, gradients
    # and condition scales.
    f = load("c4_step_b8")
    p0 = [f[n + "_0"] for n in NAMES]
    l1, n1, g1, s1 = f64ref.mlp_step_f64(f["x"], f["t"], p0)
    l2, n2, g2, s2 = mg.mlp_step_f64(f["x"], f["t"], p0)
    assert abs(l1 - l2) <= 1e-12 * abs(l2)
    for a, b in zip(n1 + g1 + s1, n2 + g2 + s2):
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-300)


def test_sampled_gradients_match_the_full_step():
    # The sampled float64 gradients that check C5 at B=8192 are the full
    # step's gradients, row for row, on a small three-layer case.
    r = np.random.default_rng(3)
    dims, B = (20, 24, 16, 10), 32
    x = r.uniform(0, 1, (B, dims[0]))
    t = np.eye(10)[r.integers(0, 10, B)]
    params = []
    for i in range(3):
        params += [r.standard_normal((dims[i + 1], dims[i])) * 0.3, r.standard_normal(dims[i + 1]) * 0.1]
    z1 = x @ params[0].T + params[1]
    z2 = np.maximum(z1, 0) @ params[2].T + params[3]
    logits = np.maximum(z2, 0) @ params[4].T + params[5]
    loss, _, grads, scales = f64ref.mlp_step_f64(x, t, params)
    rows = [np.array([0, 5, 23]), np.array([1, 2, 15])]
    loss_s, out = f64ref.mlp_step_f64_sampled(x, t, params, [z1, z2], logits, rows)
    assert abs(loss - loss_s) <= 1e-12
    for i, (sel, g, s) in out.items():
        np.testing.assert_allclose(g, grads[i][sel], rtol=1e-10, atol=1e-14)
        # Scales on exact layer inputs are at most the full step's propagated ones.
        assert np.all(s <= scales[i][sel] * (1 + 1e-12) + 1e-300)


# ── the oracle reproduces the fixtures exactly ──────────────────────────────

def test_oracle_reproduces_fixtures(fg, cpu):
    f = load("c1_64x64")
    assert np.array_equal(mg.run_c1(fg, cpu, f["x"]), f["out"])
    f = load("c2_4096")
    assert np.array_equal(mg.run_c2(fg, cpu, f["a"], f["b"], f["c"]), f["out"])
    f = load("c3_64")
    assert np.array_equal(mg.run_c3(fg, cpu, f["x"], f["w"], f["b"]), f["out"])
    f = load("c4_step_b8")
    p0, loss, p1 = mg.run_c4(fg, cpu, f["x"], f["t"])
    for n, p in zip(NAMES, p0):
        assert np.array_equal(p, f[n + "_0"]), n
    assert np.float32(loss) == f["loss"][0]
    for n, p in zip(NAMES, p1):
        assert np.array_equal(p, f[n + "_1"]), n


# ── the HIP path against the fixtures ───────────────────────────────────────

@pytest.mark.gpu
def test_hip_c2_fixture_bit_exact(fg, hip):
    f = load("c2_4096")
    got = mg.run_c2(fg, hip, f["a"], f["b"], f["c"])
    assert np.array_equal(got.view(np.uint32), f["out"].view(np.uint32))


@pytest.mark.gpu
def test_hip_c1_fixture(fg, hip):
    f = load("c1_64x64")
    got = mg.run_c1(fg, hip, f["x"])
    scale = np.maximum(f["x"].astype(np.float64) * 0.5 + 1.0, 0).sum(1)
    assert rel_err_bound(got, f["out"], scale, 1e-4) <= 1.0


@pytest.mark.gpu
def test_hip_c3_fixture(fg, hip):
    f = load("c3_64")
    got = mg.run_c3(fg, hip, f["x"], f["w"], f["b"])
    scale = np.abs(f["x"]).astype(np.float64) @ np.abs(f["w"]).T.astype(np.float64) + np.abs(f["b"])
    assert rel_err_bound(got, f["out"], scale, 1e-4) <= 1.0


@pytest.mark.gpu
def test_hip_c4_step_fixture(fg, hip):
    f = load("c4_step_b8")
    p0, loss, p1 = mg.run_c4(fg, hip, f["x"], f["t"])
    for n, p in zip(NAMES, p0):  # the init runs on the host: identical bits
        assert np.array_equal(p, f[n + "_0"]), n
    assert abs(loss - float(f["loss"][0])) <= 1e-4 * abs(float(f["loss"][0]))
    # Effective gradients against float64 (and so against the oracle's, which
    # the same check pins).
    mg.check_c4(f, p0, loss, p1)
