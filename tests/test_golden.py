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
    _, _, grads = mg.mlp_step_f64(f["x"], f["t"], [f[n + "_0"] for n in NAMES])
    for n, p, g in zip(NAMES, p1, grads):
        scale = np.abs(f[n + "_0"]) + 0.01 * (np.abs(g) + 1e-3)
        assert rel_err_bound(p, f[n + "_1"], scale, 1e-4) <= 1.0, n
