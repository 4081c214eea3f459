"""OPT pass selection on the HIP path and the DEVICE switch.

OPT keeps the reference's grammar (src/optimize/mod.rs:85-112) and names the
HIP passes (symbolic, mfma, narrow, fuse); DEVICE picks the device a program
uses when it names none (the reference's tensor::cpu(), tensor.rs:1122-1127).
Both are read once per process, so every case runs in a child process.
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Prints, for a few programs, each planned kernel's HIP lowering class and
# whether hiprtc compiles every function of its source (no GPU needed).
PLAN_SCRIPT = r"""
import ctypes, json, re, sys
import numpy as np
sys.path.insert(0, %r)
import ferrograd_amd as fg, oracle
from ferrograd_amd.hip import api
oracle.load()
out = {"passes": fg.gpu_passes(), "default_device": fg.default_device(), "programs": {}}
r = np.random.default_rng(0)
def t(shape):
    return fg.Tensor.new(r.standard_normal(shape).astype(np.float32), list(shape), "cpu")
x, w, b = t((256, 784)), t((128, 784)), t((128,))
progs = {
    "matmul": [x.matmul(w.permute([1, 0])).add(b)],
    "narrow": [t((4096, 512)).matmul(t((10, 512)).permute([1, 0]))],
    "row_sum": [t((64, 300)).mul(t((64, 300))).add(t((64, 300))).relu().sum([1])],
    "col_max": [t((300, 64)).max([0])],
    "log_softmax": [t((32, 10)).log_softmax(1)],
}
for name, ts in progs.items():
    items = fg.debug_plan(ts, fuse=True, render_hip=True)["items"]
    rows = []
    for it in items:
        src = it["source"]
        fns = re.findall(r"extern \"C\" __global__ void (?:__launch_bounds__\(\d+\) )?(?:__attribute__\(\(.*?\)\) )?(\w+)\(", src)
        ok = True
        for fn in fns:
            h = ctypes.c_void_p()
            ok = ok and api().fg_hip_compile(None, src.encode(), fn.encode(), 8, ctypes.byref(h)) == 0
        rows.append({"class": it["class"], "compiles": ok, "functions": len(fns)})
    out["programs"][name] = rows
print(json.dumps(out))
"""


def run_child(env_extra: dict, script: str = PLAN_SCRIPT, check: bool = True):
    env = {k: v for k, v in os.environ.items() if k not in ("OPT", "DEVICE", "FG_FUSE")}
    env.update(env_extra)
    p = subprocess.run([sys.executable, "-c", script % ROOT], env=env, capture_output=True, text=True, timeout=300)
    if check:
        assert p.returncode == 0, p.stderr[-3000:]
    return p


def classes(report, prog):
    return [r["class"] for r in report["programs"][prog]]


def test_opt_unset_enables_every_gpu_pass():
    rep = json.loads(run_child({}).stdout)
    assert rep["passes"] == {"symbolic": True, "mfma": True, "narrow": True, "fuse": True, "block": True, "batch": True}
    assert rep["default_device"] == "hip"
    assert "gemm_mfma_f32" in classes(rep, "matmul")
    assert "gemm_narrow_f32" in classes(rep, "narrow")


@pytest.mark.parametrize("value", ["0", "off", "none", " none "])
def test_opt_off_disables_every_gpu_pass_and_still_lowers(value):
    rep = json.loads(run_child({"OPT": value}).stdout)
    assert rep["passes"] == {"symbolic": False, "mfma": False, "narrow": False, "fuse": False, "block": False,
                             "batch": False}
    for prog, rows in rep["programs"].items():
        for r in rows:
            assert r["class"] not in ("gemm_mfma_f32", "gemm_narrow_f32", "block"), (prog, r)
            assert r["compiles"] and r["functions"] >= 1, (prog, r)


@pytest.mark.parametrize("value", ["1", "on", "all", ""])
def test_opt_all_spellings(value):
    rep = json.loads(run_child({"OPT": value}).stdout)
    assert all(rep["passes"].values())


def test_opt_list_selects_named_passes_and_ignores_cpu_pass_names():
    # "upcast" and "unroll" are the CPU backend's passes: ignored by the HIP
    # path, as the reference ignores names it does not know.
    rep = json.loads(run_child({"OPT": "symbolic, mfma,upcast,unroll,bogus"}).stdout)
    assert rep["passes"] == {"symbolic": True, "mfma": True, "narrow": False, "fuse": False, "block": False,
                             "batch": False}
    assert "gemm_mfma_f32" in classes(rep, "matmul")
    # Without the narrow pass the 10-wide product is no longer a narrow kernel.
    assert "gemm_narrow_f32" not in classes(rep, "narrow")
    for rows in rep["programs"].values():
        assert all(r["compiles"] for r in rows)


def test_opt_narrow_without_mfma():
    rep = json.loads(run_child({"OPT": "narrow"}).stdout)
    assert rep["passes"] == {"symbolic": False, "mfma": False, "narrow": True, "fuse": False, "block": False,
                             "batch": False}
    assert "gemm_narrow_f32" in classes(rep, "narrow")
    assert "gemm_mfma_f32" not in classes(rep, "matmul")


def test_fuse_pass_splits_kernels_like_the_reference_partition():
    fused = json.loads(run_child({}).stdout)
    unfused = json.loads(run_child({"OPT": "symbolic,mfma,narrow"}).stdout)
    env_off = json.loads(run_child({"FG_FUSE": "0"}).stdout)
    assert unfused["passes"]["fuse"] is False and env_off["passes"]["fuse"] is False
    # debug_plan(fuse=True) plans with the HIP fusions whatever the device's
    # switch says; the switch itself is what the HIP device reads.
    assert len(fused["programs"]["row_sum"]) == len(unfused["programs"]["row_sum"])


def test_device_switch():
    assert json.loads(run_child({"DEVICE": "cpu"}).stdout)["default_device"] == "cpu"
    assert json.loads(run_child({"DEVICE": "hip"}).stdout)["default_device"] == "hip"
    p = run_child({"DEVICE": "tpu"}, check=False)
    assert p.returncode != 0 and "DEVICE must be 'hip' or 'cpu'; got 'tpu'" in p.stderr


DEFAULT_DEVICE_SCRIPT = r"""
import sys
import numpy as np
sys.path.insert(0, %r)
import ferrograd_amd as fg, oracle
oracle.load()
a = fg.Tensor.new(np.arange(6, dtype=np.float32), [2, 3])
print(a.device, a.add(a).sum([1]).numpy().tolist())
"""


def test_programs_that_name_no_device_follow_device_cpu():
    p = run_child({"DEVICE": "cpu"}, script=DEFAULT_DEVICE_SCRIPT)
    assert p.stdout.split()[0] == "cpu" and "[[6.0], [24.0]]" in p.stdout


# The HIP device with every pass off against the oracle: the generic lowering
# classes carry matmuls, narrow products and a train step.
PARITY_SCRIPT = r"""
import json, sys
import numpy as np
sys.path.insert(0, %r)
sys.path.insert(0, %r + "/tests")
import ferrograd_amd as fg, oracle
from ferrograd_amd.mlp import mlp_setup
oracle.load()
rep = {"passes": fg.gpu_passes()}
r = np.random.default_rng(3)
xs, ws, bs = (r.standard_normal(s).astype(np.float32) for s in ((96, 200), (40, 200), (40,)))
zs, vs = (r.standard_normal(s).astype(np.float32) for s in ((512, 300), (10, 300)))
def run(dev):
    x, w, b = (fg.Tensor.new(v, list(v.shape), dev) for v in (xs, ws, bs))
    z, v = (fg.Tensor.new(a, list(a.shape), dev) for a in (zs, vs))
    return [x.matmul(w.permute([1, 0])).add(b).relu().numpy(), z.relu().matmul(v.permute([1, 0])).numpy(),
            x.mul(x).sum([1]).numpy().reshape(-1), x.max([0]).numpy().reshape(-1)]
hip, cpu = run("hip"), run("cpu")
def scale(dev_x, dev_w):
    return np.abs(dev_x.astype(np.float64)) @ np.abs(dev_w.astype(np.float64)).T
bounds = [1e-4 * (scale(xs, ws) + np.abs(bs)) + 1e-30, 1e-4 * scale(np.maximum(zs, 0), vs) + 1e-30,
          1e-4 * (xs.astype(np.float64) ** 2).sum(1) + 1e-30, None]
rep["err_over_bound"] = [float(np.max(np.abs(h.astype(np.float64) - c) / bd)) for h, c, bd in zip(hip, cpu, bounds) if bd is not None]
rep["max_bit_exact"] = bool(np.array_equal(hip[3], cpu[3]))
hs, _ = mlp_setup(fg, "hip", batch=64, dims=(784, 32, 10))
cs, _ = mlp_setup(fg, "cpu", batch=64, dims=(784, 32, 10))
lh = [hs() for _ in range(3)]
lc = [cs() for _ in range(3)]
rep["loss_rel"] = float(max(abs(a - b) / abs(b) for a, b in zip(lh, lc)))
rep["stats"] = fg.stats()["kernels_launched"]
print(json.dumps(rep))
"""


@pytest.mark.gpu
@pytest.mark.parametrize("opt", ["0", "symbolic,fuse", "symbolic,mfma,narrow,block,batch"])
def test_hip_with_gpu_passes_off_matches_oracle(opt):
    # The third leaves out only the schedule-time fusion: the reference
    # partition, whose materialised relu masks are small bool kernels that
    # run (and batch) as one-workgroup block kernels.
    env = {k: v for k, v in os.environ.items() if k not in ("OPT", "DEVICE", "FG_FUSE")}
    env["OPT"] = opt
    print(f"OPT={opt}: child process", flush=True)
    p = subprocess.run([sys.executable, "-u", "-c", PARITY_SCRIPT % (ROOT, ROOT)], env=env, capture_output=True,
                       text=True, timeout=110)
    assert p.returncode == 0, p.stderr[-3000:]
    rep = json.loads(p.stdout.strip().splitlines()[-1])
    names = opt.split(",")
    assert all(rep["passes"][k] == (k in names) for k in ("fuse", "mfma", "narrow", "block", "batch"))
    assert max(rep["err_over_bound"]) <= 1.0, rep
    assert rep["max_bit_exact"], rep
    assert rep["loss_rel"] <= 1e-4, rep
