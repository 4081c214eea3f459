"""gfx950 lowering and HIP codegen, checked without a GPU: each benchmark
config's kernels are classified as expected and hiprtc compiles them for
gfx950 (compile-only: fg_hip_compile with a NULL context)."""
import ctypes
import re

import numpy as np
import pytest


def hip_plan(fg, roots):
    return fg.debug_plan(roots, fuse=True, render_hip=True)["items"]


def compile_only(fg, source: str, name: str):
    from ferrograd_amd.hip import api

    out = ctypes.c_void_p()
    rc = api().fg_hip_compile(None, source.encode(), name.encode(), 0, ctypes.byref(out))
    assert rc == 0, api().fg_hip_last_error().decode()


def test_c2_is_one_vectorised_elementwise_kernel(fg, cpu):
    a, b, c = (fg.Tensor.new(np.ones(1 << 16, np.float32), [1 << 16], cpu) for _ in range(3))
    items = hip_plan(fg, [a.mul(b).add(c).relu()])
    assert [it["class"] for it in items] == ["elementwise"]
    src = items[0]["source"]
    assert src.count("__builtin_nontemporal_load((const fg_f4*)") == 3 and "*(float4*)" in src
    compile_only(fg, src, items[0]["name"])


def test_large_elementwise_output_uses_streaming_stores(fg, cpu):
    # >= 128 MiB of output (2^25 f32) is written past the caches; smaller outputs are not.
    n = 1 << 25
    a = fg.Tensor.new(np.ones(n, np.float32), [n], cpu)
    src = hip_plan(fg, [a.mul(a).relu()])[0]["source"]
    assert "__builtin_nontemporal_store(vout, (fg_f4*)" in src and "*(float4*)" not in src
    compile_only(fg, src, hip_plan(fg, [a.mul(a).relu()])[0]["name"])
    small = fg.Tensor.new(np.ones(n // 2, np.float32), [n // 2], cpu)
    assert "__builtin_nontemporal_store" not in hip_plan(fg, [small.mul(small).relu()])[0]["source"]


def test_c1_is_one_row_reduce_with_dpp_tree(fg, cpu):
    x = fg.Tensor.new(np.ones((64, 4096), np.float32), [64, 4096], cpu)
    y = x.mul(fg.Tensor.scalar(0.5, cpu)).add(fg.Tensor.scalar(1.0, cpu)).relu().sum([1])
    items = hip_plan(fg, [y])
    assert [it["class"] for it in items] == ["row_reduce"]
    src = items[0]["source"]
    assert "FG_DPP(racc, 0xB1)" in src and "fg_x32_f" in src and "__syncthreads" in src
    compile_only(fg, src, items[0]["name"])


def test_c3_is_one_mfma_gemm_reading_w_directly(fg, cpu):
    # matmul's permute(...).contiguous() of Wᵀ is a copy of W in W's own order
    # (tensor.rs:771-777): the GEMM reads W itself; the reference partition
    # keeps the copy kernel.
    x = fg.Tensor.new(np.ones((512, 512), np.float32), [512, 512], cpu)
    w = fg.Tensor.new(np.ones((512, 512), np.float32), [512, 512], cpu)
    b = fg.Tensor.new(np.ones(512, np.float32), [512], cpu)
    y = x.matmul(w.permute([1, 0])).add(b)
    items = hip_plan(fg, [y])
    assert [it["class"] for it in items] == ["gemm_mfma_f32"]
    assert len(fg.debug_plan([y], fuse=False)["items"]) == 2  # the copy, then matmul + b
    src = items[0]["source"]
    assert "__builtin_amdgcn_mfma_f32_32x32x2f32" in src
    compile_only(fg, src, items[0]["name"])


@pytest.mark.parametrize("mnk,kind", [((256, 128, 784), "small"), ((100, 20, 8192), "small"),
                                      ((128, 10, 256), "small"), ((128, 784, 256), "small"),
                                      ((4096, 4096, 64), "whole"), ((1024, 20, 8192), "split"),
                                      ((2048, 64, 2048), "split")])
def test_gemm_forms_by_size(fg, cpu, mnk, kind):
    # Up to M*N*K = 2^26 (an MLP's layers at batch 256): one pass of 16x16
    # tiles with K split over the workgroup's waves, no scratch. Larger
    # products: 32x32 MFMA tiles, split-K (or stream-K) with a finishing pass
    # when whole tiles would not fill the chip.
    m, n, k = mnk
    x = fg.Tensor.new(np.ones((m, k), np.float32), [m, k], cpu)
    w = fg.Tensor.new(np.ones((n, k), np.float32), [n, k], cpu)
    items = hip_plan(fg, [x.matmul(w.permute([1, 0]))])
    gemm = [it for it in items if it["class"] == "gemm_mfma_f32"]
    assert len(gemm) == 1
    src = gemm[0]["source"]
    split = "_part(" in src and "_fin(" in src and "fg_scratch" in src
    small = "__builtin_amdgcn_mfma_f32_16x16x4f32" in src and "fg_part[" in src
    assert (kind == "small") == small and (kind == "split") == split, (small, split)
    if kind == "small":
        assert gemm[0]["grid"] == [((m + 15) // 16) * ((n + 15) // 16), 1, 1]
    compile_only(fg, src, gemm[0]["name"] + ("_part" if split else ""))


@pytest.mark.parametrize("batch,dims", [(256, (784, 128, 10)), (512, (784, 256, 256, 10))])
def test_train_step_kernels_compile_and_use_mfma(fg, cpu, batch, dims):
    from ferrograd_amd.mlp import Mlp, synthetic_batch

    fg.reset_init_seed(42)
    model = Mlp(dims, cpu)
    xs, ts = synthetic_batch(batch, dims[0], dims[-1], 7, 8)
    x = fg.Tensor.new(xs, list(xs.shape), cpu)
    t = fg.Tensor.new(ts, list(ts.shape), cpu)
    loss = model.forward(x).cross_entropy(t)
    loss.backward()
    params = model.parameters()
    for p in params:
        p.assign(p.detach().sub(p.grad().mul(fg.Tensor.scalar(0.01, cpu))))
    items = hip_plan(fg, params + [loss])
    classes = [it["class"] for it in items]
    # One thread per output folds serially only the recomputed class-axis sums
    # of the log_softmax gradient: loops of at most 16 iterations, no longer.
    for it in items:
        if it["class"] == "serial":
            trips = [int(n) for n in re.findall(r"for \(int \w+ = 0; \w+ < (\d+);", it["source"])]
            assert trips and max(trips) <= 16, (it["name"], trips)
    assert classes.count("serial") <= 2
    # forward, dW and dX products of every layer wide enough for tiles
    assert classes.count("gemm_mfma_f32") >= 2 * (len(dims) - 1) - 1
    for it in items:
        compile_only(fg, it["source"], it["name"])


def test_narrowed_operands_stay_on_mfma_with_vector_loads(fg, cpu):
    # A batch taken with narrow() carries its start as a kernel scalar; a
    # start times the 784-float row stride keeps 16-byte alignment.
    x = fg.Tensor.new(np.ones((1024, 784), np.float32), [1024, 784], cpu).narrow(0, 256, 256)
    w = fg.Tensor.new(np.ones((128, 784), np.float32), [128, 784], cpu)
    items = hip_plan(fg, [x.matmul(w.permute([1, 0]))])
    gemm = [it for it in items if it["class"] == "gemm_mfma_f32"]
    assert len(gemm) == 1
    src = gemm[0]["source"]
    assert "*(const fg_f4*)(data" in src and "_part(" not in src and "*784)" in src
    compile_only(fg, src, gemm[0]["name"])


def test_in_place_update_reading_other_indices_runs_sequentially(fg, cpu):
    # One thread in the reference's loop order (tests/test_in_place.py has
    # the values): no parallel class may take it, whatever OPT enables.
    w = fg.Tensor.new(np.arange(4, dtype=np.float32), [2, 2], cpu)
    w.assign(w.add(w.permute([1, 0])))
    (it,) = hip_plan(fg, [w])
    assert it["class"] == "sequential" and it["base_class"] == "sequential"
    assert it["grid"] == [1, 1, 1] and "threadIdx.x != 0) return;" in it["source"]
    compile_only(fg, it["source"], it["name"])


def test_reshape_of_permuted_view_is_an_error_not_a_crash(fg, cpu):
    w = fg.Tensor.new(np.arange(4, dtype=np.float32), [2, 2], cpu)
    with pytest.raises(fg.FerrogradError, match="reshape that is not a squeeze reaches a view of several dimensions"):
        hip_plan(fg, [w.permute([1, 0]).reshape([4]).add(fg.Tensor.new(np.ones(4, np.float32), [4], cpu))])


def test_reshape_index_rules_follow_the_reference(fg, cpu):
    # indexing.rs:143-169: a reshape that only adds or drops size-1 dims maps
    # indices one to one; any other reshape flattens to one index, which only
    # a one-dimensional buffer takes. A created tensor is Reshape(Buffer,
    # shape) (tensor.rs:260-284), so [6, 8] -> [48] reaches a two-dimensional
    # view with one index: the reference's flat_index assertion panics there
    # (indexing.rs:42-46), and this build reports it.
    import numpy as np

    a = np.arange(48, dtype=np.float32)
    flat = fg.Tensor.new(a, [48], cpu)
    assert np.array_equal(flat.reshape([6, 8]).add(flat.reshape([6, 8])).numpy(), (a + a).reshape(6, 8))
    mat = fg.Tensor.new(a.reshape(6, 8), [6, 8], cpu)
    sq = mat.reshape([6, 1, 8]).reshape([1, 6, 8, 1]).add(mat.reshape([1, 6, 8, 1]))
    assert np.array_equal(sq.numpy().reshape(6, 8), (a + a).reshape(6, 8))
    with pytest.raises(fg.FerrogradError, match="reshape that is not a squeeze reaches a view of several dimensions"):
        fg.Tensor.realize_many([mat.reshape([48]).add(flat)])


def test_kernels_beyond_int32_indexing_are_refused(fg, cpu):
    # 2^32 outputs from a broadcast scalar: no storage is allocated to plan it.
    s = fg.Tensor.new([1.0], [1], cpu).reshape([1, 1]).expand([1 << 16, 1 << 16])
    with pytest.raises(fg.FerrogradError, match="int32"):
        hip_plan(fg, [s.add(s)])


def test_float_literals_match_reference_text(fg, cpu):
    x = fg.Tensor.new(np.ones(8, np.float32), [8], cpu)
    items = hip_plan(fg, [x.exp()])
    # LOG2_E as f32 (tensor.rs:697-700) is a loaded scalar; exp2 runs in double.
    assert "(float)exp2((double)" in items[0]["source"]


@pytest.mark.parametrize("m,n,k,layout", [(8192, 10, 4096, "rows"), (10, 4096, 2048, "rows"), (2048, 12, 1024, "rows"),
                                           (4096, 10, 2048, "rows")])
def test_narrow_products_lower_to_the_narrow_class(fg, cpu, m, n, k, layout):
    # x·Wᵀ with 16 or fewer outputs on one side: the VALU narrow kernel, not a
    # 32-wide MFMA tile.
    x = fg.Tensor.new(np.ones((m, k), np.float32), [m, k], cpu)
    w = fg.Tensor.new(np.ones((n, k), np.float32), [n, k], cpu)
    (it,) = fg.debug_plan([x.matmul(w.permute([1, 0]))], fuse=True, render_hip=True)["items"]
    assert it["class"] == "gemm_narrow_f32" and it["name"].endswith("_ngemm")
    # The rows layout sums its per-wave totals through the fg_nt LDS array.
    assert ("fg_nt[" in it["source"]) == (layout == "rows")


@pytest.mark.parametrize("m,n,k,cached", [(8192, 10, 4096, True), (1500, 10, 2000, True), (1537, 16, 1500, True),
                                           (300, 10, 4096, True), (602, 12, 4000, False), (4096, 10, 8192, False),
                                           (140000, 16, 64, False)])
def test_narrow_rows_hold_the_narrow_operand_in_registers_when_it_fits(fg, cpu, m, n, k, cached):
    # N x ceil(K/1024) x 4 floats of the narrow operand per thread: at most
    # 160 (two waves per SIMD), and the workgroup's sums (4 x rows x N) within
    # 64 KB of LDS; else the row-group layout that re-reads it.
    x = fg.Tensor.new(np.ones((m, k), np.float32), [m, k], cpu)
    w = fg.Tensor.new(np.ones((n, k), np.float32), [n, k], cpu)
    (it,) = fg.debug_plan([x.matmul(w.permute([1, 0]))], fuse=True, render_hip=True)["items"]
    assert it["class"] == "gemm_narrow_f32"
    assert ("nb0_0[" in it["source"]) == cached
    if cached:
        rows = -(-m // min(512, m))
        assert it["grid"] == [-(-m // rows), 1, 1] and it["block"] == [256, 1, 1]


def test_narrow_rows_ring_holds_each_load_of_a_fused_operand(fg, cpu):
    # relu(a*b)·Wᵀ: two loads per wide element, each with its own ring buffers
    # (w<buffer>_<load>_<k block>), evaluated when the row is folded.
    a = fg.Tensor.new(np.ones((4096, 2048), np.float32), [4096, 2048], cpu)
    b = fg.Tensor.new(np.ones((4096, 2048), np.float32), [4096, 2048], cpu)
    w = fg.Tensor.new(np.ones((10, 2048), np.float32), [10, 2048], cpu)
    (it,) = fg.debug_plan([a.mul(b).relu().matmul(w.permute([1, 0]))], fuse=True, render_hip=True)["items"]
    src = it["source"]
    assert it["class"] == "gemm_narrow_f32" and "nb0_0[" in src
    assert all(f"w{d}_{i}_{j}[4]" in src for d in (0, 1) for i in (0, 1) for j in (0, 1))


def test_narrow_weight_gradient_lowers_to_split_cols(fg, cpu):
    g = fg.Tensor.new(np.ones((8192, 10), np.float32), [8192, 10], cpu)
    h = fg.Tensor.new(np.ones((8192, 4096), np.float32), [8192, 4096], cpu)
    w = fg.Tensor.new(np.ones((10, 4096), np.float32), [10, 4096], cpu).with_requires_grad(True)
    (dw,) = h.matmul(w.permute([1, 0])).mul(g).sum([0, 1]).gradient([w])
    (it,) = fg.debug_plan([dw], fuse=True, render_hip=True)["items"]
    assert it["class"] == "gemm_narrow_f32" and "_ngemm_part" in it["source"] and "_ngemm_fin" in it["source"]
