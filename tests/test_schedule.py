"""Kernel partitioning (src/schedule.rs) — the reference's schedule tests
(schedule.rs:421-570) through the public API, plus the value-preserving fusion
the HIP device enables. CPU only: plans are inspected, not run."""
import numpy as np
import pytest


def plan(fg, roots, fuse=False, render=False):
    return fg.debug_plan(roots, fuse=fuse, render_hip=render)["items"]


def test_nested_reductions_materialize_via_shared_buffer(fg, cpu):  # schedule.rs:421-434
    x = fg.Tensor.new([1.0, 2.0, 3.0, 4.0], [2, 2], cpu)
    items = plan(fg, [x.sum([1]).sum([0])])
    assert len(items) == 2
    assert items[1]["inputs"][0] == {"buffer": items[0]["output"]}


def test_shared_subexpression_materializes_once(fg, cpu):  # schedule.rs:436-464
    left = fg.Tensor.new([1.0, 2, 3, 4], [2, 2], cpu)
    right = fg.Tensor.new([10.0, 20, 30, 40], [2, 2], cpu)
    shared = left.add(right)
    root = shared.sum([1]).add(shared.max([1]))
    items = plan(fg, [root])
    assert len(items) == 4
    assert items[1]["inputs"][0] == {"buffer": items[0]["output"]}
    assert items[2]["inputs"][0] == {"buffer": items[0]["output"]}
    assert items[3]["inputs"][0] == {"buffer": items[1]["output"]}
    assert items[3]["inputs"][1] == {"buffer": items[2]["output"]}


def test_each_shrink_occurrence_gets_its_own_scalar(fg, cpu):  # schedule.rs:466-490
    x = fg.Tensor.new([1.0, 2, 3, 4, 5, 6], [3, 2], cpu)
    items = plan(fg, [x.narrow(0, 0, 2).add(x.narrow(0, 1, 2))])
    scalars = [i for it in items for i in it["inputs"] if "i32" in i or "f32" in i or "bool" in i]
    assert len(scalars) == 2
    assert sorted(s["i32"] for s in scalars) == [0, 1]


def test_store_turns_shrink_start_into_scalar(fg, cpu):  # schedule.rs:492-506
    src = fg.Tensor.new([1.0, 2, 3, 4, 5, 6], [3, 2], cpu)
    dst = fg.Tensor.new([0.0, 0, 0, 0], [2, 2], cpu)
    dst.assign(src.narrow(0, 1, 2))
    items = plan(fg, [dst])
    assert len(items) == 1 and items[0]["output"] is None
    ins = items[0]["inputs"]
    assert "buffer" in ins[0] and "buffer" in ins[1] and ins[2] == {"i32": 1}


def test_shared_movement_view_does_not_materialize(fg, cpu):  # schedule.rs:508-537
    left = fg.Tensor.new([1.0, 2, 3, 4], [2, 2], cpu)
    right = fg.Tensor.new([10.0, 20, 30, 40], [2, 2], cpu)
    moved = left.add(right).reshape([4]).reshape([2, 2])
    items = plan(fg, [moved.sum([1]).add(moved.max([1]))])
    # The reshape chain is a view; the Add under it still has two consumers
    # through the shared view only, so it is not materialised.
    assert len(items) == 3
    assert all("buffer" in i for i in items[0]["inputs"][:2])
    assert items[2]["inputs"][0] == {"buffer": items[0]["output"]}
    assert items[2]["inputs"][1] == {"buffer": items[1]["output"]}


def test_shared_view_stays_inlined_for_assignments(fg, cpu):  # schedule.rs:539-570
    left = fg.Tensor.new([1.0, 2, 3, 4], [2, 2], cpu)
    right = fg.Tensor.new([10.0, 20, 30, 40], [2, 2], cpu)
    dst_a = fg.Tensor.new([0.0] * 4, [2, 2], cpu)
    dst_b = fg.Tensor.new([0.0] * 4, [2, 2], cpu)
    moved = left.add(right).permute([1, 0])
    dst_a.assign(moved)
    dst_b.assign(moved)
    items = plan(fg, [dst_a, dst_b])
    assert len(items) == 2
    assert all(it["output"] is None for it in items)
    assert all(all("buffer" in i for i in it["inputs"][:3]) for it in items)


def test_matmul_emits_contiguous_copy_then_reduce(fg, cpu):  # tensor.rs:762-778
    x = fg.Tensor.new(np.ones((4, 8), np.float32), [4, 8], cpu)
    w = fg.Tensor.new(np.ones((8, 6), np.float32), [8, 6], cpu)
    items = plan(fg, [x.matmul(w)])
    assert len(items) == 2
    assert items[0]["out_shape"] == [6, 8]  # permute(...).contiguous()
    assert {"buffer": items[0]["output"]} in items[1]["inputs"]


def test_relu_input_materialised_without_fusion(fg, cpu):  # tensor.rs:517-531, schedule.rs:321-326
    a, b, c = (fg.Tensor.new(np.ones(64, np.float32), [64], cpu) for _ in range(3))
    items = plan(fg, [a.mul(b).add(c).relu()])
    assert len(items) == 2
    assert len(items[1]["inputs"]) == 2  # the zeros buffer and the materialised input


def test_fusion_makes_c2_one_kernel_without_zero_buffer(fg, cpu):
    a, b, c = (fg.Tensor.new(np.ones(64, np.float32), [64], cpu) for _ in range(3))
    items = plan(fg, [a.mul(b).add(c).relu()], fuse=True)
    assert len(items) == 1
    assert len(items[0]["inputs"]) == 3  # a, b, c only: the zeros are a literal


def test_fusion_makes_c1_one_kernel(fg, cpu):
    x = fg.Tensor.new(np.ones((16, 16), np.float32), [16, 16], cpu)
    y = x.mul(fg.Tensor.scalar(0.5, cpu)).add(fg.Tensor.scalar(1.0, cpu)).relu().sum([1])
    items = plan(fg, [y], fuse=True)
    assert len(items) == 1 and len(items[0]["inputs"]) == 3


def test_fusion_keeps_nodes_with_diverging_consumers(fg, cpu):
    # The pre-activation feeds relu and an unrelated sum: still materialised
    # (two loaded inputs, so it is not cheap enough to recompute either).
    x = fg.Tensor.new(np.ones((8, 8), np.float32), [8, 8], cpu)
    w = fg.Tensor.new(np.ones((8, 8), np.float32), [8, 8], cpu)
    z = x.add(w)
    items_ref = plan(fg, [z.relu(), z.sum([1])])
    items_fused = plan(fg, [z.relu(), z.sum([1])], fuse=True)
    assert len(items_fused) == len(items_ref)


def test_zero_buffer_folds_only_while_it_holds_zeros(fg, cpu):
    ones = fg.Tensor.new([1.0] * 4, [4], cpu)
    z = fg.Tensor.zeros([4], cpu)
    assert len(plan(fg, [z.add(ones)], fuse=True)[0]["inputs"]) == 1  # zeros became a literal
    z.assign(fg.Tensor.new([1.0, 2.0, 3.0, 4.0], [4], cpu))
    fg.Tensor.realize_many([z])
    y = z.add(ones)
    assert len(plan(fg, [y], fuse=True)[0]["inputs"]) == 2  # written: loaded again
    assert y.to_vec() == [2.0, 3.0, 4.0, 5.0]


def test_assign_in_same_schedule_disables_folding_for_later_kernels(fg, cpu):
    z = fg.Tensor.zeros([4], cpu)
    z.assign(fg.Tensor.new([1.0, 2.0, 3.0, 4.0], [4], cpu))
    y = z.add(fg.Tensor.new([1.0] * 4, [4], cpu))
    items = plan(fg, [z, y], fuse=True)
    assert len(items) == 2 and len(items[1]["inputs"]) == 2


def mlp_forward(fg, dev, dims=(32, 64, 48, 10), batch=16):
    fg.reset_init_seed(42)
    layers = [fg.Linear(dims[i], dims[i + 1], dev) for i in range(len(dims) - 1)]
    x = fg.Tensor.new(np.full((batch, dims[0]), 0.5, np.float32), [batch, dims[0]], dev)
    t = fg.Tensor.new(np.eye(dims[-1], dtype=np.float32)[np.arange(batch) % dims[-1]], [batch, dims[-1]], dev)
    h = x
    for i, l in enumerate(layers):
        h = l(h)
        if i + 1 < len(layers):
            h = h.relu()
    return layers, h.cross_entropy(t)


def test_fusion_runs_linear_bias_as_reduce_epilogue_and_recomputes_relu_mask(fg, cpu):
    # Reference partition: the matmul reduce and `mm + b` are separate kernels
    # (nested-reduce rule), and relu's mask `0 < pre` is a bool buffer shared by
    # forward and backward. Fused: `mm + b` is the reduce's epilogue and the
    # mask is recomputed from pre by its readers.
    layers, loss = mlp_forward(fg, cpu)
    loss.backward()
    params = [p for l in layers for p in l.parameters()]
    for p in params:
        p.assign(p.detach().sub(p.grad().mul(fg.Tensor.scalar(0.01, cpu))))
    ref = plan(fg, params + [loss])
    fused = plan(fg, params + [loss], fuse=True, render=True)
    assert len(fused) < len(ref)
    assert not any("bool* __restrict__ data0" in it["source"] for it in fused)  # no mask buffer
    # Every [16, 64] / [16, 48] pre-activation is written by a reduction kernel.
    pre = [it for it in fused if it.get("out_shape") in ([16, 64], [16, 48])]
    assert pre and all(it["base_class"] != "elementwise" for it in pre)


def test_cheap_node_with_scalar_inputs_is_recomputed(fg, cpu):
    # t * -(1/B) (the cross-entropy gradient seed) feeds two kernels; two ops
    # over one loaded tensor and a 1-element scalar are recomputed by each.
    t = fg.Tensor.new(np.ones((8, 16), np.float32), [8, 16], cpu)
    g = t.mul(fg.Tensor.scalar(0.125, cpu).neg())
    w = fg.Tensor.new(np.ones((8, 16), np.float32), [8, 16], cpu)
    roots = [g.add(w).sum([1]), g.mul(w).sum([1])]
    assert len(plan(fg, roots)) == 3
    # While a tensor points at g, g gets the buffer the reference gives it.
    assert len(plan(fg, roots, fuse=True)) == 3
    del g
    assert len(plan(fg, roots, fuse=True)) == 2


def test_identity_copy_is_read_in_place_but_a_transpose_is_copied(fg, cpu):
    x = fg.Tensor.new(np.ones((4, 8), np.float32), [4, 8], cpu)
    w = fg.Tensor.new(np.ones((6, 8), np.float32), [6, 8], cpu)
    # w.permute().permute().contiguous(): a copy in w's own layout
    assert len(plan(fg, [x.matmul(w.permute([1, 0]))], fuse=True)) == 1
    assert len(plan(fg, [x.matmul(w.permute([1, 0]))])) == 2
    # x @ v with v [8, 6]: permute(v).contiguous() is a real transpose
    v = fg.Tensor.new(np.ones((8, 6), np.float32), [8, 6], cpu)
    items = plan(fg, [x.matmul(v)], fuse=True)
    assert len(items) == 2 and items[0]["out_shape"] == [6, 8]


def test_a_requested_contiguous_is_materialised_even_in_layout_order(fg, cpu):
    # Only matmul's own copy is read in place. A contiguous() the caller holds
    # becomes a buffer at realize, as in the reference, so a later in-place
    # update of w does not show through it.
    w = fg.Tensor.new(np.arange(48, dtype=np.float32), [6, 8], cpu)
    c = w.permute([1, 0]).permute([1, 0]).contiguous()
    y = c.add(fg.Tensor.scalar(1.0, cpu))
    items = plan(fg, [y], fuse=True)
    assert len(items) == 2 and items[0]["out_shape"] == [6, 8]


def test_identity_copy_read_after_an_in_place_store_is_taken_first(fg, cpu):
    # Root 0 stores into w; root 1 reads w through an identity copy and runs
    # after it, so it must see the copy taken before the store.
    x = fg.Tensor.new(np.ones((4, 8), np.float32), [4, 8], cpu)
    w = fg.Tensor.new(np.ones((6, 8), np.float32), [6, 8], cpu)
    y = x.matmul(w.permute([1, 0]))
    w.assign(w.add(fg.Tensor.scalar(1.0, cpu)))
    items = plan(fg, [w, y], fuse=True)
    assert [it["out_shape"] for it in items] == [[6, 8], [], [4, 6]]
    assert items[0]["inputs"] == [{"buffer": items[1]["inputs"][0]["buffer"]}]  # the copy reads w
    assert {"buffer": items[0]["output"]} in items[2]["inputs"]  # y reads the copy


def test_a_held_intermediate_is_realised_as_in_the_reference(fg, cpu):
    # h = x + y feeds relu and its mask, which reconverge: fused, h has no
    # kernel. While the caller holds h, the reference's rule applies: h is
    # materialised and, after realize, h points at its buffer.
    x = fg.Tensor.new(np.arange(8, dtype=np.float32) - 4, [8], cpu)
    y = fg.Tensor.new(np.ones(8, np.float32), [8], cpu)
    h = x.add(y)
    r = h.relu()
    assert len(plan(fg, [r], fuse=True)) == 2
    r2 = x.add(y).relu()  # the same graph, no tensor at x + y other than h
    del h
    assert len(plan(fg, [r2], fuse=True)) == 1


def test_a_held_view_of_a_reduce_keeps_the_reference_partition(fg, cpu):
    # y = x @ wᵀ is a reshape of the matmul reduce. The reduce feeds a later
    # reduction, so the reference materialises it (nested) and repoints y.
    # Fused, it would run as the epilogue of y + b; while y is held, it keeps
    # its kernel instead.
    x = fg.Tensor.new(np.ones((4, 8), np.float32), [4, 8], cpu)
    w = fg.Tensor.new(np.ones((6, 8), np.float32), [6, 8], cpu)
    b = fg.Tensor.new(np.ones(6, np.float32), [6], cpu)
    y = x.matmul(w.permute([1, 0]))
    c = y.add(b)  # two consumers: a kernel of its own, with R as its epilogue when fused
    roots = [c.relu(), c.sum([1])]
    del c
    held = plan(fg, roots, fuse=True)
    del y
    free = plan(fg, roots, fuse=True)
    assert len(held) == len(free) + 1
    assert [4, 6, 1] in [it["out_shape"] for it in held]  # the matmul reduce's own buffer


def test_reduce_read_through_broadcast_stays_materialised(fg, cpu):
    # y = 2 * x.sum(1) feeds a broadcast: fusing it into the consumer would
    # recompute the 64-element sum for every broadcast element, so it keeps
    # its kernel.
    x = fg.Tensor.new(np.ones((4, 64), np.float32), [4, 64], cpu)
    y = x.sum([1]).mul(fg.Tensor.scalar(2.0, cpu))
    z = y.expand([4, 64]).add(x)
    items = plan(fg, [z], fuse=True, render=True)
    assert [it["base_class"] for it in items] == ["row_reduce", "elementwise"]


def test_small_reduce_is_recomputed_by_its_consumer(fg, cpu):
    # A sum over 8 elements read through an 8-fold broadcast (log_softmax's
    # class-axis max and sums) is folded again by each consumer element
    # instead of getting a kernel of its own; the reference partition keeps it.
    x = fg.Tensor.new(np.ones((4, 8), np.float32), [4, 8], cpu)
    z = x.sum([1]).mul(fg.Tensor.scalar(2.0, cpu)).expand([4, 8]).add(x)
    items = plan(fg, [z], fuse=True, render=True)
    assert [it["base_class"] for it in items] == ["row_reduce"]
    assert items[0]["out_shape"] == [4, 8]
    assert len(plan(fg, [z], fuse=False)) == 2


def test_small_reduce_broadcast_far_stays_materialised(fg, cpu):
    # Read through a 200-fold broadcast, recomputing would multiply its loads.
    x = fg.Tensor.new(np.ones((4, 8), np.float32), [4, 8], cpu)
    y = x.sum([1]).mul(fg.Tensor.scalar(2.0, cpu))
    z = y.expand([4, 200]).add(fg.Tensor.new(np.ones((4, 200), np.float32), [4, 200], cpu))
    items = plan(fg, [z], fuse=True, render=True)
    assert [it["base_class"] for it in items] == ["row_reduce", "elementwise"]


def test_small_reduce_feeding_a_reduce_stays_materialised(fg, cpu):
    # Inlined into the outer sum, the inner 8-element sums would make that
    # kernel fold serially; the inner reduce keeps its kernel.
    x = fg.Tensor.new(np.ones((64, 8), np.float32), [64, 8], cpu)
    z = x.sum([1]).mul(fg.Tensor.scalar(2.0, cpu)).sum([0])
    items = plan(fg, [z], fuse=True, render=True)
    assert len(items) == 2 and "serial" not in [it["base_class"] for it in items]


def test_two_reduces_into_one_consumer_keep_one_per_kernel(fg, cpu):
    # Reductions over more elements than are recomputed inline (64 > 16).
    x = fg.Tensor.new(np.ones((4, 64), np.float32), [4, 64], cpu)
    w = fg.Tensor.new(np.ones((4, 64), np.float32), [4, 64], cpu)
    z = x.sum([1]).add(w.max([1]))
    items = plan(fg, [z], fuse=True, render=True)
    assert len(items) == 2 and all(it["base_class"] == "row_reduce" for it in items)


def test_reduce_read_after_an_in_place_store_is_materialised_first(fg, cpu):
    # realize_many([w.assign(w + 1), 2 * w.sum(0)]): the reference materialises
    # the sum (a reduce consumed by ALU) in phase 1, before the store. Fused,
    # the sum would otherwise run as the epilogue of the root that reads it,
    # after root 0's store.
    w = fg.Tensor.new(np.arange(6, dtype=np.float32), [2, 3], cpu)
    y = w.sum([0]).mul(fg.Tensor.scalar(2.0, cpu))
    w.assign(w.add(fg.Tensor.scalar(1.0, cpu)))
    items = plan(fg, [w, y], fuse=True)
    assert [it["out_shape"] for it in items] == [[1, 3], [], [1, 3]]
    assert {"buffer": items[0]["output"]} in items[2]["inputs"]
    # Read before any store, the sum stays the root's epilogue.
    assert [it["out_shape"] for it in plan(fg, [y, w], fuse=True)] == [[1, 3], []]


def test_roots_are_compiled_in_the_order_given(fg, cpu):
    # schedule.rs:118-133 compiles the roots in the order given and replaces
    # each with its buffer only after compiling it; a root is never
    # materialised in phase 1 (schedule.rs:294-296). Listed after a root
    # that reads it, a reduction root is therefore inlined into that root's
    # kernel, a reduction nested inside another (the reference's CPU
    # renderer cannot emit it: the oracle reports it). Listed first, it is a
    # buffer the other root reads.
    r = np.random.default_rng(3)
    x = fg.Tensor.new(r.uniform(-1, 1, (8, 16)).astype(np.float32), [8, 16], cpu)
    w = fg.Tensor.new(r.uniform(-1, 1, (16, 8)).astype(np.float32), [16, 8], cpu)
    s = x.sum([0])
    m = s.matmul(w)
    # (Phase 1 first copies W for matmul's permute().contiguous(), tensor.rs:771-777.)
    producer_first = plan(fg, [s, m])
    assert [it["out_shape"] for it in producer_first] == [[8, 16], [1, 16], [1, 8]]
    assert {"buffer": producer_first[1]["output"]} in producer_first[2]["inputs"]
    consumer_first = plan(fg, [m, s])
    assert [it["out_shape"] for it in consumer_first] == [[8, 16], [1, 8], [1, 16]]
    assert {"buffer": consumer_first[2]["output"]} not in consumer_first[1]["inputs"]
    with pytest.raises(fg.FerrogradError, match="range used outside its loop"):
        fg.Tensor.realize_many([m, s])
