// Kernel partitioning and rangeify.
// schedule_many/should_materialize/parameterize*: src/schedule.rs:64-405.
// rangeify + index pushing: src/schedule/rangeify.rs:42-206,
// src/schedule/indexing.rs:22-242.
#include "schedule.hpp"

#include <algorithm>
#include <unordered_set>

namespace fg {

namespace {

KernelArg scalar_input(const Arg& lit) {  // schedule.rs:247-257
  switch (lit.kind) {
    case Arg::Kind::Float: return KernelArg::f32(static_cast<float>(lit.f));
    case Arg::Kind::Int:
      FG_CHECK(lit.a >= INT32_MIN && lit.a <= INT32_MAX, "kernel scalar int must fit in i32");
      return KernelArg::i32(static_cast<int32_t>(lit.a));
    case Arg::Kind::Bool: return KernelArg::boolean(lit.a != 0);
    default: fail("kernel scalar input must be a literal");
  }
}

// schedule.rs:176-245. Replaces Buffers, Binds and constant Shrink starts with
// numbered parameters; the output (if any) owns slot 0.
std::pair<UOp, std::vector<KernelArg>> parameterize_inputs(const UOp& root, size_t slot_offset,
                                                           const ScheduleOptions& opt) {
  DeviceId device = root.device();
  std::vector<KernelArg> inputs;
  std::unordered_map<const BufferInner*, UOp> params;
  UOpMap<UOp> scalar_params;
  auto fn = [&](const UOp& node) -> UOp {
    switch (node.op()) {
      case Op::Buffer: {
        const Buffer& h = node.arg().buf;
        if (!h) return UOp();
        if (opt.fuse && h->known_zero && node.dtype() == DType::F32()) {
          // A buffer that still holds allocate()'s zeros reads as 0.0f at
          // every index: the literal is the same value without the load.
          UOp zero = UOp::make(Op::Const, node.dtype(), {UOp::device_uop(device)}, Arg::flt(0.0),
                               true, kZeroBufferTag);
          UOp base = UOp::reshape(zero, Shape{1});
          if (h->numel == 1) return base;
          return UOp::expand(base, Shape{h->numel});
        }
        auto it = params.find(h.get());
        if (it != params.end()) return it->second;
        size_t slot = inputs.size() + slot_offset;
        inputs.push_back(KernelArg::buf(h));
        UOp p = UOp::param_buffer(static_cast<int64_t>(slot), node.dtype(),
                                  static_cast<int64_t>(h->numel), device);
        params.emplace(h.get(), p);
        return p;
      }
      case Op::Bind: {
        const UOp& var = node.src(0);
        auto it = scalar_params.find(var);
        if (it != scalar_params.end()) return it->second;
        size_t slot = inputs.size() + slot_offset;
        inputs.push_back(scalar_input(node.src(1).arg()));
        UOp p = UOp::param_scalar(static_cast<int64_t>(slot), node.dtype(), device);
        scalar_params.emplace(var, p);
        return p;
      }
      case Op::Shrink: {
        Shape src_shape;
        if (!node.src(0).shape_opt(&src_shape)) return UOp();
        const auto& lens = node.arg().v;
        bool changed = false;
        std::vector<UOp> ns{node.src(0)};
        for (size_t ax = 0; ax + 1 < node.srcs().size() && ax < lens.size(); ax++) {
          const UOp& start = node.src(ax + 1);
          if (static_cast<size_t>(lens[ax]) != src_shape[ax] && start.op() == Op::Const) {
            size_t slot = inputs.size() + slot_offset;
            inputs.push_back(scalar_input(start.arg()));
            ns.push_back(UOp::param_scalar(static_cast<int64_t>(slot), start.dtype(), device));
            changed = true;
            continue;
          }
          ns.push_back(start);
        }
        for (size_t i = ns.size(); i < node.srcs().size(); i++) ns.push_back(node.src(i));
        if (!changed) return UOp();
        return UOp::make_new(Op::Shrink, node.dtype(), ns, node.arg());
      }
      default:
        return UOp();
    }
  };
  // One bottom-up pass in toposort order visits leaves in the same order as
  // the first iteration of the reference's fixed-point rewrite (so slots
  // match), and the rule never fires on its own output, so no second pass.
  UOpMap<UOp> sub;
  auto order = root.toposort();
  sub.reserve(order.size() * 2);
  for (auto& node : order) {
    std::vector<UOp> ns;
    ns.reserve(node.srcs().size());
    bool changed = false;
    for (auto& s : node.srcs()) {
      const UOp& x = sub.at(s);
      ns.push_back(x);
      changed = changed || x != s;
    }
    UOp rebuilt = node;
    if (changed)
      rebuilt = node.op() == Op::Sink ? UOp::sink(ns) : UOp::make_new(node.op(), node.dtype(), ns, node.arg());
    UOp r = fn(rebuilt);
    sub[node] = r ? r : rebuilt;
  }
  return {sub.at(root), inputs};
}

// schedule.rs:131-151
ScheduleItem parameterize(const UOp& expr, const ScheduleOptions& opt) {
  Device& backend = get_device(expr.device());
  auto [p, inputs] = parameterize_inputs(expr, 1, opt);
  Shape out_shape;
  if (!p.shape_opt(&out_shape)) out_shape = Shape{1};
  Buffer out = backend.reserve_buffer(expr.dtype(), numel(out_shape));
  UOp out_param = UOp::param_buffer(0, expr.dtype(), static_cast<int64_t>(numel(out_shape)), expr.device());
  UOp store = UOp::make_new(Op::Store, DType::Void(), {out_param, p}, Arg::none());
  ScheduleItem item;
  item.sink = UOp::sink({store});
  item.inputs = std::move(inputs);
  item.output_buffer = out;
  item.out_shape = out_shape;
  return item;
}

// schedule.rs:264-272
UOpSet nested_reduce_inputs(const std::vector<UOp>& order) {
  UOpSet feeds;
  for (size_t i = order.size(); i-- > 0;) {
    const UOp& n = order[i];
    if (n.op() == Op::ReduceAxis || feeds.count(n))
      for (auto& s : n.srcs()) feeds.insert(s);
  }
  return feeds;
}

// Reconvergence test for value-preserving fusion: every consumer path out of
// `node` runs through elementwise nodes of the same shape and ends in one
// elementwise node `d`, so computing `node` inside `d`'s kernel reads each
// input element once (identical loads intern to one node).
bool reconverges(const UOp& node, const UOpMap<std::vector<UOp>>& consumers, const UOpSet& roots,
                 const UOpMap<size_t>& topo_idx) {
  if (!is_alu(node.op())) return false;
  Shape s;
  if (!node.shape_opt(&s)) return false;
  auto it = consumers.find(node);
  if (it == consumers.end() || it->second.size() < 2) return false;
  // Candidate: the latest consumer in topological order.
  UOp d;
  size_t best = 0;
  for (auto& c : it->second) {
    size_t k = topo_idx.at(c);
    if (!d || k > best) { d = c; best = k; }
  }
  if (!is_alu(d.op())) return false;
  Shape ds;
  if (!d.shape_opt(&ds) || ds != s) return false;
  // Every other consumer must flow only into d (or into nodes that do), via
  // single-purpose elementwise nodes of the same shape, within a small depth.
  std::function<bool(const UOp&, int)> flows_to_d = [&](const UOp& c, int depth) -> bool {
    if (c == d) return true;
    if (depth > 4 || roots.count(c) || !is_alu(c.op())) return false;
    Shape cs;
    if (!c.shape_opt(&cs) || cs != s) return false;
    auto ci = consumers.find(c);
    if (ci == consumers.end() || ci->second.empty()) return false;
    for (auto& cc : ci->second)
      if (!flows_to_d(cc, depth + 1)) return false;
    return true;
  };
  for (auto& c : it->second)
    if (!flows_to_d(c, 0)) return false;
  return true;
}

// What a kernel reading `src` loads: a literal, one buffer, or something that
// needs computing. Movement views of constants, of allocate()'s still-zero
// buffers (read as literals when fusing) and of buffers are leaves, as are
// nodes already materialised.
enum class LeafKind { Literal, Buffer, Computed };
LeafKind leaf_kind(const UOp& src, const UOpMap<UOp>& materialized) {
  UOp b = src;
  while (true) {
    if (materialized.count(b)) return LeafKind::Buffer;
    if (!is_movement(b.op()) || b.op() == Op::Contiguous) break;
    b = b.src(0);
  }
  if (b.op() == Op::Const) return LeafKind::Literal;
  if (b.op() == Op::Buffer) {
    const Buffer& h = b.arg().buf;
    if (h && h->known_zero && b.dtype() == DType::F32()) return LeafKind::Literal;
    return LeafKind::Buffer;
  }
  return LeafKind::Computed;
}

// Elements behind a leaf (a materialised node, or a buffer seen through views).
size_t leaf_numel(const UOp& src, const UOpMap<UOp>& materialized) {
  UOp b = src;
  while (!materialized.count(b) && is_movement(b.op())) b = b.src(0);
  if (!materialized.count(b) && b.op() == Op::Buffer && b.arg().buf) return b.arg().buf->numel;
  Shape s;
  return b.shape_opt(&s) ? numel(s) : 0;
}

// A multi-consumer node cheap enough to recompute in each consumer: at most
// three comparisons or arithmetic ops over literals, 1-element scalars and at
// most one other loaded value. relu's mask `0 < x` and the cross-entropy
// gradient seed `t * -(1/B)` are the cases that matter. Recomputing it reads
// that one value where the materialised node would have been read, and gives
// the same bits.
bool cheap_to_recompute(const UOp& node, const UOpMap<UOp>& materialized) {
  int ops = 0, loads = 0;
  std::vector<UOp> stack{node};
  UOpSet seen;
  while (!stack.empty()) {
    UOp n = stack.back();
    stack.pop_back();
    if (!seen.insert(n).second) continue;
    if (n != node) {
      LeafKind k = leaf_kind(n, materialized);
      if (k == LeafKind::Literal) continue;
      if (k == LeafKind::Buffer) {
        if (leaf_numel(n, materialized) != 1) loads++;
        continue;
      }
      if (is_movement(n.op())) {  // index arithmetic only
        stack.push_back(n.src(0));
        continue;
      }
    }
    switch (n.op()) {
      case Op::CmpLt: case Op::Neg: case Op::Add: case Op::Mul: case Op::Max: case Op::Where: break;
      default: return false;
    }
    if (++ops > 3) return false;
    for (auto& s : n.srcs()) stack.push_back(s);
  }
  return loads <= 1;
}

bool has_unmaterialized_reduce(const UOp& expr, const UOpMap<UOp>& materialized, const UOp& except);

// A reduction over at most kSmallReduce elements that each elementwise
// consumer can recompute instead of reading a materialised [.., 1] buffer: the
// class-axis max and sums of log_softmax and its gradient over 10 classes,
// which otherwise cost one launch each in every train step. Value-preserving:
// each consumer folds the same loaded values in the same order. Kept
// materialised when its input still computes (more than a few elementwise ops,
// or another pending reduction), when it feeds a reduction (whose kernel would
// then fold serially), and when a consumer broadcasts it more than
// kSmallReduce-fold (the recompute would multiply the loads).
constexpr size_t kSmallReduce = 16;

// Whether the kernels that would compute `node` inline all stay small enough:
// every path from it through elementwise and movement consumers must end at a
// root or at a node with a kernel of its own (a multi-consumer node that
// neither reconverges nor is cheap to recompute) without meeting a
// ReduceAxis (that kernel would fold `node` serially) or any node of more than
// `max_numel` elements (each would fold it again).
bool inline_consumers_fit(const UOp& node, size_t max_numel, const UOpMap<std::vector<UOp>>& consumers,
                          const UOpSet& roots, const UOpMap<size_t>& topo_idx, const UOpMap<UOp>& materialized) {
  std::vector<std::pair<UOp, int>> stack;
  auto push_consumers = [&](const UOp& n, int depth) {
    auto it = consumers.find(n);
    if (it != consumers.end())
      for (auto& c : it->second) stack.emplace_back(c, depth + 1);
  };
  push_consumers(node, 0);
  UOpSet seen;
  while (!stack.empty()) {
    auto [c, depth] = stack.back();
    stack.pop_back();
    if (!seen.insert(c).second || c.op() == Op::Sink) continue;
    Shape cs;
    if (c.op() == Op::ReduceAxis || depth > 8 || !c.shape_opt(&cs) || numel(cs) > max_numel) return false;
    if (roots.count(c)) continue;
    if (is_alu(c.op())) {
      auto ci = consumers.find(c);
      bool own = ci != consumers.end() && ci->second.size() > 1 && !reconverges(c, consumers, roots, topo_idx) &&
                 !cheap_to_recompute(c, materialized);
      if (own) continue;
    } else if (!is_movement(c.op())) {
      return false;
    }
    push_consumers(c, depth);
  }
  return true;
}

bool small_reduce_recomputable(const UOp& node, const UOpMap<std::vector<UOp>>& consumers, const UOpSet& roots,
                               const UOpMap<size_t>& topo_idx, const UOpMap<UOp>& materialized) {
  if (node.op() != Op::ReduceAxis) return false;
  Shape in_shape, out_shape;
  if (!node.src(0).shape_opt(&in_shape) || !node.shape_opt(&out_shape)) return false;
  const size_t out_n = numel(out_shape), extent = numel(in_shape) / std::max<size_t>(1, out_n);
  if (extent > kSmallReduce) return false;
  // The input: elementwise ops over literals and loaded values only.
  int alu = 0;
  std::vector<UOp> stack{node.src(0)};
  UOpSet seen;
  while (!stack.empty()) {
    UOp n = stack.back();
    stack.pop_back();
    if (!seen.insert(n).second) continue;
    if (leaf_kind(n, materialized) != LeafKind::Computed) continue;
    if (is_movement(n.op())) {
      stack.push_back(n.src(0));
      continue;
    }
    if (!is_alu(n.op()) || ++alu > 4) return false;
    for (auto& s : n.srcs()) stack.push_back(s);
  }
  if (has_unmaterialized_reduce(node.src(0), materialized, UOp())) return false;
  return inline_consumers_fit(node, kSmallReduce * out_n, consumers, roots, topo_idx, materialized);
}

// Whether `expr` (a kernel value under construction) computes a reduction
// that is not yet materialised.
bool has_unmaterialized_reduce(const UOp& expr, const UOpMap<UOp>& materialized, const UOp& except) {
  std::vector<UOp> stack{expr};
  UOpSet seen;
  while (!stack.empty()) {
    UOp n = stack.back();
    stack.pop_back();
    if (n == except || materialized.count(n) || !seen.insert(n).second) continue;
    if (n.op() == Op::ReduceAxis) return true;
    for (auto& s : n.srcs()) stack.push_back(s);
  }
  return false;
}

// When `node` (matmul's own Contiguous, tagged kMatmulCopyTag) copies a buffer
// in the buffer's own memory order, the buffer node; else null. Its source must be the buffer seen only
// through permutes and reshapes that compose to the row-major layout of the
// copy, as nn.rs:98's `weight.permute([1, 0])` followed by matmul's
// `other.permute([1, 0]).contiguous()` (tensor.rs:771-777) is. Readers can
// then load the buffer where they would have loaded the copy: same elements,
// same order.
UOp identity_copy_source(const UOp& node) {
  if (node.op() != Op::Contiguous || !node.has_tag() || node.tag() != kMatmulCopyTag) return UOp();
  std::vector<UOp> chain;
  UOp b = node.src(0);
  while (b.op() == Op::Permute || b.op() == Op::Reshape) {
    chain.push_back(b);
    b = b.src(0);
  }
  if (b.op() != Op::Buffer || !b.arg().buf) return UOp();
  Shape shape{b.arg().buf->numel};
  std::vector<size_t> strides{1};
  auto row_major = [](const Shape& sh, const std::vector<size_t>& st) {
    size_t expect = 1;
    for (size_t d = sh.size(); d-- > 0;) {
      if (sh[d] == 1) continue;
      if (st[d] != expect) return false;
      expect *= sh[d];
    }
    return true;
  };
  for (auto it = chain.rbegin(); it != chain.rend(); ++it) {
    const UOp& m = *it;
    if (m.op() == Op::Permute) {
      auto ax = m.arg().usizes();
      Shape ns;
      std::vector<size_t> nt;
      for (auto a : ax) {
        ns.push_back(shape[a]);
        nt.push_back(strides[a]);
      }
      shape = ns;
      strides = nt;
      continue;
    }
    Shape ns = m.arg().usizes();
    if (row_major(shape, strides)) {
      shape = ns;
      strides = contiguous_strides(ns);
    } else {
      return UOp();  // a reshape of a permuted view is no plain view
    }
  }
  return row_major(shape, strides) ? b : UOp();
}

bool is_held(const UOp& node, const ScheduleOptions& opt) {
  return opt.held && opt.held->get(node.get()) != PtrIndexMap::kAbsent;
}

// schedule.rs:289-335
bool should_materialize(const UOp& node, const UOpSet& roots,
                        const UOpMap<std::vector<UOp>>& consumers, const UOpSet& nested,
                        const ScheduleOptions& opt, const UOpMap<size_t>& topo_idx,
                        const UOpMap<UOp>& materialized) {
  if (roots.count(node) || !node.has_shape()) return false;
  switch (node.op()) {
    case Op::Sink: case Op::Store: case Op::After: case Op::Assign: case Op::DefineAcc:
    case Op::Buffer: case Op::Const: case Op::DefineVar: case Op::Bind:
      return false;
    default: break;
  }
  const bool fuse = opt.fuse && !is_held(node, opt);
  if (node.op() == Op::Contiguous) return !(fuse && identity_copy_source(node));
  if (is_movement(node.op())) return false;
  if (node.has_buffer_identity()) return false;
  if (fuse && small_reduce_recomputable(node, consumers, roots, topo_idx, materialized)) return false;
  auto it = consumers.find(node);
  if (it != consumers.end() && it->second.size() > 1) {
    if (fuse && (reconverges(node, consumers, roots, topo_idx) || cheap_to_recompute(node, materialized)))
      return false;
    return true;
  }
  if (node.op() == Op::ReduceAxis && it != consumers.end()) {
    for (auto& c : it->second)
      if (is_alu(c.op())) return true;
  }
  return node.op() == Op::ReduceAxis && nested.count(node);
}

// The elementwise node a reduce feeds through a chain of single-consumer
// reshapes/permutes (views that read each reduced value once), or null. When
// fusing, the reduce can run as that node's epilogue instead of writing its
// own buffer.
UOp epilogue_consumer(const UOp& reduce, const UOpMap<std::vector<UOp>>& consumers, const UOpSet& roots) {
  UOp cur = reduce;
  while (true) {
    if (roots.count(cur)) return UOp();
    auto it = consumers.find(cur);
    if (it == consumers.end() || it->second.size() != 1) return UOp();
    const UOp& c = it->second[0];
    if (c.op() == Op::Reshape || c.op() == Op::Permute) {
      cur = c;
      continue;
    }
    return is_alu(c.op()) ? c : UOp();
  }
}

// schedule.rs:340-353
UOp buffer_replacement(const ScheduleItem& item) {
  FG_CHECK(item.output_buffer, "buffer_replacement requires an allocated output");
  UOp b = UOp::buffer(item.output_buffer, item.output_buffer->dtype, item.sink.device());
  return UOp::reshape(b, item.out_shape);
}

// schedule.rs:359-365
bool assignment_effect(const UOp& root, UOp* store, UOp* value) {
  if (root.op() != Op::After || root.srcs().size() != 2) return false;
  if (root.src(1).op() != Op::Store) return false;
  *store = root.src(1);
  *value = root.src(0);
  return true;
}

// schedule.rs:371-405. Same result as the reference's full-graph walk, but
// the walk stops at nodes already replaced by a buffer: nothing below them can
// appear in this kernel.
UOp substitute_materialized(const UOp& root, const UOpMap<UOp>& replacements) {
  UOpMap<UOp> sub;
  std::vector<std::pair<UOp, bool>> stack{{root, false}};
  while (!stack.empty()) {
    auto [node, expanded] = stack.back();
    stack.pop_back();
    if (sub.count(node)) continue;
    if (node != root) {
      auto r = replacements.find(node);
      if (r != replacements.end()) {
        sub[node] = r->second;
        continue;
      }
    }
    if (!expanded) {
      stack.emplace_back(node, true);
      for (auto& s : node.srcs())
        if (!sub.count(s)) stack.emplace_back(s, false);
      continue;
    }
    std::vector<UOp> ns;
    ns.reserve(node.srcs().size());
    bool changed = false;
    for (auto& s : node.srcs()) {
      const UOp& x = sub.at(s);
      ns.push_back(x);
      changed = changed || x != s;
    }
    sub[node] = changed ? (node.op() == Op::Sink ? UOp::sink(ns)
                                                 : UOp::make_new(node.op(), node.dtype(), ns, node.arg()))
                        : node;
  }
  return sub.at(root);
}

// Marks the store destination's buffer as written (it no longer holds zeros).
void mark_written(const UOp& dest) {
  UOp d = dest;
  while (d && d.op() != Op::Buffer) {
    if (d.srcs().empty()) return;
    d = d.src(0);
  }
  if (d && d.arg().buf) d.arg().buf->known_zero = false;
}

}  // namespace

// schedule.rs:156-170
ScheduleItem parameterize_store(const UOp& store, const ScheduleOptions& opt) {
  FG_CHECK(store.op() == Op::Store, "parameterize_store requires a Store root");
  // The destination is about to be written: it must not fold to zeros in this
  // kernel or any kernel scheduled after it.
  mark_written(store.src(0));
  auto [p, inputs] = parameterize_inputs(store, 0, opt);
  ScheduleItem item;
  item.sink = UOp::sink({p});
  item.inputs = std::move(inputs);
  return item;
}

// schedule.rs:64-126
SchedulePlan schedule_many(const std::vector<UOp>& exprs, const ScheduleOptions& opt) {
  FG_CHECK(!exprs.empty(), "schedule_many requires at least one root");
  UOp uni = UOp::sink(exprs);
  auto order = uni.toposort();
  auto consumers = build_consumer_map(order);
  auto nested = nested_reduce_inputs(order);
  UOpSet roots(exprs.begin(), exprs.end());
  UOpMap<size_t> topo_idx;
  for (size_t i = 0; i < order.size(); i++) topo_idx[order[i]] = i;

  SchedulePlan plan;
  auto materialize = [&](const UOp& node) {
    UOp kexpr = substitute_materialized(node, plan.replacements);
    ScheduleItem item = parameterize(kexpr, opt);
    plan.replacements[node] = buffer_replacement(item);
    plan.items.push_back(std::move(item));
  };
  // Reduces held back to run as the epilogue of the elementwise node they
  // feed (fusing only), keyed by that node. Value-preserving: the kernel
  // applies the same elementwise ops to the same reduced values.
  UOpMap<UOp> deferred;
  for (auto& node : order) {
    auto d = deferred.find(node);
    if (d != deferred.end()) {
      // The reduce stays fused only if this node gets a kernel of its own and
      // that kernel computes no other reduction.
      bool own_kernel = roots.count(node) ||
                        should_materialize(node, roots, consumers, nested, opt, topo_idx, plan.replacements);
      if (!own_kernel || has_unmaterialized_reduce(node, plan.replacements, d->second)) materialize(d->second);
      deferred.erase(d);
    }
    if (!should_materialize(node, roots, consumers, nested, opt, topo_idx, plan.replacements)) continue;
    if (opt.fuse && node.op() == Op::ReduceAxis && !is_held(node, opt)) {
      UOp c = epilogue_consumer(node, consumers, roots);
      // One reduce per consumer; and not into a root that other nodes read
      // (roots are computed inline by their readers until the end).
      bool root_read = false;
      if (c && roots.count(c) && consumers.count(c))
        for (auto& r : consumers.at(c)) root_read = root_read || r != uni;
      if (c && !root_read && !deferred.count(c)) {
        deferred[c] = node;
        continue;
      }
    }
    materialize(node);
  }
  if (opt.fuse) {
    // Every node the reference materialises runs in phase 1, ahead of every
    // root, and so reads each buffer before any in-place store of this
    // schedule (schedule.rs:88-121). The fusions above move some of those
    // nodes into the kernels that read them: skipped identity copies, deferred
    // reduce epilogues, recomputed cheap nodes and small reductions. Inside
    // root i such a node runs after the stores of roots 0..i, so when it reads
    // a buffer one of them stores it is materialised here instead, still ahead
    // of every root, and reads what the reference's kernel would have read.
    ScheduleOptions ref_opt = opt;
    ref_opt.fuse = false;
    std::unordered_set<const BufferInner*> stored;
    for (auto& expr : exprs) {
      UOp st, val;
      if (assignment_effect(expr, &st, &val)) {
        UOp d = st.src(0);
        while (is_movement(d.op())) d = d.src(0);
        if (d.op() == Op::Buffer && d.arg().buf) stored.insert(d.arg().buf.get());
      }
      if (stored.empty()) continue;
      // The nodes this root's kernel computes (the walk stops at nodes that
      // already have a buffer), children first, and whether each reads a
      // stored buffer.
      std::vector<UOp> order;
      UOpMap<bool> reads;
      std::vector<std::pair<UOp, bool>> stack{{expr, false}};
      while (!stack.empty()) {
        auto [n, expanded] = stack.back();
        stack.pop_back();
        if (reads.count(n)) continue;
        if (!expanded) {
          if (n != expr && plan.replacements.count(n)) {
            reads[n] = false;
            continue;
          }
          stack.emplace_back(n, true);
          for (auto& s : n.srcs())
            if (!reads.count(s)) stack.emplace_back(s, false);
          continue;
        }
        bool r = n.op() == Op::Buffer && n.arg().buf && stored.count(n.arg().buf.get());
        for (auto& s : n.srcs()) r = r || reads.at(s);
        reads[n] = r;
        order.push_back(n);
      }
      for (auto& n : order) {
        if (n == expr || !reads.at(n)) continue;
        if (should_materialize(n, roots, consumers, nested, ref_opt, topo_idx, plan.replacements)) materialize(n);
      }
    }
  }
  for (auto& expr : exprs) {
    UOp fin = substitute_materialized(expr, plan.replacements);
    UOp store, value;
    if (assignment_effect(fin, &store, &value)) {
      plan.items.push_back(parameterize_store(store, opt));
      plan.replacements[expr] = value;
    } else {
      ScheduleItem item = parameterize(fin, opt);
      plan.replacements[expr] = buffer_replacement(item);
      plan.items.push_back(std::move(item));
    }
  }
  return plan;
}

std::vector<ScheduleItem> schedule(const UOp& expr, const ScheduleOptions& opt) {
  return schedule_many({expr}, opt).items;
}

// ── rangeify ────────────────────────────────────────────────────────────────
namespace {

// indexing.rs:42-62
UOp flat_index(const std::vector<UOp>& idxs, const std::vector<size_t>& strides) {
  FG_CHECK(idxs.size() == strides.size() && !idxs.empty(), "flat_index requires matching indices");
  DeviceId d = idxs[0].device();
  UOp acc;
  for (size_t i = 0; i < idxs.size(); i++) {
    if (strides[i] == 0) continue;
    UOp term = strides[i] == 1
                   ? idxs[i]
                   : UOp::mul(idxs[i], UOp::const_int(static_cast<int64_t>(strides[i]), DType::I32(), idxs[i].device()));
    acc = acc ? UOp::add(acc, term) : term;
  }
  return acc ? acc : UOp::const_int(0, DType::I32(), d);
}

UOp index_wrap(const UOp& src, const std::vector<UOp>& idxs) {  // indexing.rs:66-70
  std::vector<UOp> s{src};
  s.insert(s.end(), idxs.begin(), idxs.end());
  return UOp::make_new(Op::Index, src.dtype(), s, Arg::none());
}

bool same_squeezed_dims(const Shape& a, const Shape& b) {  // indexing.rs:76-80
  std::vector<size_t> x, y;
  for (auto d : a) if (d != 1) x.push_back(d);
  for (auto d : b) if (d != 1) y.push_back(d);
  return x == y;
}

UOp rewrite_index_alu(const UOp& inner, const std::vector<UOp>& idxs) {  // indexing.rs:85-97
  std::vector<UOp> ns;
  for (auto& s : inner.srcs()) ns.push_back(index_wrap(s, idxs));
  if (inner.has_tag()) return UOp::make(inner.op(), inner.dtype(), ns, inner.arg(), true, inner.tag());
  return UOp::make_new(inner.op(), inner.dtype(), ns, inner.arg());
}

// indexing.rs:102-175
UOp rewrite_index_movement(const UOp& inner, const std::vector<UOp>& idxs) {
  const UOp& src = inner.src(0);
  std::vector<UOp> ni;
  // A reshape that is not a squeeze flattens to one index (indexing.rs:167);
  // only a one-dimensional buffer can consume it. Any view of rank > 1 under
  // such a reshape (a permute, or the Reshape(Buffer, shape) that every
  // created or realised tensor is, tensor.rs:260-284, schedule.rs:340-353)
  // receives one index for several dimensions, and the reference's
  // flat_index assertion panics (indexing.rs:42-46): report it instead.
  Shape inner_shape;
  if (inner.op() != Op::Contiguous && inner.shape_opt(&inner_shape) && idxs.size() != inner_shape.size())
    fail(std::string("rangeify: ") + op_name(inner.op()) + " of rank " + std::to_string(inner_shape.size()) +
         " indexed with " + std::to_string(idxs.size()) +
         " indices (a reshape that is not a squeeze reaches a view of several dimensions; the reference's index "
         "rules support it only over a one-dimensional buffer)");
  switch (inner.op()) {
    case Op::Shrink:
      for (size_t ax = 0; ax < idxs.size(); ax++) {
        const UOp& start = inner.src(ax + 1);
        ni.push_back(start.is_zero() ? idxs[ax] : UOp::add(idxs[ax], start));
      }
      break;
    case Op::Expand: {
      Shape ss;
      if (!src.shape_opt(&ss)) return UOp();
      const auto& ex = inner.arg().v;
      for (size_t ax = 0; ax < idxs.size(); ax++) {
        if (ss[ax] == 1 && ex[ax] > 1) ni.push_back(UOp::const_int(0, DType::I32(), idxs[ax].device()));
        else ni.push_back(idxs[ax]);
      }
      break;
    }
    case Op::Permute: {
      auto inv = invert_permutation(inner.arg().usizes());
      for (auto ax : inv) ni.push_back(idxs[ax]);
      break;
    }
    case Op::Reshape: {
      Shape ss;
      if (!src.shape_opt(&ss)) return UOp();
      Shape ds = inner.arg().usizes();
      if (same_squeezed_dims(ss, ds)) {
        std::vector<UOp> non1;
        for (size_t i = 0; i < idxs.size(); i++) if (ds[i] != 1) non1.push_back(idxs[i]);
        size_t next = 0;
        for (auto d : ss) {
          if (d == 1) ni.push_back(UOp::const_int(0, DType::I32(), src.device()));
          else ni.push_back(non1[next++]);
        }
      } else {
        ni.push_back(flat_index(idxs, contiguous_strides(ds)));
      }
      break;
    }
    case Op::Contiguous:
      ni = idxs;
      break;
    default:
      fail("rangeify only sends movement ops here");
  }
  return index_wrap(src, ni);
}

// indexing.rs:184-217
UOp rewrite_index_reduce(const UOp& inner, const std::vector<UOp>& idxs) {
  const UOp& src = inner.src(0);
  Shape ss;
  if (!src.shape_opt(&ss)) return UOp();
  FG_CHECK(idxs.size() == ss.size(), "idxs should match source ndim");
  const auto& axes = inner.arg().v;
  std::vector<UOp> full, rr;
  for (size_t ax = 0; ax < ss.size(); ax++) {
    if (std::find(axes.begin(), axes.end(), static_cast<int64_t>(ax)) != axes.end()) {
      UOp bound = UOp::const_int(static_cast<int64_t>(ss[ax]), DType::I32(), src.device());
      UOp r = UOp::make_new(Op::Range, DType::I32(), {bound}, Arg::range(static_cast<int64_t>(ax), AxisKind::Reduce));
      full.push_back(r);
      rr.push_back(r);
    } else {
      full.push_back(idxs[ax]);
    }
  }
  std::vector<UOp> srcs{index_wrap(src, full)};
  srcs.insert(srcs.end(), rr.begin(), rr.end());
  return UOp::make_new(Op::Reduce, inner.dtype(), srcs, Arg::reduce(inner.arg().rop, {}));
}

UOp rewrite_index_param(const UOp& inner, const std::vector<UOp>& idxs) {  // indexing.rs:233-242
  FG_CHECK(idxs.size() == 1, "Param should have exactly one flat index");
  UOp index = UOp::make_new(Op::Index, inner.dtype(), {inner, idxs[0]}, Arg::index(0));
  return UOp::make_new(Op::Load, inner.dtype(), {index}, Arg::none());
}

UOp new_range(size_t axis, size_t size, DeviceId d) {  // rangeify.rs:42-52
  if (size == 1) return UOp::const_int(0, DType::I32(), d);
  return UOp::make_new(Op::Range, DType::I32(), {UOp::const_int(static_cast<int64_t>(size), DType::I32(), d)},
                       Arg::range(static_cast<int64_t>(axis), AxisKind::Loop));
}

UOp chain_ends(const std::vector<UOp>& ranges, const UOp& body) {  // rangeify.rs:57-68
  UOp cur = body;
  for (size_t i = ranges.size(); i-- > 0;)
    cur = UOp::make_new(Op::End, DType::Void(), {ranges[i], cur}, Arg::none());
  return cur;
}

UOp store_output_index(const UOp& dest, const std::vector<UOp>& idxs) {  // rangeify.rs:75-96
  if (dest.op() == Op::ParamBuffer || dest.op() == Op::Buffer) {
    FG_CHECK(idxs.size() == 1, "store destination must be flattened before reaching ParamBuffer/Buffer");
    return UOp::make_new(Op::Index, dest.dtype(), {dest, idxs[0]}, Arg::index(0));
  }
  if (is_movement(dest.op())) {
    UOp moved = rewrite_index_movement(dest, idxs);
    if (!moved) return UOp();
    std::vector<UOp> rest(moved.srcs().begin() + 1, moved.srcs().end());
    return store_output_index(moved.src(0), rest);
  }
  return UOp();
}

UOp rewrite_store_add_ranges(const UOp& store) {  // rangeify.rs:118-161
  if (store.srcs().size() != 2) return UOp();
  const UOp& out = store.src(0);
  const UOp& expr = store.src(1);
  Shape s;
  if (!expr.shape_opt(&s)) return UOp();
  DeviceId d = expr.device();
  std::vector<UOp> ax;
  for (size_t i = 0; i < s.size(); i++) ax.push_back(new_range(i, s[i], d));
  UOp indexed = index_wrap(expr, ax);
  UOp out_flat = flat_index(ax, contiguous_strides(s));
  std::vector<UOp> out_ranges;
  for (auto& r : ax) if (r.op() == Op::Range) out_ranges.push_back(r);
  UOp out_idx = out.op() == Op::ParamBuffer
                    ? UOp::make_new(Op::Index, out.dtype(), {out, out_flat}, Arg::index(0))
                    : store_output_index(out, ax);
  if (!out_idx) return UOp();
  UOp ns = UOp::make_new(Op::Store, DType::Void(), {out_idx, indexed}, Arg::none());
  return chain_ends(out_ranges, ns);
}

UOp rangeify_rule(const UOp& node) {  // rangeify.rs:173-194
  if (node.op() == Op::Store) return rewrite_store_add_ranges(node);
  if (node.op() == Op::Index && node.arg().kind == Arg::Kind::None) {
    const UOp& inner = node.src(0);
    std::vector<UOp> idxs(node.srcs().begin() + 1, node.srcs().end());
    Op io = inner.op();
    if (is_alu(io)) return rewrite_index_alu(inner, idxs);
    switch (io) {
      case Op::Expand: case Op::Permute: case Op::Reshape: case Op::Shrink: case Op::Contiguous:
        return rewrite_index_movement(inner, idxs);
      case Op::ReduceAxis: return rewrite_index_reduce(inner, idxs);
      case Op::Const: case Op::ParamScalar: return inner;
      case Op::ParamBuffer: return rewrite_index_param(inner, idxs);
      default: return UOp();
    }
  }
  return UOp();
}

}  // namespace

UOp rangeify(const UOp& sink) { return graph_rewrite(sink, rangeify_rule); }

}  // namespace fg
