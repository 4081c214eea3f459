// Tensor front end, realisation driver, autograd, Linear and SGD.
// Follows src/tensor.rs, src/gradient.rs, src/nn.rs and src/optim.rs.
#include "tensor.hpp"

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <unordered_set>

namespace fg {

namespace {

// tensor.rs:79-81 — weak handles to every live tensor.
std::vector<std::weak_ptr<TensorInner>>& live_list() {
  static auto* v = new std::vector<std::weak_ptr<TensorInner>>();
  return *v;
}

size_t g_kernel_count = 0;  // tensor.rs:71

uint64_t now_ns() {
  return static_cast<uint64_t>(
      std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now().time_since_epoch()).count());
}

// Lowering cache: scheduled kernel sink -> compiled program, per device. The
// sink is interned, and rangeify/optimize/render are pure functions of it, so a
// hit skips the host passes as well as the compile (the reference caches by
// the lowered sink and re-runs the passes every realize: tensor.rs:804-846).
UOpMap<std::shared_ptr<Program>>& lowering_cache(DeviceId d) {
  static UOpMap<std::shared_ptr<Program>> caches[2];
  return caches[static_cast<int>(d)];
}

}  // namespace

RealizeStats& realize_stats() {
  static RealizeStats s;
  return s;
}

int debug_level() {  // tensor.rs:62-67
  static int lvl = [] {
    const char* e = std::getenv("DEBUG");
    return e ? std::atoi(e) : 0;
  }();
  return lvl;
}

void clear_kernel_caches() {
  clear_plan_cache();
  for (int d = 0; d < 2; d++) {
    lowering_cache(static_cast<DeviceId>(d)).clear();
    if (has_device(static_cast<DeviceId>(d))) get_device(static_cast<DeviceId>(d)).clear_for_tests();
  }
}

Tensor Tensor::from_uop(const UOp& u, bool rg) {  // tensor.rs:151-159
  auto inner = std::make_shared<TensorInner>();
  inner->uop = u;
  inner->requires_grad = rg;
  live_list().push_back(inner);
  return Tensor(inner);
}

static std::vector<Tensor> live_tensors() {  // tensor.rs:201-214
  std::vector<Tensor> out;
  auto& l = live_list();
  size_t w = 0;
  for (size_t i = 0; i < l.size(); i++) {
    if (auto p = l[i].lock()) {
      out.emplace_back(p);
      l[w++] = l[i];
    }
  }
  l.resize(w);
  return out;
}

// A tensor at a view (reshape, permute, expand, shrink) of a node is repointed
// when that node is materialised (apply_map_to_tensors substitutes through the
// view), so the first node under the views counts as held too.
void collect_held_nodes(PtrIndexMap* held, std::vector<const UOpInner*>* list) {
  auto add = [&](const UOpInner* raw) {
    const size_t before = held->size();
    held->put(raw, 1);
    if (list && held->size() != before) list->push_back(raw);
  };
  for (auto& w : live_list()) {
    if (auto p = w.lock()) {
      const UOpInner* raw = p->uop.get();
      add(raw);
      while (is_movement(raw->op) && !raw->srcs.empty()) raw = raw->srcs[0].get();
      add(raw);
    }
  }
}

UOp Tensor::uop() const { return p_->uop; }
void Tensor::set_uop(const UOp& u) const { p_->uop = u; }

// tensor.rs:222-252
// Every live tensor whose graph reaches a replaced node is repointed at the
// substituted graph. One memoised walk serves all live tensors and stops at
// replaced nodes (the reference toposorts each live tensor's whole graph and
// substitutes over the full graphs; the resulting graphs are the same).
static void apply_map_to_tensors(const UOpMap<UOp>& replacements) {
  if (replacements.empty()) return;
  std::vector<Tensor> live = live_tensors();
  std::vector<UOp> roots;
  roots.reserve(live.size());
  for (auto& t : live) roots.push_back(t.uop());
  std::vector<UOp> subst = substitute_many(roots, replacements);
  for (size_t i = 0; i < live.size(); i++)
    if (subst[i] != roots[i]) live[i].set_uop(subst[i]);
}

Tensor Tensor::from_bytes(const void* data, size_t nbytes, const Shape& shape, DType dtype, DeviceId dev) {
  size_t n = fg::numel(shape);
  FG_CHECK(nbytes == n * dtype.size_bytes(),
           "data length " + std::to_string(nbytes / std::max<size_t>(1, dtype.size_bytes())) +
               " doesn't match shape " + shape_str(shape));
  Device& backend = get_device(dev);
  Buffer b = backend.allocate(dtype, n);
  backend.copy_from_host(b, data, nbytes);
  return from_uop(UOp::reshape(UOp::buffer(b, dtype, dev), shape), false);
}

Tensor Tensor::new_f32(const std::vector<float>& data, const Shape& shape, DeviceId dev) {
  return from_bytes(data.data(), data.size() * 4, shape, DType::F32(), dev);
}

Tensor Tensor::zeros(const Shape& shape, DeviceId dev, DType dtype) {  // tensor.rs:278-284
  Device& backend = get_device(dev);
  Buffer b = backend.allocate(dtype, fg::numel(shape));
  return from_uop(UOp::reshape(UOp::buffer(b, dtype, dev), shape), false);
}

Tensor Tensor::ones(const Shape& shape, DeviceId dev, DType dtype) {  // tensor.rs:292-299
  size_t n = fg::numel(shape);
  switch (dtype.kind) {
    case DTypeKind::F32: return full_f32(shape, 1.0f, dev);
    case DTypeKind::I32: {
      std::vector<int32_t> d(n, 1);
      return from_bytes(d.data(), n * 4, shape, dtype, dev);
    }
    case DTypeKind::Bool: {
      std::vector<uint8_t> d(n, 1);
      return from_bytes(d.data(), n, shape, dtype, dev);
    }
    default: fail("ones requires a concrete dtype");
  }
}

Tensor Tensor::full_f32(const Shape& shape, float v, DeviceId dev) {
  std::vector<float> d(fg::numel(shape), v);
  return new_f32(d, shape, dev);
}

Tensor Tensor::scalar_f32(float v, DeviceId dev) { return new_f32({v}, Shape{1}, dev); }

DeviceId Tensor::device() const { return uop().device(); }
DType Tensor::dtype() const { return uop().dtype(); }
Shape Tensor::shape() const { return uop().shape(); }
const Shape& Tensor::shape_ref() const { return p_->uop.shape_ref(); }
size_t Tensor::numel() const { return fg::numel(shape()); }
size_t Tensor::ndim() const { return shape().size(); }

bool Tensor::is_realized() const {  // tensor.rs:351-358
  UOp u = uop();
  if (u.op() == Op::Buffer) return true;
  if (u.op() == Op::Reshape) return u.src(0).op() == Op::Buffer;
  return false;
}

bool Tensor::requires_grad() const { return p_->requires_grad; }
std::optional<Tensor> Tensor::grad() const {
  if (!p_->grad) return std::nullopt;
  return Tensor(p_->grad);
}
void Tensor::clear_grad() const { p_->grad.reset(); }
Tensor Tensor::with_requires_grad(bool rg) const {
  p_->requires_grad = rg;
  return *this;
}
Tensor Tensor::detach() const { return from_uop(uop(), false); }

Tensor Tensor::replace(const Tensor& o) const {  // tensor.rs:399-409
  FG_CHECK(shape() == o.shape(), "replace: shape mismatch " + shape_str(shape()) + " != " + shape_str(o.shape()));
  set_uop(o.uop());
  return *this;
}

UOp Tensor::target_uop() const {  // tensor.rs:189-195
  UOp cur = uop();
  if (cur.op() == Op::After) return cur.src(0);
  return cur;
}

Tensor Tensor::assign(const Tensor& o) const {  // tensor.rs:421-440
  FG_CHECK(shape() == o.shape(), "assign: shape mismatch " + shape_str(shape()) + " != " + shape_str(o.shape()));
  FG_CHECK(dtype() == o.dtype(), "assign: dtype mismatch");
  FG_CHECK(device() == o.device(), "assign: device mismatch");
  UOp target = target_uop();
  FG_CHECK(target.has_buffer_identity(), "assign requires a tensor with concrete buffer identity");
  UOp effect = UOp::store(target, o.uop());
  set_uop(UOp::after(target, effect));
  return *this;
}

Tensor Tensor::unary(Op op) const {
  return from_uop(UOp::make_new(op, dtype(), {uop()}, Arg::none()), requires_grad());
}

Tensor Tensor::binary(const Tensor& o, Op op, DType out) const {  // tensor.rs:449-459
  FG_CHECK(device() == o.device(), "binary ops require tensors on the same device");
  FG_CHECK(shape_ref() == o.shape_ref(), std::string("shape mismatch for ") + op_name(op));
  return from_uop(UOp::make_new(op, out, {uop(), o.uop()}, Arg::none()), requires_grad() || o.requires_grad());
}

// One side of a broadcast: the reshape to `target`'s rank and the expand to
// `target`, as tensor.rs:1068-1092 builds them (each step skipped when it
// would not change the shape), without a Tensor for each intermediate view.
static UOp broadcast_side(const UOp& u, const Shape& target) {
  const Shape& s = u.shape_ref();
  Shape padded = pad_left(s, target.size());
  UOp r = padded == s ? u : UOp::reshape(u, padded);
  return padded == target ? r : UOp::expand(r, target);
}

Tensor Tensor::broadcasted(const Tensor& o, Op op, DType out) const {  // tensor.rs:461-467, 1068-1092
  if (shape_ref() == o.shape_ref()) return binary(o, op, out);
  FG_CHECK(device() == o.device(), "broadcast requires tensors on the same device");
  Shape target;
  FG_CHECK(broadcast_with(shape_ref(), o.shape_ref(), &target),
           "broadcast: incompatible dims for " + shape_str(shape()) + " vs " + shape_str(o.shape()));
  UOp l = broadcast_side(uop(), target), r = broadcast_side(o.uop(), target);
  return from_uop(UOp::make_new(op, out, {l, r}, Arg::none()), requires_grad() || o.requires_grad());
}

Tensor Tensor::add(const Tensor& o) const { return broadcasted(o, Op::Add, dtype()); }
Tensor Tensor::mul(const Tensor& o) const { return broadcasted(o, Op::Mul, dtype()); }
Tensor Tensor::neg() const { return unary(Op::Neg); }
Tensor Tensor::sub(const Tensor& o) const { return add(o.neg()); }
Tensor Tensor::reciprocal() const { return unary(Op::Reciprocal); }
Tensor Tensor::exp2() const { return unary(Op::Exp2); }
Tensor Tensor::log2() const { return unary(Op::Log2); }
Tensor Tensor::sqrt() const { return unary(Op::Sqrt); }

// relu's zeros (tensor.rs:517-531). The reference allocates a fresh zero
// tensor at every call; that buffer is never handed out or written, so on a
// device that allows it (the HIP device) one zero buffer per (dtype, shape)
// gives the same graphs and values without a buffer per call, and a loop
// that rebuilds the same relu gets the same graph nodes every time. At most
// 64 shapes are kept; past that the cache starts over (buffers in use stay
// alive through their graphs). Other devices allocate per call.
static UOp relu_zeros(const Shape& shape, DeviceId dev, DType dt) {
  Device& backend = get_device(dev);
  if (!backend.shares_relu_zeros())
    return UOp::reshape(UOp::buffer(backend.allocate(dt, fg::numel(shape)), dt, dev), shape);
  struct Entry {
    DeviceId dev;
    DType dt;
    Shape shape;
    UOp zeros;
  };
  static auto* cache = new std::vector<Entry>();
  for (auto& e : *cache)
    if (e.dev == dev && e.dt == dt && e.shape == shape) return e.zeros;
  if (cache->size() >= 64) cache->clear();
  Buffer b = backend.allocate(dt, fg::numel(shape));
  cache->push_back({dev, dt, shape, UOp::reshape(UOp::buffer(b, dt, dev), shape)});
  return cache->back().zeros;
}

Tensor Tensor::relu() const {  // tensor.rs:517-531
  const UOp zero = relu_zeros(shape_ref(), device(), dtype());
  const UOp cond = UOp::make_new(Op::CmpLt, DType::Bool(), {zero, uop()}, Arg::none());
  return from_uop(UOp::make_new(Op::Where, dtype(), {cond, uop(), zero}, Arg::none()), requires_grad());
}

// A constant the library itself builds into graphs (LOG2_E in exp, LN_2 in
// log, 1/n in cross_entropy). The reference creates a fresh scalar buffer at
// every call (tensor.rs:697-750); these buffers are never handed out or
// written, so one buffer per (device, value) gives the same graphs and values
// without an allocation and a host->device copy per call. The cache is never
// destroyed: its buffers live until the process ends.
static Tensor constant_scalar(float v, DeviceId dev) {
  static auto* cache = new std::vector<std::pair<std::pair<DeviceId, uint32_t>, Tensor>>();
  uint32_t bits = 0;
  std::memcpy(&bits, &v, 4);
  for (auto& [k, t] : *cache)
    if (k.first == dev && k.second == bits) return t;
  cache->emplace_back(std::make_pair(dev, bits), Tensor::scalar_f32(v, dev));
  return cache->back().second;
}

Tensor Tensor::exp() const {  // tensor.rs:697-700 (f32 LOG2_E)
  Tensor log2e = constant_scalar(1.44269504088896340736f, device());
  return mul(log2e).exp2();
}

Tensor Tensor::log() const {  // tensor.rs:704-707 (f32 LN_2)
  Tensor ln2 = constant_scalar(0.693147180559945309417f, device());
  return log2().mul(ln2);
}

Tensor Tensor::reshape(const Shape& ns) const {  // tensor.rs:539-552
  if (shape() == ns) return *this;
  FG_CHECK(numel() == fg::numel(ns), "reshape: numel mismatch for " + shape_str(shape()) + " -> " + shape_str(ns));
  return from_uop(UOp::reshape(uop(), ns), requires_grad());
}

Tensor Tensor::narrow(size_t dim, size_t start, size_t len) const {  // tensor.rs:561-603
  Shape s = shape();
  FG_CHECK(dim < s.size(), "narrow: dim " + std::to_string(dim) + " out of range");
  size_t end = start + len;
  FG_CHECK(end <= s[dim], "narrow: range [" + std::to_string(start) + ", " + std::to_string(end) +
                              ") out of bounds for axis " + std::to_string(dim) + " with size " +
                              std::to_string(s[dim]));
  if (start == 0 && len == s[dim]) return *this;
  std::vector<UOp> starts;
  std::vector<size_t> lens;
  for (size_t ax = 0; ax < s.size(); ax++) {
    starts.push_back(UOp::const_int(ax == dim ? static_cast<int64_t>(start) : 0, DType::I32(), device()));
    lens.push_back(ax == dim ? len : s[ax]);
  }
  return from_uop(UOp::shrink(uop(), starts, lens), requires_grad());
}

Tensor Tensor::permute(const std::vector<size_t>& order) const {  // tensor.rs:611-621
  size_t nd = ndim();
  FG_CHECK(order.size() == nd, "permute: wrong number of axes");
  std::vector<bool> seen(nd, false);
  for (auto ax : order) {
    FG_CHECK(ax < nd, "permute: axis " + std::to_string(ax) + " out of range");
    FG_CHECK(!seen[ax], "permute: axis " + std::to_string(ax) + " duplicated");
    seen[ax] = true;
  }
  return from_uop(UOp::permute(uop(), order), requires_grad());
}

Tensor Tensor::contiguous() const {  // tensor.rs:625-630
  if (is_realized()) return *this;
  return from_uop(UOp::contiguous(uop()), requires_grad());
}

Tensor Tensor::expand(const Shape& ns) const {  // tensor.rs:638-657
  if (shape() == ns) return *this;
  Shape s = shape();
  FG_CHECK(s.size() == ns.size(), "expand: rank mismatch for " + shape_str(s) + " -> " + shape_str(ns));
  for (size_t i = 0; i < s.size(); i++)
    FG_CHECK(s[i] == ns[i] || s[i] == 1, "expand: incompatible source shape " + shape_str(s) + " -> " + shape_str(ns));
  return from_uop(UOp::expand(uop(), ns), requires_grad());
}

Tensor Tensor::sum(const std::vector<size_t>& axes) const {  // tensor.rs:665-675
  size_t nd = ndim();
  for (auto a : axes) FG_CHECK(a < nd, "sum: axes out of range for ndim " + std::to_string(nd));
  return from_uop(UOp::reduce_axis(uop(), Op::Add, axes), requires_grad());
}

Tensor Tensor::max(const std::vector<size_t>& axes) const {  // tensor.rs:683-693
  size_t nd = ndim();
  for (auto a : axes) FG_CHECK(a < nd, "max: axes out of range for ndim " + std::to_string(nd));
  return from_uop(UOp::reduce_axis(uop(), Op::Max, axes), requires_grad());
}

Tensor Tensor::log_softmax(size_t axis) const {  // tensor.rs:715-721
  FG_CHECK(axis < ndim(), "log_softmax: axis " + std::to_string(axis) + " out of range");
  Tensor mx = max({axis});
  Tensor shifted = sub(mx);
  Tensor se = shifted.exp().sum({axis});
  return shifted.sub(se.log());
}

Tensor Tensor::cross_entropy(const Tensor& targets) const {  // tensor.rs:738-752
  FG_CHECK(shape() == targets.shape(), "cross_entropy: target shape " + shape_str(targets.shape()) +
                                            " must match logits shape " + shape_str(shape()));
  size_t cax = ndim() != 1 ? 1 : 0;
  Tensor lp = log_softmax(cax);
  Tensor per = targets.mul(lp).sum({cax}).neg();
  std::vector<size_t> red;
  for (size_t i = 0; i < per.ndim(); i++) red.push_back(i);
  Tensor scale = constant_scalar(1.0f / static_cast<float>(per.numel()), device());
  return per.sum(red).mul(scale);
}

Tensor Tensor::matmul(const Tensor& other) const {  // tensor.rs:762-778
  FG_CHECK(ndim() == 2, "matmul: lhs must be 2D");
  FG_CHECK(other.ndim() == 2, "matmul: rhs must be 2D");
  Shape ls = shape(), rs = other.shape();
  size_t m = ls[0], k = ls[1], k2 = rs[0], n = rs[1];
  FG_CHECK(k == k2, "matmul: inner dim mismatch (" + std::to_string(k) + " vs " + std::to_string(k2) + ")");
  Tensor a = reshape({m, 1, k}).expand({m, n, k});
  // other.permute([1, 0]).contiguous(), tagged as matmul's own copy.
  Tensor t = other.permute({1, 0});
  Tensor tc = t.is_realized() ? t
                              : from_uop(UOp::make_tagged(Op::Contiguous, t.dtype(), {t.uop()}, Arg::none(),
                                                          kMatmulCopyTag),
                                         t.requires_grad());
  Tensor b = tc.reshape({1, n, k}).expand({m, n, k});
  return a.mul(b).sum({2}).reshape({m, n});
}

// tensor.rs:1097-1121
static void assert_kernel_ready(const UOp& root) {
  FG_CHECK(root.op() == Op::Sink, "render: root must be a Sink node");
  for (auto& n : root.toposort()) {
    switch (n.op()) {
      case Op::DefineVar: case Op::Bind: case Op::Buffer: case Op::Shrink: case Op::Reshape:
      case Op::Permute: case Op::Expand: case Op::Contiguous: case Op::ReduceAxis:
        fail(std::string(op_name(n.op())) + " should be lowered before codegen");
      default: break;
    }
  }
}

// tensor.rs:831-898
static std::shared_ptr<Program> execute_item(const ScheduleItem& item) {
  const uint64_t start_ns = now_ns();
  Device& backend = get_device(item.sink.device());
  int debug = debug_level();
  size_t num_args = item.output_buffer ? item.inputs.size() + 1 : item.inputs.size();
  auto& lc = lowering_cache(backend.id());
  std::shared_ptr<Program> program;
  auto hit = lc.find(item.sink);
  if (hit != lc.end()) {
    program = hit->second;
    realize_stats().lowering_cache_hits++;
    if (debug >= 1) {
      size_t kid = g_kernel_count++;
      std::fprintf(stderr, "*** %s %4zu  (cached)         arg %2zu\n", backend.id() == DeviceId::Hip ? "HIP" : "CPU",
                   kid, num_args);
    }
  } else {
    if (debug >= 3) std::fprintf(stderr, "━━━ rangeify [before] ━━━\n%s", item.sink.dump().c_str());
    UOp rangeified = rangeify(item.sink);
    if (debug >= 3) std::fprintf(stderr, "━━━ optimize [before] ━━━\n%s", rangeified.dump().c_str());
    UOp optimized = backend.bind_params(backend.optimize(rangeified), item.sink);
    if (debug >= 3) std::fprintf(stderr, "━━━ codegen [before] ━━━\n%s", optimized.dump().c_str());
    assert_kernel_ready(optimized);
    program = backend.cached_program(optimized);
    if (program) {
      if (debug >= 1) {
        size_t kid = g_kernel_count++;
        std::fprintf(stderr, "*** %s %4zu  (cached)         arg %2zu\n",
                     backend.id() == DeviceId::Hip ? "HIP" : "CPU", kid, num_args);
      }
    } else {
      size_t kid = g_kernel_count++;
      std::string name = "kernel_" + std::to_string(kid);
      RenderedKernel rk = backend.render(optimized, name);
      if (debug >= 4) std::fprintf(stderr, "%s\n", rk.source.c_str());
      program = backend.compile(rk, num_args);
      realize_stats().programs_compiled++;
      if (debug >= 1)
        std::fprintf(stderr, "*** %s %4zu  %-16s arg %2zu  [%s]\n", backend.id() == DeviceId::Hip ? "HIP" : "CPU", kid,
                     name.c_str(), num_args, rk.kind.c_str());
      backend.insert_program(optimized, program);
    }
    lc[item.sink] = program;
  }

  std::vector<KernelArg> args;
  args.reserve(num_args);
  if (item.output_buffer) {
    // The store covers every output element, so the output needs no zero fill.
    if (!item.output_buffer->is_realized()) backend.realize_storage(*item.output_buffer, false);
    item.output_buffer->known_zero = false;
    args.push_back(KernelArg::buf(item.output_buffer));
  }
  for (auto& in : item.inputs) {
    if (in.kind == KernelArg::Kind::Buffer && !in.buffer->is_realized()) {
      // Zero-initialised allocations may be materialised lazily by the device.
      FG_CHECK(in.buffer->zero_init, "scheduled input buffer missing");
      backend.realize_storage(*in.buffer, true);
    }
    args.push_back(in);
  }
  auto t0 = std::chrono::steady_clock::now();
  uint64_t l0 = now_ns();
  realize_stats().ns_lower += l0 - start_ns;
  backend.execute(*program, args);
  realize_stats().ns_launch += now_ns() - l0;
  realize_stats().kernels_launched++;
  if (debug >= 2) {
    backend.synchronize();
    double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    std::fprintf(stderr, "              exec time=%.3fms\n", ms);
  }
  return program;
}

// ── plan cache ──────────────────────────────────────────────────────────────
// schedule_many is a pure function of the lazy graph's structure, of which
// buffers are shared between leaves, and of which leaf buffers still hold
// allocate()'s zeros (zero-folding). A train loop rebuilds the same structure
// over the same parameter buffers every step, so the whole realisation (kernel
// partition, parameter slots, programs, argument wiring, replacement map) is
// recorded once per structure and replayed: no rewrites, no interning beyond
// the replacement buffers. The key is an exact serialisation, compared in full
// on a hash match.
namespace {

struct GraphKey {
  std::vector<UOp> order;            // toposort of Sink(roots)
  std::vector<Buffer> leaves;        // distinct buffers, first-visit order
  std::vector<uint64_t> code;        // exact structural serialisation
  std::vector<uint32_t> scalar_nodes;  // positions of parameterised Shrink starts
  uint64_t hash = 0;
};

void key_word(GraphKey& k, uint64_t w) { k.code.push_back(w); }

// A depth-first walk yields the toposort (the order UOp::toposort produces:
// sources first, left to right, except After which walks its effect first),
// using one open-addressing map for the visited set and node positions; a
// second pass serialises it.
//
// Integer constants used only as Shrink starts that parameterize turns into
// ParamScalar kernel arguments (schedule.rs:217-239) are serialised without
// their value: narrow(0, start, len) over successive batches is then one plan,
// and replays read the start from the current graph (scalar_nodes).
GraphKey graph_key(const std::vector<UOp>& roots, bool fuse, const std::vector<const UOpInner*>* held) {
  GraphKey k;
  const UOp sink = UOp::sink(roots);
  PtrIndexMap pos(128);  // grows on demand
  PtrIndexMap leaf(32);
  k.order.reserve(128);
  std::vector<std::pair<const UOp*, bool>> stack;
  stack.reserve(64);
  stack.emplace_back(&sink, false);
  bool has_bind = false;
  while (!stack.empty()) {
    auto [np, processed] = stack.back();
    stack.pop_back();
    const UOpInner* raw = np->get();
    if (pos.get(raw) != PtrIndexMap::kAbsent) continue;
    const auto& srcs = raw->srcs;
    if (!processed) {
      stack.emplace_back(np, true);
      if (raw->op == Op::After) {
        for (size_t i = 0; i < srcs.size(); i++)
          if (pos.get(srcs[i].get()) == PtrIndexMap::kAbsent) stack.emplace_back(&srcs[i], false);
      } else {
        for (size_t i = srcs.size(); i-- > 0;)
          if (pos.get(srcs[i].get()) == PtrIndexMap::kAbsent) stack.emplace_back(&srcs[i], false);
      }
      continue;
    }
    pos.set(raw, static_cast<uint32_t>(k.order.size()));
    k.order.push_back(*np);
    has_bind = has_bind || raw->op == Op::Bind;
  }
  // Which integer constants are parameterised Shrink starts and nothing else
  // (1 = such a use seen, 2 = another use seen).
  std::vector<uint8_t> use(k.order.size(), 0);
  if (!has_bind) {
    for (auto& n : k.order) {
      const auto& srcs = n.srcs();
      Shape src_shape;
      bool shrink = n.op() == Op::Shrink && srcs[0].shape_opt(&src_shape);
      for (size_t j = 0; j < srcs.size(); j++) {
        if (srcs[j].op() != Op::Const || srcs[j].dtype() != DType::I32()) continue;
        uint32_t sp = pos.get(srcs[j].get());
        bool param = shrink && j >= 1 && j - 1 < n.arg().v.size() &&
                     static_cast<size_t>(n.arg().v[j - 1]) != src_shape[j - 1];
        use[sp] |= param ? 1 : 2;
      }
    }
  }
  k.code.reserve(k.order.size() * 8 + 4);
  key_word(k, fuse ? 1 : 0);
  for (uint32_t i = 0; i < k.order.size(); i++) {
    const UOpInner* raw = k.order[i].get();
    const auto& srcs = raw->srcs;
    const Arg& a = raw->arg;
    key_word(k, static_cast<uint64_t>(raw->op) | (static_cast<uint64_t>(raw->dtype.kind) << 8) |
                    (static_cast<uint64_t>(raw->dtype.vcount) << 16) | (static_cast<uint64_t>(raw->has_tag) << 32) |
                    (static_cast<uint64_t>(a.kind) << 40) | (static_cast<uint64_t>(a.rop) << 48));
    if (raw->has_tag) key_word(k, raw->tag);
    key_word(k, srcs.size());
    for (auto& s : srcs) key_word(k, pos.get(s.get()));
    if (use[i] == 1) {
      key_word(k, 0x5354415254ULL);  // a start value supplied per replay
      k.scalar_nodes.push_back(i);
      continue;
    }
    if (a.kind == Arg::Kind::Buffer) {
      const Buffer& b = a.buf;
      if (!b) {
        key_word(k, ~uint64_t(0));
        continue;
      }
      uint32_t li = leaf.put(b.get(), static_cast<uint32_t>(k.leaves.size()));
      if (li == k.leaves.size()) k.leaves.push_back(b);
      key_word(k, li);
      key_word(k, static_cast<uint64_t>(b->dtype.kind) | (static_cast<uint64_t>(b->known_zero) << 8) |
                      (static_cast<uint64_t>(b->device) << 16));
      key_word(k, b->numel);
      continue;
    }
    uint64_t fbits;
    std::memcpy(&fbits, &a.f, sizeof(fbits));
    key_word(k, static_cast<uint64_t>(a.a));
    key_word(k, static_cast<uint64_t>(a.b));
    key_word(k, static_cast<uint64_t>(a.c));
    key_word(k, fbits);
    key_word(k, a.v.size());
    for (auto x : a.v) key_word(k, static_cast<uint64_t>(x));
    key_word(k, a.name.size());
    for (size_t c = 0; c < a.name.size(); c += 8) {
      uint64_t w = 0;
      std::memcpy(&w, a.name.data() + c, std::min<size_t>(8, a.name.size() - c));
      key_word(k, w);
    }
  }
  if (held) {
    // Which nodes live tensors point at decides the fused partition too.
    std::vector<uint32_t> hp;
    for (const UOpInner* raw : *held) {
      uint32_t p = pos.get(raw);
      if (p != PtrIndexMap::kAbsent) hp.push_back(p);
    }
    std::sort(hp.begin(), hp.end());
    hp.erase(std::unique(hp.begin(), hp.end()), hp.end());
    key_word(k, 0x48454c44ULL);  // "HELD"
    key_word(k, hp.size());
    for (auto p : hp) key_word(k, p);
  }
  uint64_t h = 1469598103934665603ULL;
  for (uint64_t w : k.code) h = (h ^ w) * 1099511628211ULL;
  k.hash = h;
  return k;
}

struct PlanArg {
  enum Kind : uint8_t { Leaf, Output, Value, Start } kind = Value;
  uint32_t index = 0;
  KernelArg value;
};

struct PlanKernel {
  std::shared_ptr<Program> program;
  bool has_output = false;
  DType out_dtype;
  size_t out_numel = 0;
  Shape out_shape;
  std::vector<PlanArg> args;
};

struct PlanReplacement {
  uint32_t node = 0;       // position of the replaced node in the key's order
  int32_t kernel = -1;     // its kernel's output buffer, or
  uint32_t value = 0;      // (kernel < 0) another node of the graph
};

struct CachedPlan {
  std::vector<uint64_t> code;
  std::vector<PlanKernel> kernels;
  std::vector<PlanReplacement> replacements;
  std::vector<uint32_t> written_leaves;  // leaves scheduling marked as overwritten
  mutable std::shared_ptr<void> device_state;  // the device's replay state (Device::execute_sequence)
  mutable std::vector<void*> last_storage;     // each kernel's output storage at the last replay
};

struct PlanCache {
  std::unordered_map<uint64_t, std::vector<std::shared_ptr<CachedPlan>>> map;
  size_t entries = 0;
  bool enabled = true;
  uint64_t hits = 0, misses = 0;
};

PlanCache& plan_cache() {
  static PlanCache* c = new PlanCache();
  return *c;
}

constexpr size_t kMaxCachedPlans = 512;

std::shared_ptr<CachedPlan> find_plan(const GraphKey& k) {
  auto it = plan_cache().map.find(k.hash);
  if (it == plan_cache().map.end()) return nullptr;
  for (auto& p : it->second)
    if (p->code == k.code) return p;
  return nullptr;
}

// Builds a replayable record of a realisation that just ran, or null when some
// part of it is not expressible in terms of the key (then it is not cached).
std::shared_ptr<CachedPlan> record_plan(const GraphKey& k, const SchedulePlan& plan,
                                        const std::vector<std::shared_ptr<Program>>& programs,
                                        const std::vector<uint8_t>& zero_before) {
  auto rec = std::make_shared<CachedPlan>();
  std::unordered_map<const BufferInner*, uint32_t> leaf_of, out_of;
  for (uint32_t i = 0; i < k.leaves.size(); i++) leaf_of.emplace(k.leaves[i].get(), i);
  for (size_t j = 0; j < plan.items.size(); j++) {
    const ScheduleItem& item = plan.items[j];
    PlanKernel pk;
    pk.program = programs[j];
    if (item.output_buffer) {
      pk.has_output = true;
      pk.out_dtype = item.output_buffer->dtype;
      pk.out_numel = item.output_buffer->numel;
      pk.out_shape = item.out_shape;
      out_of.emplace(item.output_buffer.get(), static_cast<uint32_t>(j));
    }
    for (auto& in : item.inputs) {
      PlanArg pa;
      if (in.kind == KernelArg::Kind::Buffer) {
        auto l = leaf_of.find(in.buffer.get());
        auto o = out_of.find(in.buffer.get());
        if (l != leaf_of.end()) {
          pa.kind = PlanArg::Leaf;
          pa.index = l->second;
        } else if (o != out_of.end()) {
          pa.kind = PlanArg::Output;
          pa.index = o->second;
        } else {
          return nullptr;
        }
      } else {
        pa.value = in;
        if (in.kind == KernelArg::Kind::I32) {
          // A Shrink start: bind it to the start node (interning makes the
          // constant node of a value unique) so replays read the new value.
          for (uint32_t p : k.scalar_nodes)
            if (k.order[p].arg().a == in.i) {
              pa.kind = PlanArg::Start;
              pa.index = p;
            }
        }
      }
      pk.args.push_back(std::move(pa));
    }
    rec->kernels.push_back(std::move(pk));
  }
  std::unordered_map<const UOpInner*, uint32_t> pos;
  for (uint32_t i = 0; i < k.order.size(); i++) pos.emplace(k.order[i].get(), i);
  for (auto& [node, repl] : plan.replacements) {
    auto np = pos.find(node.get());
    if (np == pos.end()) return nullptr;
    PlanReplacement pr;
    pr.node = np->second;
    if (repl.op() == Op::Reshape && repl.src(0).op() == Op::Buffer && repl.src(0).arg().buf &&
        out_of.count(repl.src(0).arg().buf.get())) {
      pr.kernel = static_cast<int32_t>(out_of.at(repl.src(0).arg().buf.get()));
      if (rec->kernels[pr.kernel].out_shape != repl.arg().usizes()) return nullptr;
    } else {
      auto vp = pos.find(repl.get());
      if (vp == pos.end()) return nullptr;
      pr.value = vp->second;
    }
    rec->replacements.push_back(pr);
  }
  for (uint32_t i = 0; i < k.leaves.size(); i++)
    if (zero_before[i] && !k.leaves[i]->known_zero) rec->written_leaves.push_back(i);
  rec->code = k.code;
  return rec;
}

// ── step capture ────────────────────────────────────────────────────────────
// A training loop repeats one step: the same realize_many calls, each a replay
// of the same plan over the same parameter buffers. While a step runs under a
// recorder, every replay is noted; a miss (a realisation that had to be
// scheduled) makes the step unrecordable.
struct ReplayRecord {
  std::shared_ptr<CachedPlan> plan;
  std::vector<Buffer> leaves;          // the key's leaves
  std::vector<int32_t> start_values;   // the Start arguments, in kernel and argument order
  std::vector<Buffer> outs;            // each kernel's output (null where it has none)
};

struct StepRecorder {
  bool valid = true;
  std::vector<ReplayRecord> records;
};

thread_local StepRecorder* g_step_recorder = nullptr;

void replay_plan(Device& backend, const GraphKey& k, const std::shared_ptr<CachedPlan>& planp) {
  const CachedPlan& plan = *planp;
  std::vector<int32_t> starts;
  for (uint32_t i : plan.written_leaves) k.leaves[i]->known_zero = false;
  std::vector<Buffer> outs(plan.kernels.size());
  std::vector<Program*> progs(plan.kernels.size());
  std::vector<std::vector<KernelArg>> seq_args(plan.kernels.size());
  int debug = debug_level();
  uint64_t l0 = now_ns();
  // Every output and lazily zeroed input gets storage first (zero fills are
  // queued on the stream ahead of the launches), then the whole sequence runs.
  for (size_t j = 0; j < plan.kernels.size(); j++) {
    const PlanKernel& pk = plan.kernels[j];
    std::vector<KernelArg>& args = seq_args[j];
    progs[j] = pk.program.get();
    if (pk.has_output) {
      Buffer out = backend.reserve_buffer(pk.out_dtype, pk.out_numel);
      // The same storage as last time when it is free again, so a device that
      // recorded this sequence finds its launch arguments unchanged.
      if (plan.last_storage.size() != plan.kernels.size()) plan.last_storage.assign(plan.kernels.size(), nullptr);
      backend.realize_storage_at(*out, false, plan.last_storage[j]);
      plan.last_storage[j] = out->storage;
      out->known_zero = false;
      outs[j] = out;
      args.push_back(KernelArg::buf(out));
    }
    for (auto& pa : pk.args) {
      if (pa.kind == PlanArg::Value) {
        args.push_back(pa.value);
        continue;
      }
      if (pa.kind == PlanArg::Start) {
        starts.push_back(static_cast<int32_t>(k.order[pa.index].arg().a));
        args.push_back(KernelArg::i32(starts.back()));
        continue;
      }
      const Buffer& b = pa.kind == PlanArg::Leaf ? k.leaves[pa.index] : outs[pa.index];
      if (!b->is_realized()) {
        FG_CHECK(b->zero_init, "scheduled input buffer missing");
        backend.realize_storage(*b, true);
      }
      args.push_back(KernelArg::buf(b));
    }
    realize_stats().lowering_cache_hits++;
    realize_stats().kernels_launched++;
    if (debug >= 1) {
      size_t kid = g_kernel_count++;
      std::fprintf(stderr, "*** %s %4zu  (plan)           arg %2zu\n", backend.id() == DeviceId::Hip ? "HIP" : "CPU",
                   kid, args.size());
    }
  }
  uint64_t l1 = now_ns();
  realize_stats().ns_lower += l1 - l0;
  backend.execute_sequence(progs, seq_args, plan.device_state);
  realize_stats().ns_launch += now_ns() - l1;
  if (g_step_recorder) g_step_recorder->records.push_back({planp, k.leaves, std::move(starts), outs});
  uint64_t t2 = now_ns();
  UOpMap<UOp> repl;
  repl.reserve(plan.replacements.size() * 2);
  for (auto& pr : plan.replacements) {
    const UOp& node = k.order[pr.node];
    if (pr.kernel >= 0) {
      const PlanKernel& pk = plan.kernels[pr.kernel];
      repl[node] = UOp::reshape(UOp::buffer(outs[pr.kernel], pk.out_dtype, node.device()), pk.out_shape);
    } else {
      repl[node] = k.order[pr.value];
    }
  }
  apply_map_to_tensors(repl);
  realize_stats().ns_apply_map += now_ns() - t2;
}

// A step whose realisations can be launched again without rebuilding its
// graphs: every kernel of every replayed plan, in order, with each buffer
// argument resolved to a persistent buffer (parameters, inputs, uploaded
// constants: the same buffer in two consecutive steps) or to an output of an
// earlier kernel of the same step.
struct CapturedStep {
  struct Arg {
    // StepStart: the start of the step's batch (a narrow() of the inputs
    // that moves every step), passed in by each replay.
    enum Kind : uint8_t { Persistent, Output, Value, StepStart } kind = Value;
    Buffer buf;
    uint32_t out = 0;
    KernelArg value;
  };
  struct Kernel {
    Program* prog = nullptr;
    bool has_output = false;
    DType out_dtype;
    size_t out_numel = 0;
    std::vector<Arg> args;
  };
  std::vector<std::shared_ptr<CachedPlan>> plans;  // keep the programs alive
  std::vector<Kernel> kernels;
  std::vector<void*> last_storage;
  std::shared_ptr<void> device_state;  // the device's replay state for the whole step
  uint32_t result_kernel = 0;          // whose output is the step's result (the loss)
};

// The capture of step `cur`, given the step before it, or null when the two
// did not replay the same plans over the same persistent buffers, or when
// `result` is not one of the step's outputs. A Shrink start (a narrow())
// that has the same value in both steps stays a constant; one that equals
// each step's batch start (`start_prev`, `start_cur`, which differ) becomes
// that start on every replay; any other change gives up.
std::unique_ptr<CapturedStep> capture_step(const std::vector<ReplayRecord>& prev,
                                           const std::vector<ReplayRecord>& cur, const Buffer& result,
                                           int64_t start_prev = 0, int64_t start_cur = 0) {
  if (cur.empty() || prev.size() != cur.size()) return nullptr;
  auto cap = std::make_unique<CapturedStep>();
  std::unordered_map<const BufferInner*, uint32_t> out_cur, out_prev;  // output buffer -> kernel of the step
  uint32_t base = 0;
  for (size_t r = 0; r < cur.size(); r++) {
    const ReplayRecord& c = cur[r];
    const ReplayRecord& p = prev[r];
    if (c.plan != p.plan || c.start_values.size() != p.start_values.size()) return nullptr;
    size_t si = 0;
    for (const PlanKernel& pk : c.plan->kernels) {
      CapturedStep::Kernel k;
      k.prog = pk.program.get();
      k.has_output = pk.has_output;
      k.out_dtype = pk.out_dtype;
      k.out_numel = pk.out_numel;
      for (const PlanArg& pa : pk.args) {
        CapturedStep::Arg a;
        if (pa.kind == PlanArg::Value) {
          a.value = pa.value;
        } else if (pa.kind == PlanArg::Start) {
          const int32_t vc = c.start_values.at(si), vp = p.start_values.at(si);
          si++;
          if (vc == vp) {
            a.value = KernelArg::i32(vc);
          } else if (start_cur != start_prev && vc == start_cur && vp == start_prev) {
            a.kind = CapturedStep::Arg::StepStart;
          } else {
            return nullptr;
          }
        } else if (pa.kind == PlanArg::Output) {
          a.kind = CapturedStep::Arg::Output;
          a.out = base + pa.index;
        } else {
          const Buffer& lc = c.leaves[pa.index];
          const Buffer& lp = p.leaves[pa.index];
          auto oc = out_cur.find(lc.get());
          auto op = out_prev.find(lp.get());
          if (oc != out_cur.end() && op != out_prev.end() && oc->second == op->second) {
            a.kind = CapturedStep::Arg::Output;
            a.out = oc->second;
          } else if (oc == out_cur.end() && op == out_prev.end() && lc->is_realized() &&
                     (lc.get() == lp.get() || (lc->known_zero && lp->known_zero && lc->numel == lp->numel &&
                                               lc->dtype == lp->dtype))) {
            // The same buffer in both steps, or, like relu's zeros
            // (tensor.rs:517-531), a fresh buffer that still holds allocate()'s
            // zeros after either step: nothing writes it, so this one serves.
            a.kind = CapturedStep::Arg::Persistent;
            a.buf = lc;
          } else {
            return nullptr;
          }
        }
        k.args.push_back(std::move(a));
      }
      cap->kernels.push_back(std::move(k));
    }
    for (size_t j = 0; j < c.outs.size(); j++) {
      if (c.outs[j]) out_cur[c.outs[j].get()] = base + static_cast<uint32_t>(j);
      if (p.outs[j]) out_prev[p.outs[j].get()] = base + static_cast<uint32_t>(j);
    }
    base += static_cast<uint32_t>(c.plan->kernels.size());
    cap->plans.push_back(c.plan);
  }
  auto res = out_cur.find(result.get());
  if (res == out_cur.end()) return nullptr;
  cap->result_kernel = res->second;
  cap->last_storage.assign(cap->kernels.size(), nullptr);
  return cap;
}

// The device's replay state of the last captured step, kept across native
// loop calls: a call whose capture launches the same programs over the same
// wiring (the same persistent buffers, outputs and values in every argument)
// reuses it instead of grouping, rendering and loading the step's batch
// kernels again on its first replay (0.23 ms per C4 call). The entry holds
// the step's plans, so the program pointers it compares stay valid; buffers
// are compared by address only (equal addresses give the same aliasing, so
// the same launch decisions). Never freed: it may hold programs of a device
// the process tears down at exit.
struct CaptureReuse {
  const Device* dev = nullptr;
  std::vector<std::shared_ptr<CachedPlan>> plans;
  std::vector<uint64_t> shape;
  std::shared_ptr<void> device_state;
};

CaptureReuse& capture_reuse() {
  static CaptureReuse* r = new CaptureReuse();
  return *r;
}

std::vector<uint64_t> capture_shape(const CapturedStep& cap) {
  std::vector<uint64_t> v{cap.kernels.size(), cap.result_kernel};
  auto ptr = [](const void* p) { return static_cast<uint64_t>(reinterpret_cast<uintptr_t>(p)); };
  for (const CapturedStep::Kernel& k : cap.kernels) {
    v.push_back(ptr(k.prog));
    v.push_back(k.has_output);
    v.push_back(k.out_numel);
    v.push_back((static_cast<uint64_t>(k.out_dtype.kind) << 16) | k.out_dtype.vcount);
    v.push_back(k.args.size());
    for (const CapturedStep::Arg& a : k.args) {
      v.push_back(a.kind);
      if (a.kind == CapturedStep::Arg::Persistent) {
        v.push_back(ptr(a.buf.get()));
      } else if (a.kind == CapturedStep::Arg::Output) {
        v.push_back(a.out);
      } else if (a.kind == CapturedStep::Arg::Value) {
        const KernelArg& x = a.value;
        v.push_back(static_cast<uint64_t>(x.kind));
        uint32_t fbits = 0;
        std::memcpy(&fbits, &x.f, sizeof(fbits));
        v.push_back(x.kind == KernelArg::Kind::Buffer ? ptr(x.buffer.get())
                    : x.kind == KernelArg::Kind::F32  ? fbits
                    : x.kind == KernelArg::Kind::Bool ? static_cast<uint64_t>(x.b)
                                                      : static_cast<uint64_t>(static_cast<uint32_t>(x.i)));
      }
    }
  }
  return v;
}

// Launches every kernel of a captured step as one sequence (a single HIP
// graph from its second run on), with the step's result (the loss) read back
// into `slot` (Device::read_async) behind it.
void replay_step(Device& backend, CapturedStep& cap, int slot, int64_t start = 0) {
  const size_t n = cap.kernels.size();
  std::vector<Buffer> outs(n);
  std::vector<Program*> progs(n);
  std::vector<std::vector<KernelArg>> args(n);
  uint64_t l0 = now_ns();
  for (size_t j = 0; j < n; j++) {
    const CapturedStep::Kernel& k = cap.kernels[j];
    progs[j] = k.prog;
    if (k.has_output) {
      Buffer out = backend.reserve_buffer(k.out_dtype, k.out_numel);
      backend.realize_storage_at(*out, false, cap.last_storage[j]);
      cap.last_storage[j] = out->storage;
      out->known_zero = false;
      outs[j] = out;
      args[j].push_back(KernelArg::buf(out));
    }
    for (const CapturedStep::Arg& a : k.args) {
      if (a.kind == CapturedStep::Arg::Value) args[j].push_back(a.value);
      else if (a.kind == CapturedStep::Arg::StepStart) args[j].push_back(KernelArg::i32(static_cast<int32_t>(start)));
      else if (a.kind == CapturedStep::Arg::Persistent) args[j].push_back(KernelArg::buf(a.buf));
      else args[j].push_back(KernelArg::buf(outs[a.out]));
    }
  }
  uint64_t l1 = now_ns();
  realize_stats().ns_lower += l1 - l0;
  backend.execute_sequence_read(progs, args, cap.device_state, outs[cap.result_kernel], slot);
  realize_stats().ns_launch += now_ns() - l1;
  realize_stats().kernels_launched += n;
  realize_stats().lowering_cache_hits += n;
}

// Steps of the native loop queued ahead of the device: FG_STEPS_IN_FLIGHT,
// 1 to 8 (the HIP device's read-back slots), 8 when unset. Read once. C4 on
// one box, three runs each: 14.7-14.8K steps/s with 1, 16.9-17.5K with 2,
// 17.2-17.5K with 4, 17.6-17.8K with 8.
int steps_in_flight() {
  static const int n = [] {
    const char* e = std::getenv("FG_STEPS_IN_FLIGHT");
    if (!e || !*e) return 8;
    char* end = nullptr;
    const long v = std::strtol(e, &end, 10);
    FG_CHECK(*end == '\0' && v >= 1 && v <= 8, std::string("FG_STEPS_IN_FLIGHT must be 1 to 8; got '") + e + "'");
    return static_cast<int>(v);
  }();
  return n;
}

bool step_capture_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("FG_STEP_CAPTURE");
    return !(e && std::strcmp(e, "0") == 0);
  }();
  return on;
}

}  // namespace

void set_plan_cache_enabled(bool on) {
  plan_cache().enabled = on;
  if (!on) clear_plan_cache();
}

void clear_plan_cache() {
  plan_cache().map.clear();
  plan_cache().entries = 0;
}

void plan_cache_stats(uint64_t* hits, uint64_t* misses, uint64_t* entries) {
  *hits = plan_cache().hits;
  *misses = plan_cache().misses;
  *entries = plan_cache().entries;
}

void Tensor::realize_many(const std::vector<Tensor>& tensors) {  // tensor.rs:781-821
  std::vector<UOp> roots;
  UOpSet seen;
  for (auto& t : tensors) {
    if (t.is_realized()) continue;
    UOp r = t.uop();
    if (seen.insert(r).second) roots.push_back(r);
  }
  if (roots.empty()) return;
  if (debug_level() >= 3) std::fprintf(stderr, "━━━ schedule [before] ━━━\n%s", UOp::sink(roots).dump().c_str());
  ScheduleOptions opt;
  opt.fuse = get_device(roots[0].device()).fuse_elementwise();
  uint64_t t0 = now_ns();
  PtrIndexMap held(64);
  std::vector<const UOpInner*> held_list;
  if (opt.fuse) {
    collect_held_nodes(&held, &held_list);
    opt.held = &held;
  }
  PlanCache& pc = plan_cache();
  GraphKey key;
  std::vector<uint8_t> zero_before;
  if (pc.enabled) {
    key = graph_key(roots, opt.fuse, opt.fuse ? &held_list : nullptr);
    if (auto hit = find_plan(key)) {
      pc.hits++;
      realize_stats().ns_schedule += now_ns() - t0;
      replay_plan(get_device(roots[0].device()), key, hit);
      return;
    }
    pc.misses++;
    for (auto& b : key.leaves) zero_before.push_back(b->known_zero ? 1 : 0);
  }
  if (g_step_recorder) g_step_recorder->valid = false;  // a realisation no plan records
  SchedulePlan plan = schedule_many(roots, opt);
  uint64_t t1 = now_ns();
  realize_stats().ns_schedule += t1 - t0;
  std::vector<std::shared_ptr<Program>> programs;
  programs.reserve(plan.items.size());
  for (auto& item : plan.items) programs.push_back(execute_item(item));
  if (pc.enabled) {
    if (auto rec = record_plan(key, plan, programs, zero_before)) {
      if (pc.entries >= kMaxCachedPlans) clear_plan_cache();
      pc.map[key.hash].push_back(std::move(rec));
      pc.entries++;
    }
  }
  uint64_t t2 = now_ns();
  apply_map_to_tensors(plan.replacements);
  realize_stats().ns_apply_map += now_ns() - t2;
}

Tensor Tensor::realize() const {
  realize_many({*this});
  return *this;
}

Buffer Tensor::realized_buffer() const {
  realize();
  UOp u = uop();
  UOp b;
  if (u.op() == Op::Buffer) b = u;
  else if (u.op() == Op::Reshape) b = u.src(0);
  else fail("realized tensor must point at a buffer");
  FG_CHECK(b.arg().kind == Arg::Kind::Buffer, "realized tensor must point at Arg::Buffer");
  return b.arg().buf;
}

std::vector<uint8_t> Tensor::to_bytes() const {
  Buffer b = realized_buffer();
  return get_device(b->device).copy_to_host(b);
}

std::vector<float> Tensor::to_vec() const {  // tensor.rs:912-930
  Buffer b = realized_buffer();
  FG_CHECK(b->dtype == DType::F32(), "to_vec requires F32 tensor data");
  auto bytes = get_device(b->device).copy_to_host(b);
  std::vector<float> out(bytes.size() / 4);
  std::memcpy(out.data(), bytes.data(), bytes.size());
  return out;
}

std::vector<Tensor> Tensor::gradient(const std::vector<Tensor>& targets) const {  // tensor.rs:938-964
  for (auto& t : targets) FG_CHECK(t.device() == device(), "gradient targets must share the same device");
  UOp rg = UOp::full(shape(), DType::F32(), device(), 1.0);
  std::vector<UOp> tu;
  for (auto& t : targets)
    if (t.requires_grad()) tu.push_back(t.uop());
  auto gm = compute_gradient(uop(), rg, tu);
  std::vector<Tensor> out;
  for (auto& t : targets) {
    auto it = gm.find(t.uop());
    if (it != gm.end()) out.push_back(from_uop(it->second, false));
    else out.push_back(from_uop(UOp::full(t.shape(), DType::F32(), t.device(), 0.0), false));
  }
  return out;
}

void Tensor::backward() const {  // tensor.rs:971-998
  struct Timer {
    uint64_t t = now_ns();
    ~Timer() { realize_stats().ns_backward += now_ns() - t; }
  } timer;
  FG_CHECK(numel() == 1, "backward requires a scalar loss");
  const std::vector<UOp> order = uop().toposort();
  PtrIndexMap in_graph(order.size());
  for (size_t i = 0; i < order.size(); i++) in_graph.set(order[i].get(), static_cast<uint32_t>(i));
  std::vector<Tensor> targets;
  for (auto& t : live_tensors())
    if (t.requires_grad() && in_graph.get(t.uop().get()) != PtrIndexMap::kAbsent) targets.push_back(t);
  if (targets.empty()) return;
  std::vector<UOp> tu;
  for (auto& t : targets) tu.push_back(t.uop());
  UOp rg = UOp::full(shape(), DType::F32(), device(), 1.0);
  auto grads = compute_gradient_ordered(order, rg, tu);
  for (auto& t : targets) {
    auto it = grads.find(t.uop());
    UOp g = it != grads.end() ? it->second : UOp::full(t.shape(), DType::F32(), t.device(), 0.0);
    Tensor gt = from_uop(g, false);
    auto existing = t.grad();
    Tensor acc = existing ? existing->add(gt) : gt;
    t.p_->grad = acc.p_;
  }
}

// ── gradient.rs ─────────────────────────────────────────────────────────────
namespace {

UOp const_like(const UOp& n, double v) { return UOp::const_float(v, n.dtype(), n.device()); }

UOp zero_like(const UOp& n) {  // gradient.rs:87-90
  Shape s;
  if (!n.shape_opt(&s)) s = Shape{1};
  return UOp::full(s, n.dtype(), n.device(), 0.0);
}

// gradient.rs:97-205
std::vector<UOp> gradient_for_op(const UOp& node, const UOp& grad) {
  switch (node.op()) {
    case Op::Add: return {grad, grad};
    case Op::Mul: {
      const UOp &x = node.src(0), &y = node.src(1);
      return {UOp::mul(y, grad), UOp::mul(x, grad)};
    }
    case Op::Neg: return {UOp::neg(grad)};
    case Op::Reciprocal: return {UOp::mul(UOp::neg(grad), UOp::mul(node, node))};
    case Op::Exp2: return {UOp::mul(UOp::mul(node, const_like(node, 0.69314718055994530942)), grad)};
    case Op::Log2:
      return {UOp::mul(grad, UOp::reciprocal(UOp::mul(node.src(0), const_like(node, 0.69314718055994530942))))};
    case Op::Sqrt: return {UOp::mul(grad, UOp::reciprocal(UOp::mul(const_like(node, 2.0), node)))};
    case Op::Max: {
      const UOp &x = node.src(0), &y = node.src(1);
      UOp zero = const_like(node, 0.0);
      UOp half = UOp::mul(grad, const_like(node, 0.5));
      UOp xw = UOp::cmplt(y, x), yw = UOp::cmplt(x, y);
      UOp xt = UOp::where(yw, zero, half);
      UOp xg = UOp::where(xw, grad, xt);
      UOp yt = UOp::where(xw, zero, half);
      UOp yg = UOp::where(yw, grad, yt);
      return {xg, yg};
    }
    case Op::CmpLt: return {UOp(), UOp()};
    case Op::Where: {
      const UOp& c = node.src(0);
      UOp zero = const_like(node, 0.0);
      return {UOp(), UOp::where(c, grad, zero), UOp::where(c, zero, grad)};
    }
    case Op::Reshape: return {UOp::reshape(grad, node.src(0).shape())};
    case Op::Permute: return {UOp::permute(grad, invert_permutation(node.arg().usizes()))};
    case Op::Expand: {
      Shape ss = node.src(0).shape();
      auto axes = expand_gradient_axes(ss, node.arg().usizes());
      if (axes.empty()) return {grad};
      return {UOp::reduce_axis(grad, Op::Add, axes)};
    }
    case Op::Contiguous: return {grad};
    case Op::ReduceAxis: {
      const UOp& src = node.src(0);
      Shape ss = src.shape();
      Op rop = node.arg().rop;
      if (rop == Op::Add) return {UOp::expand(grad, ss)};
      if (rop == Op::Max) {
        DType dt = grad.dtype();
        UOp mx = UOp::expand(node, ss);
        UOp ge = UOp::expand(grad, ss);
        UOp not_max = UOp::cmplt(src, mx);
        UOp zero = UOp::const_float(0.0, dt, node.device());
        UOp one = UOp::const_float(1.0, dt, node.device());
        UOp mask = UOp::where(not_max, zero, one);
        UOp count = UOp::reduce_axis(mask, Op::Add, node.arg().usizes());
        UOp ce = UOp::expand(count, ss);
        UOp weighted = UOp::mul(mask, UOp::reciprocal(ce));
        return {UOp::mul(weighted, ge)};
      }
      fail("unsupported reduce op gradient");
    }
    case Op::Buffer: case Op::Const: return {};
    default: fail(std::string("gradient not implemented for ") + op_name(node.op()));
  }
}

}  // namespace

// gradient.rs:20-81 over `order`, the toposort of the root (its last node).
// Nodes are addressed by their position: consumer lists, the `needed` set
// (nodes reachable from a target along consumer edges) and the accumulated
// gradients are flat arrays. Gradients are accumulated in reverse
// topological order with the reference's rules and operand order.
UOpMap<UOp> compute_gradient_ordered(const std::vector<UOp>& order, const UOp& root_grad,
                                     const std::vector<UOp>& targets) {
  const size_t n = order.size();
  FG_CHECK(n > 0, "gradient of an empty graph");
  PtrIndexMap index(n);
  for (size_t i = 0; i < n; i++) index.set(order[i].get(), static_cast<uint32_t>(i));
  std::vector<std::vector<uint32_t>> consumers(n);
  for (size_t i = 0; i < n; i++)
    for (auto& src : order[i].srcs()) consumers[index.get(src.get())].push_back(static_cast<uint32_t>(i));
  std::vector<char> needed(n, 0);
  std::vector<uint32_t> stack;
  for (auto& t : targets) {
    uint32_t ti = index.get(t.get());
    if (ti != PtrIndexMap::kAbsent) stack.push_back(ti);
  }
  while (!stack.empty()) {
    uint32_t v = stack.back();
    stack.pop_back();
    if (needed[v]) continue;
    needed[v] = 1;
    for (uint32_t c : consumers[v]) stack.push_back(c);
  }
  needed[n - 1] = 1;
  std::vector<UOp> grads(n);
  grads[n - 1] = root_grad;
  for (size_t i = n; i-- > 0;) {
    if (!needed[i] || !grads[i]) continue;
    const UOp& node = order[i];
    auto local = gradient_for_op(node, grads[i]);
    for (size_t s = 0; s < node.srcs().size() && s < local.size(); s++) {
      if (!local[s]) continue;
      const uint32_t si = index.get(node.src(s).get());
      if (!needed[si]) continue;
      grads[si] = grads[si] ? UOp::add(grads[si], local[s]) : local[s];
    }
  }
  UOpMap<UOp> result;
  for (auto& t : targets) {
    const uint32_t ti = index.get(t.get());
    result[t] = ti != PtrIndexMap::kAbsent && grads[ti] ? grads[ti] : zero_like(t);
  }
  return result;
}

UOpMap<UOp> compute_gradient(const UOp& root, const UOp& root_grad, const std::vector<UOp>& targets) {
  return compute_gradient_ordered(root.toposort(), root_grad, targets);
}

// ── nn.rs ───────────────────────────────────────────────────────────────────
namespace {
uint64_t g_init_seed = 42;  // nn.rs:12-14

float next_unit_f32() {  // nn.rs:16-26
  g_init_seed = g_init_seed * 6364136223846793005ULL + 1ULL;
  return static_cast<float>(g_init_seed >> 33) / static_cast<float>(1ULL << 31);
}
}  // namespace

void reset_init_seed(uint64_t seed) { g_init_seed = seed; }

Tensor kaiming_normal(const Shape& shape, size_t fan_in, DeviceId dev) {  // nn.rs:28-47
  size_t n = fg::numel(shape);
  float stdv = std::sqrt(2.0f / static_cast<float>(fan_in));
  std::vector<float> data;
  data.reserve(n);
  const float two_pi = 2.0f * 3.14159265358979323846f;
  while (data.size() < n) {
    float u1 = std::max(next_unit_f32(), 1.17549435e-38f);
    float u2 = next_unit_f32();
    float radius = std::sqrt(-2.0f * std::log(u1)) * stdv;
    float theta = two_pi * u2;
    data.push_back(radius * std::cos(theta));
    if (data.size() < n) data.push_back(radius * std::sin(theta));
  }
  return Tensor::new_f32(data, shape, dev);
}

Linear Linear::create(size_t in, size_t out, DeviceId dev, bool with_bias) {  // nn.rs:77-92
  Linear l;
  l.weight = kaiming_normal({out, in}, in, dev).with_requires_grad(true);
  if (with_bias) l.bias = Tensor::zeros({out}, dev, DType::F32()).with_requires_grad(true);
  return l;
}

Tensor Linear::forward(const Tensor& x) const {  // nn.rs:97-104
  Tensor w = weight.permute({1, 0});
  Tensor logits = x.matmul(w);
  if (bias) return logits.add(*bias);
  return logits;
}

std::vector<Tensor> Linear::parameters() const {
  std::vector<Tensor> p{weight};
  if (bias) p.push_back(*bias);
  return p;
}

// ── optim.rs ────────────────────────────────────────────────────────────────
Sgd::Sgd(const std::vector<Tensor>& ps, float lr_) : lr(lr_) {  // optim.rs:23-41
  FG_CHECK(!ps.empty(), "optimizer must have at least one parameter");
  for (auto& p : ps) {
    bool dup = false;
    for (auto& e : params) dup = dup || e.ptr_eq(p);
    if (!dup) params.push_back(p);
  }
}

void Sgd::zero_grad() const {
  for (auto& p : params) p.clear_grad();
}

void Sgd::step() const {  // optim.rs:60-71
  for (auto& p : params) {
    const Tensor* lrp = nullptr;
    for (auto& [d, t] : lr_buffers)
      if (d == p.device()) lrp = &t;
    if (!lrp) {
      lr_buffers.emplace_back(p.device(), Tensor::scalar_f32(lr, p.device()));
      lrp = &lr_buffers.back().second;
    }
    const Tensor& lrt = *lrp;
    auto g = p.grad();
    FG_CHECK(g.has_value(), "optimizer step requires parameter gradients");
    Tensor update = p.detach().sub(g->mul(lrt));
    p.assign(update);
  }
  Tensor::realize_many(params);
}

// examples/mnist.rs:84-101's loop body `steps` times. Every step runs the
// calls of the reference loop in its order (forward, cross_entropy, zero_grad,
// backward, step, the loss read back), so the device runs the same kernels in
// the same order, and the losses, parameters and tensors come out as from
// that loop. Two things differ in how the host drives it:
// - The wait for a step's loss moves: its read-back is queued behind the
//   step, and the host waits for it once the next step is queued, so that
//   host work overlaps the device's.
// - Step capture: once two consecutive steps replayed the same recorded plans
//   over the same parameter and input buffers, the following steps launch
//   that kernel sequence directly, as one device sequence (on the HIP device
//   written as AQL packets into its own queue between the replay-loop
//   brackets), without rebuilding the lazy graphs; only their losses are
//   read. The last
//   step always runs in full, so the parameters, their gradients and every
//   live tensor end as after `steps` ordinary steps.
std::vector<float> train_steps(const std::vector<const Linear*>& layers, const Sgd& opt, const Tensor& x,
                               const Tensor& targets, int steps, int64_t batch, int64_t first_batch) {
  FG_CHECK(!layers.empty(), "train_steps requires at least one layer");
  FG_CHECK(steps >= 0, "train_steps: negative step count");
  int64_t num_batches = 0;
  if (batch > 0) {
    const Shape& xs = x.shape();
    const Shape& ts = targets.shape();
    FG_CHECK(!xs.empty() && !ts.empty() && xs[0] == ts[0],
             "train_steps: images and targets must have the same number of rows");
    FG_CHECK(static_cast<int64_t>(xs[0]) >= batch, "train_steps: batch size larger than the dataset");
    FG_CHECK(first_batch >= 0, "train_steps: negative first batch");
    num_batches = static_cast<int64_t>(xs[0]) / batch;
  }
  // Step i's batch start (mnist.rs:85-87): batches in order, wrapping over
  // the whole ones as the epochs do.
  auto start_of = [&](int i) { return batch > 0 ? ((first_batch + i) % num_batches) * batch : int64_t(0); };
  std::vector<float> losses(static_cast<size_t>(steps));
  Device& dev = get_device(x.device());
  // Step i's loss lands in read-back slot i % in_flight and is waited for
  // in_flight - 1 steps later, so the host queues up to that many steps
  // ahead of the device and a slow host wake-up does not leave it idle.
  const int in_flight = steps_in_flight();
  auto slot = [in_flight](int step) { return step % in_flight; };
  auto collect = [&](int step) {
    std::vector<uint8_t> b = dev.read_wait(slot(step));
    FG_CHECK(b.size() == sizeof(float), "train_steps: the loss must be one f32");
    std::memcpy(&losses[static_cast<size_t>(step)], b.data(), sizeof(float));
  };
  struct RecorderScope {
    explicit RecorderScope(StepRecorder* r) { g_step_recorder = r; }
    ~RecorderScope() { g_step_recorder = nullptr; }
  };
  const bool capture = step_capture_enabled() && plan_cache().enabled;
  std::unique_ptr<CapturedStep> cap;
  std::vector<ReplayRecord> prev;
  bool prev_valid = false;
  // The captured steps run between the device's replay-loop brackets (the
  // HIP device's direct queue); a step built in full runs outside them.
  struct ReplayLoop {
    Device& d;
    bool on = false;
    void begin() {
      if (!on) d.begin_replay_loop();
      on = true;
    }
    void end() {
      if (on) {
        on = false;
        d.end_replay_loop();
      }
    }
    ~ReplayLoop() {
      try {
        end();
      } catch (...) {
      }
    }
  } loop{dev};
  for (int i = 0; i < steps; i++) {
    if (cap && i + 1 < steps) {
      loop.begin();
      replay_step(dev, *cap, slot(i), start_of(i));
      realize_stats().steps_replayed++;
      if (i >= in_flight - 1) collect(i - (in_flight - 1));
      continue;
    }
    loop.end();
    StepRecorder rec;
    {
      RecorderScope scope(capture && !cap ? &rec : nullptr);
      Tensor h = batch > 0 ? x.narrow(0, start_of(i), batch) : x;
      const Tensor t = batch > 0 ? targets.narrow(0, start_of(i), batch) : targets;
      for (size_t l = 0; l < layers.size(); l++) {
        h = layers[l]->forward(h);
        if (l + 1 < layers.size()) h = h.relu();
      }
      Tensor loss = h.cross_entropy(t);
      opt.zero_grad();
      loss.backward();
      opt.step();
      Buffer lb = loss.realized_buffer();
      dev.read_async(lb, slot(i));  // the loss's read-back, queued behind the step
      if (capture && !cap) {
        if (rec.valid && prev_valid && (cap = capture_step(prev, rec.records, lb, start_of(i - 1), start_of(i)))) {
          realize_stats().steps_captured++;
          CaptureReuse& reuse = capture_reuse();
          if (reuse.dev == &dev && reuse.device_state && reuse.shape == capture_shape(*cap))
            cap->device_state = reuse.device_state;
        }
        prev = cap ? std::vector<ReplayRecord>() : std::move(rec.records);
        prev_valid = !cap && rec.valid;
      }
    }
    if (i >= in_flight - 1) collect(i - (in_flight - 1));
  }
  loop.end();
  for (int i = std::max(0, steps - (in_flight - 1)); i < steps; i++) collect(i);
  if (cap && cap->device_state) {
    CaptureReuse& reuse = capture_reuse();
    reuse.dev = &dev;
    reuse.plans = cap->plans;
    reuse.shape = capture_shape(*cap);
    reuse.device_state = cap->device_state;
  }
  return losses;
}

}  // namespace fg
