// IR core: interner, shape inference, toposort, rewrite engine, symbolic folds.
// Follows src/uop.rs, src/rewrite.rs, src/shape.rs and src/optimize/symbolic.rs.
#include "ir.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <sstream>

#include "device.hpp"

namespace fg {

void fail(const std::string& msg) { throw Error(msg); }

std::string DType::str() const {
  const char* n = "f32";
  switch (kind) {
    case DTypeKind::F32: n = "f32"; break;
    case DTypeKind::I32: n = "i32"; break;
    case DTypeKind::Bool: n = "bool"; break;
    case DTypeKind::Void: n = "void"; break;
  }
  if (vcount == 1) return n;
  return std::string(n) + "x" + std::to_string(vcount);
}

// ── shape helpers (src/shape.rs:31-111, schedule/indexing.rs:22-34) ──────────
size_t numel(const Shape& s) {
  size_t n = 1;
  for (auto d : s) n *= d;
  return n;
}

Shape pad_left(const Shape& s, size_t ndim) {
  Shape out(ndim - s.size(), 1);
  out.insert(out.end(), s.begin(), s.end());
  return out;
}

bool broadcast_with(const Shape& a, const Shape& b, Shape* out) {
  size_t nd = std::max(a.size(), b.size());
  Shape l = pad_left(a, nd), r = pad_left(b, nd);
  out->assign(nd, 0);
  for (size_t i = 0; i < nd; i++) {
    if (l[i] == r[i]) (*out)[i] = l[i];
    else if (l[i] == 1) (*out)[i] = r[i];
    else if (r[i] == 1) (*out)[i] = l[i];
    else return false;
  }
  return true;
}

std::vector<size_t> expand_gradient_axes(const Shape& src, const Shape& expanded) {
  std::vector<size_t> axes;
  for (size_t i = 0; i < src.size() && i < expanded.size(); i++)
    if (src[i] == 1 && expanded[i] > 1) axes.push_back(i);
  return axes;
}

std::vector<size_t> invert_permutation(const std::vector<size_t>& order) {
  std::vector<size_t> inv(order.size(), 0);
  for (size_t i = 0; i < order.size(); i++) inv[order[i]] = i;
  return inv;
}

std::vector<size_t> contiguous_strides(const Shape& s) {
  std::vector<size_t> st(s.size(), 1);
  size_t acc = 1;
  for (size_t i = s.size(); i-- > 0;) {
    st[i] = acc;
    acc *= s[i];
  }
  return st;
}

std::string shape_str(const Shape& s) {
  std::ostringstream os;
  os << "[";
  for (size_t i = 0; i < s.size(); i++) os << (i ? ", " : "") << s[i];
  os << "]";
  return os.str();
}

// ── names ────────────────────────────────────────────────────────────────────
const char* op_name(Op op) {
  static const char* names[] = {
      "Device", "DefineVar", "Bind", "Buffer", "Shrink", "Reshape", "Permute", "Expand",
      "Contiguous", "ReduceAxis", "ParamBuffer", "ParamScalar", "Range", "End", "Sink",
      "Index", "Load", "Store", "Vectorize", "Unroll", "Contract", "Const", "Neg", "Exp2",
      "Log2", "Sqrt", "Reciprocal", "Add", "Mul", "Max", "CmpLt", "Where", "Reduce", "After",
      "DefineAcc", "Assign", "Gep"};
  return names[static_cast<int>(op)];
}

bool is_alu(Op op) {
  switch (op) {
    case Op::Add: case Op::Mul: case Op::Max: case Op::CmpLt: case Op::Where:
    case Op::Neg: case Op::Exp2: case Op::Log2: case Op::Sqrt: case Op::Reciprocal:
      return true;
    default:
      return false;
  }
}

bool is_movement(Op op) {
  return op == Op::Shrink || op == Op::Reshape || op == Op::Permute || op == Op::Expand;
}

const char* axis_kind_name(AxisKind k) {
  static const char* names[] = {"LOOP", "GLOBAL", "LOCAL", "REDUCE", "GROUP_REDUCE",
                                "UPCAST", "UNROLL", "THREAD"};
  return names[static_cast<int>(k)];
}

const char* device_name(DeviceId d) { return d == DeviceId::Cpu ? "cpu" : "hip"; }

// ── Arg ──────────────────────────────────────────────────────────────────────
Arg Arg::device(DeviceId d) { Arg x; x.kind = Kind::Device; x.a = static_cast<int64_t>(d); return x; }
Arg Arg::index(int64_t tag) { Arg x; x.kind = Kind::Index; x.a = tag; return x; }
Arg Arg::range(int64_t axis, AxisKind k) {
  Arg x; x.kind = Kind::Range; x.a = axis; x.b = static_cast<int64_t>(k); return x;
}
Arg Arg::param_buffer(int64_t slot, int64_t n) { Arg x; x.kind = Kind::ParamBuffer; x.a = slot; x.b = n; return x; }
Arg Arg::param_scalar(int64_t slot) { Arg x; x.kind = Kind::ParamScalar; x.a = slot; return x; }
Arg Arg::flt(double v) { Arg x; x.kind = Kind::Float; x.f = v; return x; }
Arg Arg::integer(int64_t v) { Arg x; x.kind = Kind::Int; x.a = v; return x; }
Arg Arg::boolean(bool v) { Arg x; x.kind = Kind::Bool; x.a = v ? 1 : 0; return x; }
Arg Arg::buffer(const Buffer& b) { Arg x; x.kind = Kind::Buffer; x.buf = b; return x; }
Arg Arg::bounds(const std::vector<size_t>& l) { Arg x; x.kind = Kind::Bounds; x.v.assign(l.begin(), l.end()); return x; }
Arg Arg::shape(const Shape& s) { Arg x; x.kind = Kind::Shape; x.v.assign(s.begin(), s.end()); return x; }
Arg Arg::axes(const std::vector<size_t>& a) { Arg x; x.kind = Kind::Axes; x.v.assign(a.begin(), a.end()); return x; }
Arg Arg::lanes(const std::vector<std::pair<int64_t, int64_t>>& l) {
  Arg x; x.kind = Kind::Lanes;
  for (auto& p : l) { x.v.push_back(p.first); x.v.push_back(p.second); }
  return x;
}
Arg Arg::reduce(Op op, const std::vector<size_t>& ax) {
  Arg x; x.kind = Kind::Reduce; x.rop = op; x.v.assign(ax.begin(), ax.end()); return x;
}

bool Arg::operator==(const Arg& o) const {
  if (kind != o.kind) return false;
  switch (kind) {
    case Kind::None: return true;
    case Kind::Device: case Kind::Index: case Kind::ParamScalar: case Kind::Int: case Kind::Bool:
      return a == o.a;
    case Kind::Range: case Kind::ParamBuffer: return a == o.a && b == o.b;
    case Kind::Variable: return name == o.name && b == o.b && c == o.c;
    case Kind::Float: {
      uint64_t x, y;
      std::memcpy(&x, &f, 8);
      std::memcpy(&y, &o.f, 8);
      return x == y;
    }
    case Kind::Buffer: return buf.get() == o.buf.get();
    case Kind::Bounds: case Kind::Shape: case Kind::Axes: case Kind::Lanes: return v == o.v;
    case Kind::Reduce: return rop == o.rop && v == o.v;
  }
  return false;
}

static inline size_t hmix(size_t h, size_t v) {
  return h ^ (v + 0x9e3779b97f4a7c15ULL + (h << 6) + (h >> 2));
}

size_t Arg::hash() const {
  size_t h = static_cast<size_t>(kind) * 1315423911u;
  switch (kind) {
    case Kind::None: break;
    case Kind::Device: case Kind::Index: case Kind::ParamScalar: case Kind::Int: case Kind::Bool:
      h = hmix(h, static_cast<size_t>(a)); break;
    case Kind::Range: case Kind::ParamBuffer:
      h = hmix(hmix(h, static_cast<size_t>(a)), static_cast<size_t>(b)); break;
    case Kind::Variable: h = hmix(h, std::hash<std::string>()(name)); break;
    case Kind::Float: {
      uint64_t x;
      std::memcpy(&x, &f, 8);
      h = hmix(h, static_cast<size_t>(x));
      break;
    }
    case Kind::Buffer: h = hmix(h, reinterpret_cast<size_t>(buf.get())); break;
    case Kind::Reduce: h = hmix(h, static_cast<size_t>(rop)); [[fallthrough]];
    case Kind::Bounds: case Kind::Shape: case Kind::Axes: case Kind::Lanes:
      for (auto x : v) h = hmix(h, static_cast<size_t>(x));
      break;
  }
  return h;
}

std::string Arg::str() const {
  std::ostringstream os;
  auto vec = [&](const std::vector<int64_t>& xs) {
    os << "[";
    for (size_t i = 0; i < xs.size(); i++) os << (i ? ", " : "") << xs[i];
    os << "]";
  };
  switch (kind) {
    case Kind::None: break;
    case Kind::Device: os << device_name(static_cast<DeviceId>(a)); break;
    case Kind::Variable: os << name << "[" << b << ", " << c << "]"; break;
    case Kind::Index: os << a; break;
    case Kind::Range: os << a << ":" << axis_kind_name(range_kind()); break;
    case Kind::ParamBuffer: os << "buf_slot=" << a << ",n=" << b; break;
    case Kind::ParamScalar: os << "scalar_slot=" << a; break;
    case Kind::Float: os << f; break;
    case Kind::Int: os << a; break;
    case Kind::Bool: os << (a ? "true" : "false"); break;
    case Kind::Buffer: os << "buf#" << (buf ? buf->id : 0) << "[" << (buf ? buf->numel : 0) << "]"; break;
    case Kind::Bounds: case Kind::Shape: case Kind::Axes: case Kind::Lanes: vec(v); break;
    case Kind::Reduce: os << op_name(rop) << "("; vec(v); os << ")"; break;
  }
  return os.str();
}

// ── interner (src/uop.rs:563-591) ───────────────────────────────────────────
namespace {
// The set of live nodes, keyed by their structural hash: open addressing with
// linear probing and backward-shift deletion, so interning a node costs no
// allocation beyond the node itself. A node enters in UOp::make and leaves in
// the first statement of its destructor, before its sources are released, so
// every entry belongs to a node that is still owned.
class InternTable {
 public:
  InternTable() { slots_.assign(size_t(1) << bits_, nullptr); }
  template <class Eq>
  const UOpInner* find(size_t h, Eq&& eq) const {
    for (size_t i = home(h);; i = next(i)) {
      const UOpInner* e = slots_[i];
      if (!e) return nullptr;
      if (e->hash == h && eq(e)) return e;
    }
  }
  void insert(const UOpInner* e) {
    if ((size_ + 1) * 2 > slots_.size()) grow();
    size_t i = home(e->hash);
    while (slots_[i]) i = next(i);
    slots_[i] = e;
    size_++;
  }
  void erase(const UOpInner* e) {
    size_t i = home(e->hash);
    while (slots_[i] != e) {
      if (!slots_[i]) return;
      i = next(i);
    }
    // Shift back every later entry of the probe run that the hole would
    // otherwise cut off from its home slot.
    for (size_t j = next(i);; j = next(j)) {
      const UOpInner* m = slots_[j];
      if (!m) break;
      const size_t k = home(m->hash);
      const bool stays = i <= j ? (i < k && k <= j) : (i < k || k <= j);
      if (stays) continue;
      slots_[i] = m;
      i = j;
    }
    slots_[i] = nullptr;
    size_--;
  }
  size_t size() const { return size_; }

 private:
  size_t home(size_t h) const { return static_cast<size_t>((h * 0x9E3779B97F4A7C15ULL) >> (64 - bits_)); }
  size_t next(size_t i) const { return (i + 1) & (slots_.size() - 1); }
  void grow() {
    std::vector<const UOpInner*> old;
    old.swap(slots_);
    bits_++;
    slots_.assign(size_t(1) << bits_, nullptr);
    size_ = 0;
    for (const UOpInner* e : old)
      if (e) insert(e);
  }
  std::vector<const UOpInner*> slots_;
  unsigned bits_ = 12;
  size_t size_ = 0;
};

InternTable& interner() {
  static auto* t = new InternTable();
  return *t;
}

size_t node_hash(Op op, DType dt, const std::vector<UOp>& srcs, const Arg& arg, bool has_tag,
                 uint64_t tag) {
  size_t h = static_cast<size_t>(op) * 2654435761u;
  h = hmix(h, static_cast<size_t>(dt.kind) | (static_cast<size_t>(dt.vcount) << 8));
  for (auto& s : srcs) h = hmix(h, s.id());
  h = hmix(h, arg.hash());
  if (has_tag) h = hmix(h, static_cast<size_t>(tag) ^ 0xabcdefULL);
  return h;
}
}  // namespace

UOpInner::~UOpInner() { interner().erase(this); }

size_t interner_size() { return interner().size(); }
void interner_clear_for_tests() {}

UOp UOp::make(Op op, DType dtype, std::vector<UOp> srcs, Arg arg, bool has_tag, uint64_t tag) {
  size_t h = node_hash(op, dtype, srcs, arg, has_tag, tag);
  InternTable& t = interner();
  const UOpInner* e = t.find(h, [&](const UOpInner* c) {
    if (c->op != op || c->dtype != dtype || c->has_tag != has_tag || c->tag != tag) return false;
    if (c->srcs.size() != srcs.size()) return false;
    for (size_t i = 0; i < srcs.size(); i++)
      if (c->srcs[i] != srcs[i]) return false;
    return c->arg == arg;
  });
  if (e) {
    if (auto sp = e->weak_from_this().lock()) return UOp(std::move(sp));
  }
  auto inner = std::make_shared<UOpInner>();
  inner->op = op;
  inner->dtype = dtype;
  inner->srcs = std::move(srcs);
  inner->arg = std::move(arg);
  inner->has_tag = has_tag;
  inner->tag = tag;
  inner->hash = h;
  if (op == Op::Device) inner->device = static_cast<DeviceId>(inner->arg.a);
  else if (!inner->srcs.empty()) inner->device = inner->srcs[0].get()->device;
  t.insert(inner.get());
  return UOp(std::shared_ptr<const UOpInner>(std::move(inner)));
}

UOp UOp::make_new(Op op, DType dtype, std::vector<UOp> srcs, Arg arg) {
  FG_CHECK(!srcs.empty(), "leaf UOps must be created with explicit device");
  DeviceId d = srcs[0].device();
  for (auto& s : srcs) FG_CHECK(s.device() == d, "all UOp sources must belong to the same device");
  return make(op, dtype, std::move(srcs), std::move(arg));
}

UOp UOp::make_tagged(Op op, DType dtype, std::vector<UOp> srcs, Arg arg, uint64_t tag) {
  FG_CHECK(!srcs.empty(), "leaf UOps must be created with explicit device");
  return make(op, dtype, std::move(srcs), std::move(arg), true, tag);
}

UOp UOp::device_uop(DeviceId d) { return make(Op::Device, DType::Void(), {}, Arg::device(d)); }
UOp UOp::param_buffer(int64_t slot, DType dt, int64_t n, DeviceId d) {
  return make(Op::ParamBuffer, dt, {device_uop(d)}, Arg::param_buffer(slot, n));
}
UOp UOp::param_scalar(int64_t slot, DType dt, DeviceId d) {
  return make(Op::ParamScalar, dt, {device_uop(d)}, Arg::param_scalar(slot));
}
UOp UOp::buffer(const Buffer& b, DType dt, DeviceId d) {
  return make(Op::Buffer, dt, {device_uop(d)}, Arg::buffer(b));
}
UOp UOp::const_float(double v, DType dt, DeviceId d) {
  return make(Op::Const, dt, {device_uop(d)}, Arg::flt(v));
}
UOp UOp::const_int(int64_t v, DType dt, DeviceId d) {
  return make(Op::Const, dt, {device_uop(d)}, Arg::integer(v));
}
UOp UOp::const_bool(bool v, DType dt, DeviceId d) {
  return make(Op::Const, dt, {device_uop(d)}, Arg::boolean(v));
}

// uop.rs:740-748
UOp UOp::full(const Shape& shape, DType dt, DeviceId d, double value) {
  Shape base(shape.size(), 1);
  UOp b = reshape(const_float(value, dt, d), base);
  bool all1 = true;
  for (auto x : shape) all1 = all1 && x == 1;
  if (all1) return b;
  return expand(b, shape);
}

UOp UOp::reshape(const UOp& src, const Shape& s) { return make_new(Op::Reshape, src.dtype(), {src}, Arg::shape(s)); }
UOp UOp::shrink(const UOp& src, const std::vector<UOp>& starts, const std::vector<size_t>& lens) {
  std::vector<UOp> srcs{src};
  srcs.insert(srcs.end(), starts.begin(), starts.end());
  return make_new(Op::Shrink, src.dtype(), srcs, Arg::bounds(lens));
}
UOp UOp::permute(const UOp& src, const std::vector<size_t>& ax) { return make_new(Op::Permute, src.dtype(), {src}, Arg::axes(ax)); }
UOp UOp::expand(const UOp& src, const Shape& s) { return make_new(Op::Expand, src.dtype(), {src}, Arg::shape(s)); }
UOp UOp::contiguous(const UOp& src) { return make_new(Op::Contiguous, src.dtype(), {src}, Arg::none()); }
UOp UOp::reduce_axis(const UOp& src, Op rop, const std::vector<size_t>& ax) {
  return make_new(Op::ReduceAxis, src.dtype(), {src}, Arg::reduce(rop, ax));
}
UOp UOp::add(const UOp& a, const UOp& b) { return make_new(Op::Add, a.dtype(), {a, b}, Arg::none()); }
UOp UOp::mul(const UOp& a, const UOp& b) { return make_new(Op::Mul, a.dtype(), {a, b}, Arg::none()); }
UOp UOp::neg(const UOp& a) { return make_new(Op::Neg, a.dtype(), {a}, Arg::none()); }
UOp UOp::reciprocal(const UOp& a) { return make_new(Op::Reciprocal, a.dtype(), {a}, Arg::none()); }
UOp UOp::cmplt(const UOp& a, const UOp& b) { return make_new(Op::CmpLt, DType::Bool(), {a, b}, Arg::none()); }
UOp UOp::where(const UOp& c, const UOp& t, const UOp& f) { return make_new(Op::Where, t.dtype(), {c, t, f}, Arg::none()); }
UOp UOp::store(const UOp& dest, const UOp& value) { return make_new(Op::Store, DType::Void(), {dest, value}, Arg::none()); }
UOp UOp::after(const UOp& value, const UOp& effect) { return make_new(Op::After, value.dtype(), {value, effect}, Arg::none()); }
UOp UOp::sink(std::vector<UOp> stores) { return make(Op::Sink, DType::Void(), std::move(stores), Arg::none()); }

Op UOp::op() const { return p_->op; }
DType UOp::dtype() const { return p_->dtype; }
const std::vector<UOp>& UOp::srcs() const { return p_->srcs; }
const Arg& UOp::arg() const { return p_->arg; }
bool UOp::has_tag() const { return p_->has_tag; }
uint64_t UOp::tag() const { return p_->tag; }

DeviceId UOp::device() const {
  FG_CHECK(p_->op == Op::Device || !p_->srcs.empty(), "non-device UOps must derive device from sources");
  return p_->device;
}

bool UOp::is_const_float(double v) const {
  return op() == Op::Const && arg() == Arg::flt(v);
}
bool UOp::is_const_int(int64_t v) const { return op() == Op::Const && arg() == Arg::integer(v); }

// uop.rs:806-866 (memoised on the node)
bool UOp::shape_opt(Shape* out) const {
  if (p_->shape_state == -1) {
    Shape s;
    bool ok = compute_shape(&s);
    p_->shape_state = ok ? 1 : 0;
    if (ok) p_->shape_cache = std::move(s);
  }
  if (p_->shape_state == 0) return false;
  *out = p_->shape_cache;
  return true;
}

bool UOp::compute_shape(Shape* out) const {
  const Arg& a = arg();
  switch (op()) {
    case Op::Buffer:
      if (a.kind != Arg::Kind::Buffer) return false;
      *out = Shape{a.buf->numel};
      return true;
    case Op::ParamBuffer:
      *out = Shape{static_cast<size_t>(a.b)};
      return true;
    case Op::Shrink:
    case Op::Reshape:
    case Op::Expand:
      *out = a.usizes();
      return true;
    case Op::Permute: {
      Shape s;
      if (!src(0).shape_opt(&s)) return false;
      Shape r;
      for (auto ax : a.v) r.push_back(s[static_cast<size_t>(ax)]);
      *out = r;
      return true;
    }
    case Op::ReduceAxis: {
      Shape s;
      if (!src(0).shape_opt(&s)) return false;
      for (auto ax : a.v) s[static_cast<size_t>(ax)] = 1;
      *out = s;
      return true;
    }
    case Op::Const:
      *out = Shape{1};
      return true;
    case Op::Contiguous:
    case Op::After:
      return src(0).shape_opt(out);
    default:
      if (is_alu(op())) return src(0).shape_opt(out);
      return false;
  }
}

bool UOp::has_shape() const {
  Shape s;
  return shape_opt(&s);
}

Shape UOp::shape() const { return shape_ref(); }

const Shape& UOp::shape_ref() const {
  if (p_->shape_state == -1) {
    Shape s;
    bool ok = compute_shape(&s);
    p_->shape_state = ok ? 1 : 0;
    if (ok) p_->shape_cache = std::move(s);
  }
  FG_CHECK(p_->shape_state == 1, "tensor must have shape");
  return p_->shape_cache;
}

bool UOp::has_buffer_identity() const {
  if (op() == Op::Buffer) return true;
  if (op() == Op::After) return src(0).has_buffer_identity();
  if (is_movement(op())) return src(0).has_buffer_identity();
  return false;
}

UOp UOp::gep(size_t i) const {
  if (op() == Op::Vectorize) return srcs()[i];
  return make_new(Op::Gep, dtype().scalar(), {*this}, Arg::integer(static_cast<int64_t>(i)));
}

// uop.rs:1044-1075 — iterative post-order DFS. Sources are pushed in reverse so
// the first source is visited first, except `After`, whose effect (last source)
// is walked first.
std::vector<UOp> UOp::toposort() const {
  // Stack entries point at the handles held in their parent's `srcs` (or at
  // *this), which stay alive for the whole walk. The visited set is a flat
  // pointer map; result order is the reference's (uop.rs:1044-1075).
  std::vector<UOp> result;
  PtrIndexMap visited(64);
  std::vector<std::pair<const UOp*, bool>> stack;
  stack.emplace_back(this, false);
  while (!stack.empty()) {
    auto [node, processed] = stack.back();
    stack.pop_back();
    const UOpInner* raw = node->get();
    if (visited.get(raw) != PtrIndexMap::kAbsent) continue;
    if (processed) {
      visited.set(raw, 1);
      result.push_back(*node);
      continue;
    }
    stack.emplace_back(node, true);
    const auto& srcs = raw->srcs;
    if (raw->op == Op::After) {
      for (size_t i = 0; i < srcs.size(); i++)
        if (visited.get(srcs[i].get()) == PtrIndexMap::kAbsent) stack.emplace_back(&srcs[i], false);
    } else {
      for (size_t i = srcs.size(); i-- > 0;)
        if (visited.get(srcs[i].get()) == PtrIndexMap::kAbsent) stack.emplace_back(&srcs[i], false);
    }
  }
  return result;
}

std::string UOp::dump() const {
  auto order = toposort();
  UOpMap<size_t> ids;
  for (size_t i = 0; i < order.size(); i++) ids[order[i]] = i;
  std::ostringstream os;
  for (auto& n : order) {
    os << "  %" << ids[n] << " = " << op_name(n.op()) << " " << n.dtype().str();
    if (!n.srcs().empty()) {
      os << " (";
      for (size_t i = 0; i < n.srcs().size(); i++) os << (i ? ", " : "") << "%" << ids[n.srcs()[i]];
      os << ")";
    }
    if (n.arg().kind != Arg::Kind::None) os << "  arg=" << n.arg().str();
    if (n.has_tag()) os << "  tag=" << n.tag();
    os << "\n";
  }
  return os.str();
}

UOpMap<std::vector<UOp>> build_consumer_map(const std::vector<UOp>& order) {
  UOpMap<std::vector<UOp>> consumers;
  for (auto& n : order)
    for (auto& s : n.srcs()) consumers[s].push_back(n);
  return consumers;
}

// ── rewrite engine (src/rewrite.rs:33-115) ──────────────────────────────────
static UOp rebuild(const UOp& node, std::vector<UOp>&& new_srcs) {
  bool changed = false;
  for (size_t i = 0; i < new_srcs.size(); i++)
    if (new_srcs[i] != node.srcs()[i]) { changed = true; break; }
  if (!changed) return node;
  // Rebuilt nodes keep their tag (the reference's rebuild drops it only for
  // untagged nodes, which is the only kind its passes rebuild).
  if (node.has_tag()) return UOp::make(node.op(), node.dtype(), std::move(new_srcs), node.arg(), true, node.tag());
  if (node.op() == Op::Sink) return UOp::make(Op::Sink, node.dtype(), std::move(new_srcs), node.arg());
  return UOp::make_new(node.op(), node.dtype(), std::move(new_srcs), node.arg());
}

UOp graph_rewrite(const UOp& root, const RewriteFn& fn) {
  UOp current = root;
  for (;;) {
    auto order = current.toposort();
    UOpMap<UOp> replace;
    replace.reserve(order.size() * 2);
    bool changed = false;
    for (auto& node : order) {
      std::vector<UOp> ns;
      ns.reserve(node.srcs().size());
      for (auto& s : node.srcs()) {
        auto it = replace.find(s);
        ns.push_back(it == replace.end() ? s : it->second);
      }
      UOp rebuilt = rebuild(node, std::move(ns));
      UOp r = fn(rebuilt);
      if (r && r != rebuilt) {
        replace[node] = r;
        changed = true;
        continue;
      }
      replace[node] = rebuilt;
    }
    auto it = replace.find(current);
    if (it != replace.end()) current = it->second;
    if (!changed) return current;
  }
}

UOp substitute_with_map(const UOp& root, const UOpMap<UOp>& replacements) {
  auto order = root.toposort();
  UOpMap<UOp> sub;
  sub.reserve(order.size() * 2);
  for (auto& node : order) {
    auto r = replacements.find(node);
    if (r != replacements.end()) {
      sub[node] = r->second;
      continue;
    }
    std::vector<UOp> ns;
    ns.reserve(node.srcs().size());
    for (auto& s : node.srcs()) {
      auto it = sub.find(s);
      ns.push_back(it == sub.end() ? s : it->second);
    }
    sub[node] = rebuild(node, std::move(ns));
  }
  auto it = sub.find(root);
  return it == sub.end() ? root : it->second;
}

std::vector<UOp> substitute_many(const std::vector<UOp>& roots, const UOpMap<UOp>& replacements) {
  // Memo: node -> index into `done` (its substituted value). The walk stops at
  // replaced nodes, so the graph beneath them is never visited.
  // Sized for the common case (realised leaves and short lazy graphs); both
  // grow on demand.
  PtrIndexMap memo(64);
  std::vector<UOp> done;
  done.reserve(64);
  std::vector<std::pair<const UOp*, bool>> stack;
  std::vector<UOp> out;
  out.reserve(roots.size());
  for (const UOp& root : roots) {
    stack.emplace_back(&root, false);
    while (!stack.empty()) {
      auto [np, expanded] = stack.back();
      stack.pop_back();
      const UOp& node = *np;
      if (memo.get(node.get()) != PtrIndexMap::kAbsent) continue;
      auto r = replacements.find(node);
      if (r != replacements.end()) {
        memo.set(node.get(), static_cast<uint32_t>(done.size()));
        done.push_back(r->second);
        continue;
      }
      const auto& srcs = node.srcs();
      if (!expanded) {
        stack.emplace_back(np, true);
        for (size_t i = srcs.size(); i-- > 0;)
          if (memo.get(srcs[i].get()) == PtrIndexMap::kAbsent) stack.emplace_back(&srcs[i], false);
        continue;
      }
      std::vector<UOp> ns;
      ns.reserve(srcs.size());
      for (auto& s : srcs) ns.push_back(done[memo.get(s.get())]);
      UOp v = rebuild(node, std::move(ns));
      memo.set(node.get(), static_cast<uint32_t>(done.size()));
      done.push_back(std::move(v));
    }
    out.push_back(done[memo.get(root.get())]);
  }
  return out;
}

UOp flatten_end_bodies(const UOp& node) {
  if (node.op() != Op::End || node.srcs().size() < 2) return UOp();
  bool changed = false;
  std::vector<UOp> srcs{node.src(0)};
  for (size_t i = 1; i < node.srcs().size(); i++) {
    const UOp& b = node.src(i);
    if (b.op() == Op::Sink) {
      changed = true;
      srcs.insert(srcs.end(), b.srcs().begin(), b.srcs().end());
    } else {
      srcs.push_back(b);
    }
  }
  if (!changed) return UOp();
  return UOp::make_new(Op::End, DType::Void(), srcs, Arg::none());
}

UOp flatten_nested_sinks(const UOp& node) {
  if (node.op() != Op::Sink) return UOp();
  bool changed = false;
  std::vector<UOp> srcs;
  for (auto& s : node.srcs()) {
    if (s.op() == Op::Sink) {
      changed = true;
      srcs.insert(srcs.end(), s.srcs().begin(), s.srcs().end());
    } else {
      srcs.push_back(s);
    }
  }
  if (!changed) return UOp();
  return UOp::sink(srcs);
}

// ── symbolic_simple (src/optimize/symbolic.rs:19-57) ────────────────────────
static UOp const_from_arg(const UOp& like, const Arg& a) {
  if (a.kind == Arg::Kind::Float) return UOp::const_float(a.f, like.dtype(), like.device());
  if (a.kind == Arg::Kind::Int) return UOp::const_int(a.a, like.dtype(), like.device());
  if (a.kind == Arg::Kind::Bool) return UOp::const_bool(a.a != 0, like.dtype(), like.device());
  fail("constant folding produced non-literal arg");
}

UOp symbolic_simple(const UOp& node) {
  Op op = node.op();
  if ((op != Op::Add && op != Op::Mul) || node.srcs().size() != 2) return UOp();
  const UOp& x = node.src(0);
  const UOp& y = node.src(1);
  // Tagged literals stand in for loaded buffer contents and are never folded.
  if (x.has_tag() || y.has_tag()) return UOp();
  if (x.is_const() && y.is_const()) {
    const Arg &a = x.arg(), &b = y.arg();
    if (a.kind == Arg::Kind::Float && b.kind == Arg::Kind::Float)
      return const_from_arg(x, Arg::flt(op == Op::Add ? a.f + b.f : a.f * b.f));
    if (a.kind == Arg::Kind::Int && b.kind == Arg::Kind::Int)
      return const_from_arg(x, Arg::integer(op == Op::Add ? a.a + b.a : a.a * b.a));
    // The const-const arm matched but has no fold: no rewrite (symbolic.rs:46-51).
    return UOp();
  }
  if (op == Op::Add) {
    if (y.is_zero()) return x;
    if (x.is_zero()) return y;
    return UOp();
  }
  if (y.is_one()) return x;
  if (x.is_one()) return y;
  if (y.is_zero()) return y;
  if (x.is_zero()) return x;
  return UOp();
}

}  // namespace fg
