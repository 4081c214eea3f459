// Core IR of the MI355X execution path: dtypes, shapes, the UOp graph node and
// its interner, plus the graph-rewrite engine.
//
// Restates the reference IR (src/dtype.rs, src/shape.rs, src/uop.rs,
// src/rewrite.rs) so lazy graphs built here schedule into the same kernels as
// the reference: identical op catalogue, interning (structural identity ==
// pointer identity) and toposort order (uop.rs:1044-1075), which fixes kernel
// parameter slot numbering (schedule.rs:185-244).
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace fg {

struct Error : std::runtime_error {
  explicit Error(const std::string& m) : std::runtime_error(m) {}
};

[[noreturn]] void fail(const std::string& msg);
#define FG_CHECK(cond, msg)                         \
  do {                                              \
    if (!(cond)) ::fg::fail(msg);                   \
  } while (0)

// ── dtype (src/dtype.rs:17-110) ──────────────────────────────────────────────
enum class DTypeKind : uint8_t { F32 = 0, I32 = 1, Bool = 2, Void = 3 };

struct DType {
  DTypeKind kind = DTypeKind::F32;
  uint16_t vcount = 1;
  constexpr DType() = default;
  constexpr DType(DTypeKind k, uint16_t v = 1) : kind(k), vcount(v) {}
  static constexpr DType F32() { return DType(DTypeKind::F32); }
  static constexpr DType I32() { return DType(DTypeKind::I32); }
  static constexpr DType Bool() { return DType(DTypeKind::Bool); }
  static constexpr DType Void() { return DType(DTypeKind::Void); }
  constexpr DType vec(uint16_t n) const { return DType(kind, n); }
  constexpr DType scalar() const { return DType(kind, 1); }
  constexpr bool is_scalar() const { return vcount == 1; }
  size_t size_bytes() const {
    switch (kind) {
      case DTypeKind::F32:
      case DTypeKind::I32: return 4;
      case DTypeKind::Bool: return 1;
      default: return 0;
    }
  }
  const char* c_type() const {
    switch (kind) {
      case DTypeKind::F32: return "float";
      case DTypeKind::I32: return "int";
      case DTypeKind::Bool: return "_Bool";
      default: return "void";
    }
  }
  std::string str() const;
  bool operator==(const DType& o) const { return kind == o.kind && vcount == o.vcount; }
  bool operator!=(const DType& o) const { return !(*this == o); }
};

// ── shape (src/shape.rs:31-111) ──────────────────────────────────────────────
using Shape = std::vector<size_t>;
size_t numel(const Shape& s);
Shape pad_left(const Shape& s, size_t ndim);
bool broadcast_with(const Shape& a, const Shape& b, Shape* out);
std::vector<size_t> expand_gradient_axes(const Shape& src, const Shape& expanded);
std::vector<size_t> invert_permutation(const std::vector<size_t>& order);
std::vector<size_t> contiguous_strides(const Shape& s);
std::string shape_str(const Shape& s);

// ── ops (src/uop.rs:26-339) ─────────────────────────────────────────────────
enum class Op : uint8_t {
  Device, DefineVar, Bind, Buffer, Shrink, Reshape, Permute, Expand, Contiguous,
  ReduceAxis, ParamBuffer, ParamScalar, Range, End, Sink, Index, Load, Store,
  Vectorize, Unroll, Contract, Const, Neg, Exp2, Log2, Sqrt, Reciprocal, Add, Mul,
  Max, CmpLt, Where, Reduce, After, DefineAcc, Assign, Gep
};
const char* op_name(Op op);
bool is_alu(Op op);
bool is_movement(Op op);

enum class AxisKind : uint8_t { Loop, Global, Local, Reduce, GroupReduce, Upcast, Unroll, Thread };
const char* axis_kind_name(AxisKind k);

enum class DeviceId : uint8_t { Cpu = 0, Hip = 1 };
const char* device_name(DeviceId d);

struct BufferInner;
using Buffer = std::shared_ptr<BufferInner>;

// ── Arg (src/uop.rs:390-497) ────────────────────────────────────────────────
struct Arg {
  enum class Kind : uint8_t {
    None, Device, Variable, Index, Range, ParamBuffer, ParamScalar, Float, Int, Bool,
    Buffer, Bounds, Shape, Axes, Lanes, Reduce
  };
  Kind kind = Kind::None;
  int64_t a = 0;                 // Device id, Index tag, Range axis, slot, Int, Bool
  int64_t b = 0;                 // Range kind, ParamBuffer numel, Variable min
  int64_t c = 0;                 // Variable max
  double f = 0.0;                // Float
  Op rop = Op::Add;              // Reduce op
  std::vector<int64_t> v;        // Bounds/Shape/Axes/Lanes(flattened pairs)/Reduce axes
  Buffer buf;                    // Buffer
  std::string name;              // Variable

  static Arg none() { return Arg(); }
  static Arg device(DeviceId d);
  static Arg index(int64_t tag);
  static Arg range(int64_t axis, AxisKind k);
  static Arg param_buffer(int64_t slot, int64_t numel);
  static Arg param_scalar(int64_t slot);
  static Arg flt(double x);
  static Arg integer(int64_t x);
  static Arg boolean(bool x);
  static Arg buffer(const Buffer& b);
  static Arg bounds(const std::vector<size_t>& lens);
  static Arg shape(const Shape& s);
  static Arg axes(const std::vector<size_t>& ax);
  static Arg lanes(const std::vector<std::pair<int64_t, int64_t>>& l);
  static Arg reduce(Op op, const std::vector<size_t>& ax);

  AxisKind range_kind() const { return static_cast<AxisKind>(b); }
  std::vector<size_t> usizes() const { return std::vector<size_t>(v.begin(), v.end()); }
  bool operator==(const Arg& o) const;
  bool operator!=(const Arg& o) const { return !(*this == o); }
  size_t hash() const;
  std::string str() const;
};

// ── UOp (src/uop.rs:527-1075) ───────────────────────────────────────────────
struct UOpInner;
class UOp {
 public:
  UOp() = default;
  explicit UOp(std::shared_ptr<const UOpInner> p) : p_(std::move(p)) {}

  // Interning constructors.
  static UOp make(Op op, DType dtype, std::vector<UOp> srcs, Arg arg, bool has_tag = false,
                  uint64_t tag = 0);
  static UOp make_new(Op op, DType dtype, std::vector<UOp> srcs, Arg arg);  // checks device
  static UOp make_tagged(Op op, DType dtype, std::vector<UOp> srcs, Arg arg, uint64_t tag);

  static UOp device_uop(DeviceId d);
  static UOp param_buffer(int64_t slot, DType dtype, int64_t numel, DeviceId d);
  static UOp param_scalar(int64_t slot, DType dtype, DeviceId d);
  static UOp buffer(const Buffer& b, DType dtype, DeviceId d);
  static UOp const_float(double v, DType dtype, DeviceId d);
  static UOp const_int(int64_t v, DType dtype, DeviceId d);
  static UOp const_bool(bool v, DType dtype, DeviceId d);
  static UOp full(const Shape& shape, DType dtype, DeviceId d, double value);

  static UOp reshape(const UOp& src, const Shape& shape);
  static UOp shrink(const UOp& src, const std::vector<UOp>& starts, const std::vector<size_t>& lens);
  static UOp permute(const UOp& src, const std::vector<size_t>& axes);
  static UOp expand(const UOp& src, const Shape& shape);
  static UOp contiguous(const UOp& src);
  static UOp reduce_axis(const UOp& src, Op rop, const std::vector<size_t>& axes);
  static UOp add(const UOp& a, const UOp& b);
  static UOp mul(const UOp& a, const UOp& b);
  static UOp neg(const UOp& a);
  static UOp reciprocal(const UOp& a);
  static UOp cmplt(const UOp& a, const UOp& b);
  static UOp where(const UOp& c, const UOp& t, const UOp& f);
  static UOp store(const UOp& dest, const UOp& value);
  static UOp after(const UOp& value, const UOp& effect);
  static UOp sink(std::vector<UOp> stores);

  Op op() const;
  DType dtype() const;
  const std::vector<UOp>& srcs() const;
  const UOp& src(size_t i) const { return srcs()[i]; }
  const Arg& arg() const;
  bool has_tag() const;
  uint64_t tag() const;
  DeviceId device() const;
  bool has_shape() const;
  Shape shape() const;  // fails if none
  const Shape& shape_ref() const;  // the cached shape, by reference; fails if none
  bool shape_opt(Shape* out) const;
  bool has_buffer_identity() const;
  bool is_const() const { return op() == Op::Const; }
  bool is_const_float(double v) const;
  bool is_const_int(int64_t v) const;
  bool is_zero() const { return is_const_float(0.0) || is_const_int(0); }
  bool is_one() const { return is_const_float(1.0) || is_const_int(1); }
  UOp gep(size_t i) const;

  std::vector<UOp> toposort() const;
  std::string dump() const;

  explicit operator bool() const { return static_cast<bool>(p_); }
  bool operator==(const UOp& o) const { return p_ == o.p_; }
  bool operator!=(const UOp& o) const { return p_ != o.p_; }
  bool operator<(const UOp& o) const { return p_ < o.p_; }
  size_t id() const { return reinterpret_cast<size_t>(p_.get()); }
  const UOpInner* get() const { return p_.get(); }

 private:
  bool compute_shape(Shape* out) const;
  std::shared_ptr<const UOpInner> p_;
};

struct UOpHash {
  size_t operator()(const UOp& u) const { return std::hash<size_t>()(u.id()); }
};
template <class V>
using UOpMap = std::unordered_map<UOp, V, UOpHash>;
using UOpSet = std::unordered_set<UOp, UOpHash>;

struct UOpInner : std::enable_shared_from_this<UOpInner> {
  Op op;
  DType dtype;
  std::vector<UOp> srcs;
  Arg arg;
  bool has_tag = false;
  uint64_t tag = 0;
  size_t hash = 0;
  DeviceId device = DeviceId::Hip;  // derived from the first source at creation
  // Lazily computed tensor shape (shape() is a pure function of the node).
  mutable int8_t shape_state = -1;  // -1 unknown, 0 none, 1 cached
  mutable Shape shape_cache;
  ~UOpInner();
};

// Open-addressing map from node (or buffer) address to a 32-bit value, for the
// per-realize graph walks where std::unordered_map's node allocations dominate.
class PtrIndexMap {
 public:
  static constexpr uint32_t kAbsent = 0xffffffffu;
  explicit PtrIndexMap(size_t expected = 256) { rehash(expected * 2); }
  uint32_t get(const void* k) const {
    for (size_t i = slot(k);; i = (i + 1) & mask_) {
      if (keys_[i] == k) return vals_[i];
      if (!keys_[i]) return kAbsent;
    }
  }
  // Inserts k -> v unless k is present; returns the stored value.
  uint32_t put(const void* k, uint32_t v) {
    if ((size_ + 1) * 2 > keys_.size()) rehash(keys_.size() * 2);
    for (size_t i = slot(k);; i = (i + 1) & mask_) {
      if (keys_[i] == k) return vals_[i];
      if (!keys_[i]) {
        keys_[i] = k;
        vals_[i] = v;
        size_++;
        return v;
      }
    }
  }
  void set(const void* k, uint32_t v) {
    if ((size_ + 1) * 2 > keys_.size()) rehash(keys_.size() * 2);
    for (size_t i = slot(k);; i = (i + 1) & mask_) {
      if (keys_[i] == k || !keys_[i]) {
        if (!keys_[i]) size_++;
        keys_[i] = k;
        vals_[i] = v;
        return;
      }
    }
  }
  size_t size() const { return size_; }

 private:
  size_t slot(const void* k) const {
    return static_cast<size_t>((reinterpret_cast<uintptr_t>(k) >> 4) * 0x9E3779B97F4A7C15ULL >> 20) & mask_;
  }
  void rehash(size_t cap) {
    size_t n = 16;
    while (n < cap) n <<= 1;
    std::vector<const void*> ok(n, nullptr);
    std::vector<uint32_t> ov(n, 0);
    ok.swap(keys_);
    ov.swap(vals_);
    mask_ = n - 1;
    size_ = 0;
    for (size_t i = 0; i < ok.size(); i++)
      if (ok[i]) set(ok[i], ov[i]);
  }
  std::vector<const void*> keys_;
  std::vector<uint32_t> vals_;
  size_t mask_ = 0, size_ = 0;
};

size_t interner_size();
void interner_clear_for_tests();

UOpMap<std::vector<UOp>> build_consumer_map(const std::vector<UOp>& order);

// ── rewrite engine (src/rewrite.rs:33-163) ──────────────────────────────────
using RewriteFn = std::function<UOp(const UOp&)>;  // returns null UOp for "no match"
UOp graph_rewrite(const UOp& root, const RewriteFn& fn);
UOp substitute_with_map(const UOp& root, const UOpMap<UOp>& replacements);
// substitute_with_map over several roots with one shared memo; the walk does
// not descend below replaced nodes (their subgraphs cannot survive).
std::vector<UOp> substitute_many(const std::vector<UOp>& roots, const UOpMap<UOp>& replacements);
UOp flatten_end_bodies(const UOp& node);
UOp flatten_nested_sinks(const UOp& node);

// symbolic_simple (src/optimize/symbolic.rs:42-57)
UOp symbolic_simple(const UOp& node);

}  // namespace fg
