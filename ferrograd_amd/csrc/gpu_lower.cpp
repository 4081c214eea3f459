// gfx950 lowering and HIP codegen for rangeified kernels.
//
// The reference lowers every kernel to nested scalar C loops (upcast/unroll in
// src/optimize/, expand.rs, devectorize.rs, linearize.rs, codegen/clang.rs).
// Here a kernel is classified and rendered as one of:
//   Gemm          Reduce(Add, Mul(Load A, Load B)) over one range with affine
//                 operand indexes (the pattern nn::Linear and its gradients
//                 produce): fp32 MFMA 32x32x2 tiles, LDS double buffering,
//                 XCD-aware tile order, the rest of the kernel as epilogue.
//   Elementwise   no reduction: one thread per 4 consecutive outputs,
//                 16-byte loads/stores where the index is unit-stride.
//   RowReduce     threads of a group split the innermost reduce range
//                 (unit-stride loads), then a wave64 DPP/ds_swizzle tree and
//                 an LDS step across waves.
//   ColumnReduce  threads own outputs along the unit-stride output range and
//                 split the reduce range; partials combine through LDS.
//   Serial        one thread per output, reductions as serial loops in the
//                 reference's exact order (REDUCE x UNROLL(4) left fold,
//                 devectorize.rs:206-214, 274-347) — bit-identical to the CPU.
#include "gpu_lower.hpp"

#include "../../include/ferrograd_hip.h"

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <set>
#include <set>
#include <sstream>

namespace fg {

// ── affine index analysis ───────────────────────────────────────────────────
int64_t Affine::coef(const UOp& t) const {
  for (auto& p : terms)
    if (p.first == t) return p.second;
  return 0;
}

bool Affine::has_scalar_terms() const {
  for (auto& p : terms)
    if (p.first.op() == Op::ParamScalar && p.second != 0) return true;
  return false;
}

static void affine_rec(const UOp& e, int64_t mul, Affine& out) {
  if (!out.ok) return;
  switch (e.op()) {
    case Op::Const:
      if (e.arg().kind == Arg::Kind::Int) out.c0 += mul * e.arg().a;
      else out.ok = false;
      return;
    case Op::Range:
    case Op::ParamScalar: {
      for (auto& p : out.terms)
        if (p.first == e) {
          p.second += mul;
          return;
        }
      out.terms.emplace_back(e, mul);
      return;
    }
    case Op::Add:
      affine_rec(e.src(0), mul, out);
      affine_rec(e.src(1), mul, out);
      return;
    case Op::Mul:
      if (e.src(1).op() == Op::Const && e.src(1).arg().kind == Arg::Kind::Int) {
        affine_rec(e.src(0), mul * e.src(1).arg().a, out);
      } else if (e.src(0).op() == Op::Const && e.src(0).arg().kind == Arg::Kind::Int) {
        affine_rec(e.src(1), mul * e.src(0).arg().a, out);
      } else {
        out.ok = false;
      }
      return;
    default:
      out.ok = false;
  }
}

Affine affine_of(const UOp& e) {
  Affine a;
  affine_rec(e, 1, a);
  return a;
}

int64_t range_extent(const UOp& r) {
  FG_CHECK(r.op() == Op::Range && !r.srcs().empty() && r.src(0).arg().kind == Arg::Kind::Int,
           "range bound must be a constant");
  return r.src(0).arg().a;
}

const char* kernel_class_name(KernelClass k) {
  switch (k) {
    case KernelClass::Gemm: return "gemm_mfma_f32";
    case KernelClass::Elementwise: return "elementwise";
    case KernelClass::RowReduce: return "row_reduce";
    case KernelClass::ColumnReduce: return "column_reduce";
    case KernelClass::Serial: return "serial";
    case KernelClass::NarrowGemm: return "gemm_narrow_f32";
    case KernelClass::Block: return "block";
    case KernelClass::Sequential: return "sequential";
  }
  return "?";
}

KernelInfo analyze_kernel(const UOp& sink) {
  FG_CHECK(sink.op() == Op::Sink && !sink.srcs().empty(), "kernel must be Sink(one effect)");
  for (size_t i = 1; i < sink.srcs().size(); i++)
    FG_CHECK(sink.src(i).op() == Op::ParamBuffer || sink.src(i).op() == Op::ParamScalar,
             "kernel must be Sink(one effect, kernel parameters)");
  KernelInfo ki;
  UOp n = sink.src(0);
  while (n.op() == Op::End) {
    FG_CHECK(n.srcs().size() == 2, "output loop End must carry exactly one body");
    ki.out_ranges.push_back(n.src(0));
    ki.out_ext.push_back(range_extent(n.src(0)));
    n = n.src(1);
  }
  FG_CHECK(n.op() == Op::Store, "kernel body must be a Store");
  ki.store = n;
  const UOp& idx = n.src(0);
  FG_CHECK(idx.op() == Op::Index && idx.srcs().size() == 2, "store target must be Index(param, flat)");
  ki.out_param = idx.src(0);
  FG_CHECK(ki.out_param.op() == Op::ParamBuffer, "store target must be a kernel buffer parameter");
  ki.out_index = idx.src(1);
  ki.value = n.src(1);
  for (auto& x : ki.value.toposort())
    if (x.op() == Op::Reduce) ki.reduces.push_back(x);
  std::map<int, UOp> ps;
  for (auto& x : sink.toposort())
    if (x.op() == Op::ParamBuffer || x.op() == Op::ParamScalar) ps[static_cast<int>(x.arg().a)] = x;
  for (auto& p : ps) ki.params.emplace_back(p.first, p.second);
  return ki;
}

UOp with_all_params(const UOp& kernel, const UOp& scheduled) {
  std::map<int64_t, UOp> want;
  for (auto& x : scheduled.toposort())
    if (x.op() == Op::ParamBuffer || x.op() == Op::ParamScalar) want.emplace(x.arg().a, x);
  for (auto& x : kernel.toposort())
    if (x.op() == Op::ParamBuffer || x.op() == Op::ParamScalar) want.erase(x.arg().a);
  if (want.empty()) return kernel;
  std::vector<UOp> srcs = kernel.srcs();
  for (auto& [slot, p] : want) srcs.push_back(p);
  return UOp::make_new(Op::Sink, kernel.dtype(), srcs, kernel.arg());
}

// ── OPT: pass selection (src/optimize/mod.rs:85-112) ───────────────────────
GpuPasses parse_gpu_passes(const char* raw) {
  GpuPasses all;
  if (!raw) return all;
  auto trim = [](const std::string& x) {
    size_t a = x.find_first_not_of(" \t\n"), b = x.find_last_not_of(" \t\n");
    return a == std::string::npos ? std::string() : x.substr(a, b - a + 1);
  };
  const std::string s = trim(raw);
  if (s.empty() || s == "1" || s == "on" || s == "all") return all;
  GpuPasses some{false, false, false, false, false, false};
  if (s == "0" || s == "off" || s == "none") return some;
  size_t p = 0;
  while (p <= s.size()) {
    size_t q = s.find(',', p);
    const std::string name = trim(s.substr(p, q == std::string::npos ? std::string::npos : q - p));
    if (name == "symbolic") some.symbolic = true;
    else if (name == "mfma") some.mfma = true;
    else if (name == "narrow") some.narrow = true;
    else if (name == "fuse") some.fuse = true;
    else if (name == "block") some.block = true;
    else if (name == "batch") some.batch = true;
    if (q == std::string::npos) break;
    p = q + 1;
  }
  return some;
}

const GpuPasses& gpu_passes() {
  static const GpuPasses on = parse_gpu_passes(std::getenv("OPT"));
  return on;
}

// ── optimize: symbolic + size-1 reduce ranges ───────────────────────────────
namespace {

// A reduction inlined in another's value can range over the very Range node
// the enclosing reduction binds: rangeify gives a reduced axis one range per
// kernel, and a log_softmax row sum summed again over the same axis reuses it.
// The inner loop shadows the outer one, as two nested C loops of one index
// name do in the CPU backend's kernel: inside the inner reduction the range
// is the inner loop's index, outside it the outer's. Give every such inner
// reduction fresh ranges of the same extents so that each loop has its own.
UOp rename_shadowed_ranges(UOp k) {
  int64_t next = 0;
  for (auto& n : k.toposort())
    if (n.op() == Op::Range) next = std::max(next, n.arg().a + 1);
  for (;;) {
    UOp inner;
    for (auto& n : k.toposort()) {
      if (n.op() != Op::Reduce || n.srcs().size() < 2) continue;
      UOpSet outer(n.srcs().begin() + 1, n.srcs().end());
      for (auto& m : n.src(0).toposort()) {
        if (m.op() != Op::Reduce) continue;
        for (size_t i = 1; i < m.srcs().size() && !inner; i++)
          if (outer.count(m.src(i))) inner = m;
        if (inner) break;
      }
      if (inner) break;
    }
    if (!inner) return k;
    UOpMap<UOp> fresh;
    std::vector<UOp> srcs{UOp()};
    for (size_t i = 1; i < inner.srcs().size(); i++) {
      const UOp& r = inner.src(i);
      UOp nr = UOp::make_new(Op::Range, r.dtype(), r.srcs(), Arg::range(next++, r.arg().range_kind()));
      fresh[r] = nr;
      srcs.push_back(nr);
    }
    srcs[0] = substitute_with_map(inner.src(0), fresh);
    k = substitute_with_map(k, {{inner, UOp::make_new(Op::Reduce, inner.dtype(), srcs, inner.arg())}});
  }
}

}  // namespace

UOp gpu_optimize(const UOp& rangeified) {
  const bool symbolic = gpu_passes().symbolic;
  UOp k = symbolic ? graph_rewrite(rangeified, symbolic_simple) : rangeified;
  k = rename_shadowed_ranges(k);
  // A reduce range of extent 1 iterates once at index 0: substitute 0 and
  // drop it from the Reduce (the accumulation itself is kept).
  auto drop_unit = [](const UOp& n) -> UOp {
    if (n.op() != Op::Reduce) return UOp();
    std::vector<UOp> keep;
    UOpMap<UOp> sub;
    for (size_t i = 1; i < n.srcs().size(); i++) {
      const UOp& r = n.src(i);
      if (r.op() == Op::Range && range_extent(r) == 1) sub[r] = UOp::const_int(0, DType::I32(), r.device());
      else keep.push_back(r);
    }
    if (sub.empty()) return UOp();
    std::vector<UOp> srcs{substitute_with_map(n.src(0), sub)};
    srcs.insert(srcs.end(), keep.begin(), keep.end());
    return UOp::make_new(Op::Reduce, n.dtype(), srcs, n.arg());
  };
  k = graph_rewrite(k, drop_unit);
  if (symbolic) k = graph_rewrite(k, symbolic_simple);
  // Output ranges map to the launch grid: retag LOOP as GLOBAL.
  auto retag = [](const UOp& n) -> UOp {
    if (n.op() != Op::Range || n.arg().range_kind() != AxisKind::Loop) return UOp();
    return UOp::make_new(Op::Range, n.dtype(), n.srcs(), Arg::range(n.arg().a, AxisKind::Global));
  };
  return graph_rewrite(k, retag);
}

// ── rendering helpers ───────────────────────────────────────────────────────
namespace {

// Elementwise outputs at least this large are written with non-temporal
// stores: half of MI355X's 256 MB Infinity Cache, beyond which a consumer
// kernel would find little of the output still cached anyway. Measured on a
// 2^26-element (a*b+c).relu() writing a fresh buffer each launch: 6.28 TB/s
// with non-temporal stores against 6.02 TB/s with plain ones.
constexpr int64_t kStreamingStoreBytes = int64_t(128) << 20;

// Threads per elementwise workgroup. Measured on the same 2^26-element
// (a*b+c).relu() with one float4 per thread and every load and store
// non-temporal, four rounds of 20 launches on one MI355X: 64 threads
// 6.33 TB/s, 128 threads 6.35, 256 threads 5.98, 1024 threads 6.19. Giving
// each XCD a contiguous eighth of the blocks instead did not help
// (128 threads: 6.05). Two float4 per thread at 128 threads: 5.93.
constexpr int kEwThreads = 128;

const char* ctype(DType d) {
  switch (d.kind) {
    case DTypeKind::F32: return "float";
    case DTypeKind::I32: return "int";
    case DTypeKind::Bool: return "bool";
    default: return "void";
  }
}

// Float literals use the text the reference emits (clang.rs:93-115): the
// shortest round-trip decimal of the f64 value with an `f` suffix, so both
// compilers round the same decimal to f32.
std::string float_lit(double v) {
  if (std::isinf(v)) return v > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
  if (std::isnan(v)) return "__builtin_nanf(\"\")";
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof(buf), v);
  std::string s(buf, r.ptr);
  if (s.find_first_of(".eE") == std::string::npos) s += ".0";
  return s + "f";
}

std::string const_lit(const UOp& c) {
  const Arg& a = c.arg();
  switch (a.kind) {
    case Arg::Kind::Float:
      if (c.dtype().kind == DTypeKind::F32) return float_lit(a.f);
      if (c.dtype().kind == DTypeKind::I32) return std::to_string(static_cast<int64_t>(a.f));
      return a.f != 0.0 ? "true" : "false";
    case Arg::Kind::Int:
      if (c.dtype().kind == DTypeKind::F32) return float_lit(static_cast<double>(a.a));
      if (c.dtype().kind == DTypeKind::Bool) return a.a ? "true" : "false";
      return std::to_string(a.a);
    case Arg::Kind::Bool:
      if (c.dtype().kind == DTypeKind::F32) return a.a ? "1.0f" : "0.0f";
      return a.a ? "true" : "false";
    default:
      fail("Const with unexpected arg");
  }
}

std::string pname(const UOp& p) { return "data" + std::to_string(p.arg().a); }

// Combine two values with a reduce op in the reference's operand order.
std::string combine(Op rop, const std::string& a, const std::string& b) {
  if (rop == Op::Add) return "(" + a + "+" + b + ")";
  if (rop == Op::Max) return "((" + a + ">" + b + ")?" + a + ":" + b + ")";
  fail("unsupported reduce op");
}

std::string init_lit(Op rop, DType dt) {  // devectorize.rs:219-225
  if (dt.kind != DTypeKind::F32) return rop == Op::Add ? "0" : "(-2147483647-1)";
  return rop == Op::Add ? "0.0f" : "(-__builtin_inff())";
}

// Scoped statement emitter for a value DAG. Each node is emitted once per
// (scope, lane); nodes are placed in the innermost open scope that defines a
// range they depend on, so loop-invariant loads hoist out of reduce loops.
class Emitter {
 public:
  struct Scope {
    std::string header, footer;
    std::ostringstream body;
    std::set<const UOpInner*> ranges;
    std::vector<std::pair<const UOpInner*, int>> keys;
    int indent = 1;
  };

  Emitter() { scopes_.emplace_back(new Scope()); }

  void define_range(const UOp& r, const std::string& expr) {
    range_expr_[r.get()] = expr;
    scopes_.back()->ranges.insert(r.get());
  }

  // The range whose value differs per lane: lane u reads `base + u`.
  void set_lane_range(const UOp& r, int lanes) {
    lane_range_ = r.get();
    lanes_ = lanes;
  }
  void clear_lane_range() {
    lane_range_ = nullptr;
    lanes_ = 1;
  }

  void open_scope(const std::string& header, const std::string& footer) {
    auto* s = new Scope();
    s->header = header;
    s->footer = footer;
    s->indent = scopes_.back()->indent + 1;
    scopes_.emplace_back(s);
  }

  void close_scope() {
    std::unique_ptr<Scope> s(scopes_.back().release());
    scopes_.pop_back();
    for (auto& k : s->keys) cache_.erase(k);
    for (auto* r : s->ranges) range_expr_.erase(r);
    Scope& p = *scopes_.back();
    std::string ind(static_cast<size_t>(p.indent) * 2, ' ');
    p.body << ind << s->header << "\n" << s->body.str() << ind << s->footer << "\n";
  }

  // Emit a raw line into the current (innermost) scope.
  void line(const std::string& l) {
    Scope& s = *scopes_.back();
    s.body << std::string(static_cast<size_t>(s.indent) * 2, ' ') << l << "\n";
  }

  std::string fresh(const char* prefix) { return std::string(prefix) + std::to_string(counter_++); }

  std::string code() { return scopes_.front()->body.str(); }

  bool depends_on(const UOp& n, const UOpInner* r) {
    if (!r) return false;
    auto key = std::make_pair(n.get(), r);
    auto it = dep_cache_.find(key);
    if (it != dep_cache_.end()) return it->second;
    bool d = n.get() == r;
    if (!d)
      for (auto& s : n.srcs())
        if (depends_on(s, r)) {
          d = true;
          break;
        }
    dep_cache_[key] = d;
    return d;
  }

  // Index of the innermost open scope that defines a range `n` depends on
  // (with no hoisting: the innermost open scope).
  size_t scope_of(const UOp& n) {
    if (no_hoist_) return scopes_.size() - 1;
    size_t best = 0;
    for (size_t i = scopes_.size(); i-- > 1;) {
      for (auto* r : scopes_[i]->ranges) {
        if (depends_on(n, r)) return i;
      }
    }
    return best;
  }

  std::string idx(const UOp& e, int lane) {
    switch (e.op()) {
      case Op::Const: return const_lit(e);
      case Op::ParamScalar: return pname(e);
      case Op::Range: {
        auto it = range_expr_.find(e.get());
        FG_CHECK(it != range_expr_.end(), "range used outside its scope");
        if (e.get() == lane_range_ && lane > 0) return "(" + it->second + "+" + std::to_string(lane) + ")";
        return it->second;
      }
      case Op::Add: return "(" + idx(e.src(0), lane) + "+" + idx(e.src(1), lane) + ")";
      case Op::Mul: return "(" + idx(e.src(0), lane) + "*" + idx(e.src(1), lane) + ")";
      default: break;
    }
    // Non-index ops inside an int expression are values.
    return val(e, lane);
  }

  // Vectorised load check: unit stride along the lane range, every other
  // term a multiple of 4 (16-byte aligned for 4-byte elements). Kernel-scalar
  // terms are int32 values, so a coefficient that is a multiple of 4 keeps
  // the alignment too.
  bool vec4_load(const UOp& load) {
    if (lanes_ != 4 || !lane_range_) return false;
    DType dt = load.dtype();
    if (dt.kind != DTypeKind::F32 && dt.kind != DTypeKind::I32) return false;
    Affine a = affine_of(load.src(0).src(1));
    if (!a.ok || a.c0 % 4 != 0) return false;
    bool unit = false;
    for (auto& t : a.terms) {
      if (t.first.get() == lane_range_) unit = t.second == 1;
      else if (t.second % 4 != 0) return false;
    }
    return unit && lane_base_aligned_;
  }
  void set_lane_base_aligned(bool b) { lane_base_aligned_ = b; }
  // Every value is emitted where it is first used instead of in the
  // outermost scope it could live in: a load then runs after every store the
  // program order puts before it (in-place kernels run sequentially).
  void set_no_hoist(bool b) { no_hoist_ = b; }
  void set_nontemporal_loads(bool b) { nt_loads_ = b; }
  // Loads of the buffers in `rsrc` (ParamBuffer -> resource name) render as
  // raw buffer loads: a 32-bit byte offset per lane, and the `k` range's term
  // as a uniform byte offset `coef * size * kvar` in the scalar offset. The
  // caller renders `k` as its per-lane part only (the k-tile's start is
  // `kvar`), and every index must be affine with non-negative terms.
  void set_buffer_loads(std::map<const UOpInner*, std::string> rsrc, const UOp& k, const std::string& kvar) {
    buf_rsrc_ = std::move(rsrc);
    buf_k_ = k;
    buf_kvar_ = kvar;
  }
  // Non-temporal loads only for addresses that depend on every one of these
  // ranges (the kernel's output ranges): such an element is read by one
  // output only. Loads shared by several outputs stay cacheable.
  void set_streaming_ranges(const std::vector<UOp>& rs) {
    nt_ranges_.clear();
    for (auto& r : rs) nt_ranges_.push_back(r.get());
  }
  bool streams(const UOp& index) {
    if (!nt_loads_) return false;
    for (auto* r : nt_ranges_)
      if (!depends_on(index, r)) return false;
    return true;
  }

  std::string val(const UOp& n, int lane) {
    bool lane_dep = lane_range_ && depends_on(n, lane_range_);
    int key_lane = lane_dep ? lane : -1;
    auto key = std::make_pair(n.get(), key_lane);
    auto it = cache_.find(key);
    if (it != cache_.end()) return it->second;
    std::string out;
    switch (n.op()) {
      case Op::Const: return const_lit(n);
      case Op::ParamScalar: return pname(n);
      case Op::Range: case Op::Add: case Op::Mul:
        if (n.dtype().kind == DTypeKind::I32 && (n.op() == Op::Range || is_index_expr(n))) return idx(n, lane);
        break;
      default: break;
    }
    size_t si = scope_of(n);
    if (n.op() == Op::Load && load_cb_) {
      // A load whose value the caller already holds (e.g. in a register).
      std::string held = load_cb_(n, lane);
      if (!held.empty()) {
        remember(si, key, held);
        return held;
      }
    }
    if (n.op() == Op::Load) {
      const UOp& ix = n.src(0);
      FG_CHECK(ix.op() == Op::Index, "Load must read through Index");
      auto rs = buf_rsrc_.find(ix.src(0).get());
      if (rs != buf_rsrc_.end()) {
        Affine a = affine_of(ix.src(1));
        FG_CHECK(a.ok, "a buffer load needs an affine index");
        const int64_t esz = n.dtype().size_bytes();
        FG_CHECK(esz == 4, "buffer loads read 4-byte elements");
        const std::string soff = "(unsigned)(" + std::to_string(a.coef(buf_k_) * esz) + " * " + buf_kvar_ + ")";
        const bool f32 = n.dtype().kind == DTypeKind::F32;
        if (lane_dep && vec4_load(n)) {
          std::string v = fresh("vec");
          const char* vt = f32 ? "fg_f4" : "fg_i4";
          emit_at(si, std::string("const ") + vt + " " + v + " = __builtin_bit_cast(" + vt +
                          ", __builtin_amdgcn_raw_buffer_load_b128(" + rs->second + ", (unsigned)(" +
                          idx(ix.src(1), 0) + ") * 4u, " + soff + ", 0));");
          static const char* comp[4] = {".x", ".y", ".z", ".w"};
          for (int u = 0; u < 4; u++) remember(si, std::make_pair(n.get(), u), v + comp[u]);
          return v + comp[lane];
        }
        std::string v = fresh("val");
        emit_at(si, std::string(ctype(n.dtype())) + " " + v + " = __builtin_bit_cast(" + ctype(n.dtype()) +
                        ", __builtin_amdgcn_raw_buffer_load_b32(" + rs->second + ", (unsigned)(" +
                        idx(ix.src(1), lane) + ") * 4u, " + soff + ", 0));");
        remember(si, key, v);
        return v;
      }
      if (lane_dep && vec4_load(n)) {
        std::string v = fresh("vec");
        const char* vt = n.dtype().kind == DTypeKind::F32 ? "fg_f4" : "fg_i4";
        std::string addr = std::string("(const ") + vt + "*)(" + pname(ix.src(0)) + "+" + idx(ix.src(1), 0) + ")";
        // Streaming kernels read each element once: non-temporal 16-byte loads.
        std::string rhs = streams(ix.src(1)) ? "__builtin_nontemporal_load(" + addr + ")" : "*" + addr;
        emit_at(si, std::string("const ") + vt + " " + v + " = " + rhs + ";");
        static const char* comp[4] = {".x", ".y", ".z", ".w"};
        for (int u = 0; u < 4; u++) remember(si, std::make_pair(n.get(), u), v + comp[u]);
        return v + comp[lane];
      }
      std::string v = fresh("val");
      emit_at(si, std::string(ctype(n.dtype())) + " " + v + " = " + pname(ix.src(0)) + "[" + idx(ix.src(1), lane) + "];");
      out = v;
    } else if (n.op() == Op::Reduce) {
      FG_CHECK(reduce_cb_, "Reduce reached a renderer without reduction support");
      out = reduce_cb_(n, lane);
      return out;  // the callback caches its own result
    } else {
      std::vector<std::string> s;
      for (auto& x : n.srcs()) s.push_back(val(x, lane));
      // Placed after its sources are emitted: a source reduction may have
      // pinned itself to the scope it ran in.
      si = scope_of(n);
      std::string e;
      switch (n.op()) {
        case Op::Neg: e = "(-" + s[0] + ")"; break;
        case Op::Exp2: e = "(float)exp2((double)" + s[0] + ")"; break;   // clang.rs:218 (double exp2)
        case Op::Log2: e = "(float)log2((double)" + s[0] + ")"; break;   // clang.rs:219 (double log2)
        case Op::Sqrt: e = "__fsqrt_rn(" + s[0] + ")"; break;            // correctly rounded, as sqrtf
        case Op::Reciprocal:
          e = n.dtype().kind == DTypeKind::F32 ? "__fdiv_rn(1.0f," + s[0] + ")" : "(1/" + s[0] + ")";
          break;
        case Op::Add: e = "(" + s[0] + "+" + s[1] + ")"; break;
        case Op::Mul: e = "(" + s[0] + "*" + s[1] + ")"; break;
        case Op::Max: e = "((" + s[0] + ">" + s[1] + ")?" + s[0] + ":" + s[1] + ")"; break;
        case Op::CmpLt: e = "(" + s[0] + "<" + s[1] + ")"; break;
        case Op::Where: e = "(" + s[0] + "?" + s[1] + ":" + s[2] + ")"; break;
        default: fail(std::string("HIP renderer cannot emit ") + op_name(n.op()));
      }
      std::string v = fresh("alu");
      emit_at(si, std::string(ctype(n.dtype())) + " " + v + " = " + e + ";");
      out = v;
    }
    remember(si, key, out);
    return out;
  }

  void remember(size_t si, std::pair<const UOpInner*, int> key, const std::string& name) {
    cache_[key] = name;
    scopes_[si]->keys.push_back(key);
  }
  // Treat `n` as defined by the current scope, so nodes that depend on it
  // (a reduction's epilogue inside a loop over outputs) are placed in it.
  void pin_here(const UOp& n) { scopes_.back()->ranges.insert(n.get()); }
  void remember_here(const UOp& n, int lane, const std::string& name) {
    bool lane_dep = lane_range_ && depends_on(n, lane_range_);
    remember(scopes_.size() - 1, std::make_pair(n.get(), lane_dep ? lane : -1), name);
  }

  void emit_at(size_t si, const std::string& l) {
    Scope& s = *scopes_[si];
    s.body << std::string(static_cast<size_t>(s.indent) * 2, ' ') << l << "\n";
  }

  size_t depth() const { return scopes_.size(); }

  std::function<std::string(const UOp&, int)> reduce_cb_;
  // Optional: returns the expression holding a load's value (empty: emit the load).
  std::function<std::string(const UOp&, int)> load_cb_;

 private:
  std::map<const UOpInner*, std::string> buf_rsrc_;
  UOp buf_k_;
  std::string buf_kvar_;
  static bool is_index_expr(const UOp& n) {
    if (n.op() == Op::Range || n.op() == Op::Const || n.op() == Op::ParamScalar) return true;
    if (n.op() == Op::Add || n.op() == Op::Mul) return is_index_expr(n.src(0)) && is_index_expr(n.src(1));
    return false;
  }

  std::vector<std::unique_ptr<Scope>> scopes_;
  std::map<std::pair<const UOpInner*, int>, std::string> cache_;
  std::map<std::pair<const UOpInner*, const UOpInner*>, bool> dep_cache_;
  std::unordered_map<const UOpInner*, std::string> range_expr_;
  const UOpInner* lane_range_ = nullptr;
  int lanes_ = 1;
  bool lane_base_aligned_ = true;
  bool nt_loads_ = false;
  bool no_hoist_ = false;
  std::vector<const UOpInner*> nt_ranges_;
  int counter_ = 0;
};

std::string signature(const KernelInfo& ki, const std::string& name, int block) {
  std::ostringstream os;
  os << "extern \"C\" __global__ void __launch_bounds__(" << block << ") " << name << "(";
  bool first = true;
  // Find which buffers are written (the store target) to drop const.
  for (auto& [slot, p] : ki.params) {
    if (!first) os << ", ";
    first = false;
    if (p.op() == Op::ParamBuffer) {
      bool written = p == ki.out_param;
      os << (written ? "" : "const ") << ctype(p.dtype()) << "* __restrict__ data" << slot;
    } else {
      os << ctype(p.dtype()) << " data" << slot;
    }
  }
  os << ")";
  return os.str();
}

const char* kPrelude = R"(// generated by ferrograd_amd for gfx950
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float fg_f4 __attribute__((ext_vector_type(4)));
typedef int fg_i4 __attribute__((ext_vector_type(4)));
// Cross-lane moves on 32-bit values. DPP row-local patterns for distances
// inside a row of 16 lanes, ds_swizzle for 16, ds_bpermute for 32.
#define FG_DPP(v, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false))
#define FG_DPPI(v, ctrl) (__builtin_amdgcn_update_dpp(0, (v), ctrl, 0xF, 0xF, false))
__device__ __forceinline__ float fg_swz16_f(float v) { return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)); }
__device__ __forceinline__ int fg_swz16_i(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }
__device__ __forceinline__ float fg_x32_f(float v) { return __int_as_float(__builtin_amdgcn_ds_bpermute(((int)(threadIdx.x ^ 32u)) << 2, __float_as_int(v))); }
__device__ __forceinline__ int fg_x32_i(int v) { return __builtin_amdgcn_ds_bpermute(((int)(threadIdx.x ^ 32u)) << 2, v); }
)";

// Group-of-T lane reduction (T a power of two <= 64, groups aligned to T).
// quad_perm xor1 (0xB1), xor2 (0x4E); row_half_mirror (0x141) and row_mirror
// (0x140) pair each half with the reflected half, so after each step every
// lane of the group holds the group total.
std::string wave_reduce(const std::string& var, int T, Op rop, DType dt) {
  std::ostringstream os;
  bool f = dt.kind == DTypeKind::F32;
  auto step = [&](const std::string& other) {
    os << "{ " << ctype(dt) << " o = " << other << "; " << var << " = " << combine(rop, var, "o") << "; }\n";
  };
  const char* dpp = f ? "FG_DPP" : "FG_DPPI";
  if (T >= 2) step(std::string(dpp) + "(" + var + ", 0xB1)");
  if (T >= 4) step(std::string(dpp) + "(" + var + ", 0x4E)");
  if (T >= 8) step(std::string(dpp) + "(" + var + ", 0x141)");
  if (T >= 16) step(std::string(dpp) + "(" + var + ", 0x140)");
  if (T >= 32) step(std::string(f ? "fg_swz16_f(" : "fg_swz16_i(") + var + ")");
  if (T >= 64) step(std::string(f ? "fg_x32_f(" : "fg_x32_i(") + var + ")");
  return os.str();
}

int pow2_floor(int64_t x) {
  int p = 1;
  while (static_cast<int64_t>(p) * 2 <= x) p *= 2;
  return p;
}

// Decode the flattened output index `lin` into range variables (innermost
// range varies fastest). Emits `int idxN = ...;` lines, skipping `skip`.
void decode_outputs(Emitter& em, const KernelInfo& ki, const std::string& lin, const UOp& skip) {
  std::string rest = lin;
  bool first = true;
  for (size_t i = ki.out_ranges.size(); i-- > 0;) {
    const UOp& r = ki.out_ranges[i];
    if (r == skip) continue;
    std::string name = "idx" + std::to_string(r.arg().a);
    int64_t e = ki.out_ext[i];
    // Is this the outermost remaining range? Then no modulo is needed.
    bool outermost = true;
    for (size_t j = 0; j < i; j++)
      if (ki.out_ranges[j] != skip) outermost = false;
    if (outermost) em.line("const int " + name + " = (int)(" + rest + ");");
    else em.line("const int " + name + " = (int)((" + rest + ") % " + std::to_string(e) + ");");
    em.define_range(r, name);
    if (!outermost) {
      std::string nr = "rest" + std::to_string(i);
      em.line("const long " + nr + " = (" + rest + ") / " + std::to_string(e) + ";");
      rest = nr;
    }
    first = false;
  }
  (void)first;
}

UOp pick_fast_output(const KernelInfo& ki) {
  if (ki.out_ranges.empty()) return UOp();
  Affine a = affine_of(ki.out_index);
  for (auto& r : ki.out_ranges)
    if (a.ok && a.coef(r) == 1) return r;
  return ki.out_ranges.back();
}

int64_t total_outputs(const KernelInfo& ki) {
  int64_t t = 1;
  for (auto e : ki.out_ext) t *= e;
  return t;
}

// Serial reduction in the reference's exact order: loops over the reduce
// ranges in source order; the innermost splits into REDUCE x UNROLL(4) when its
// extent is a multiple of 4 above 4 (unroll.rs:41-113), and each outer step
// folds acc = acc (op) (((v0 op v1) op v2) op v3) (devectorize.rs:206-214, 306-319).
//
// The loops carry unroll bounds. Left to itself, LLVM fully unrolls a nest of
// constant-trip loops; for a Max fold (a chain of compare-selects) over a few
// hundred float4 loads, e.g. max over axes [1,2,3] of f32[6,8,10,12] (8 x 10 x 3
// trips), hiprtc at -O3 then does not finish at all. So only a nest of at most
// kSerialFullUnroll iterations, with no reduction inside its value, may unroll
// fully; otherwise every loop but the innermost runs rolled and the innermost
// unrolls by at most 4. Unrolling never reorders the fold: the operations stay
// in source order, and no reassociation is allowed (no fast-math).
constexpr int64_t kSerialFullUnroll = 16;

std::string emit_serial_reduce(Emitter& em, const UOp& R, int lane_outer) {
  (void)lane_outer;
  Op rop = R.arg().rop;
  std::vector<UOp> ranges(R.srcs().begin() + 1, R.srcs().end());
  std::string acc = em.fresh("acc");
  em.line(std::string(ctype(R.dtype())) + " " + acc + " = " + init_lit(rop, R.dtype()) + ";");
  const UOp& value = R.src(0);
  bool nested = false;
  for (auto& n : value.toposort()) nested = nested || n.op() == Op::Reduce;
  // Trip count of each loop (the innermost one steps by 4 lanes when it splits).
  std::vector<int64_t> trips;
  for (size_t i = 0; i < ranges.size(); i++) {
    int64_t ext = range_extent(ranges[i]);
    bool last = i + 1 == ranges.size();
    trips.push_back(last && ext > 4 && ext % 4 == 0 ? ext / 4 : ext);
  }
  int64_t nest = 1;
  for (auto t : trips) nest *= t;
  const bool bounded = nested || nest > kSerialFullUnroll;
  size_t opened = 0;
  int unroll = 1;
  std::string unroll_var;
  for (size_t i = 0; i < ranges.size(); i++) {
    const UOp& r = ranges[i];
    int64_t ext = range_extent(r);
    std::string v = "ridx" + std::to_string(r.arg().a) + "_" + std::to_string(em.depth());
    bool last = i + 1 == ranges.size();
    std::string pragma;
    if (bounded) pragma = (last && !nested && trips[i] <= 4) ? "" : (last && !nested) ? "#pragma unroll 4\n" : "#pragma unroll 1\n";
    if (last && ext > 4 && ext % 4 == 0) {
      unroll = 4;
      unroll_var = v;
      em.open_scope(pragma + "for (int " + v + " = 0; " + v + " < " + std::to_string(ext / 4) + "; " + v + "++) {", "}");
      em.define_range(r, "(" + v + "*4)");
      em.set_lane_range(r, 4);
    } else {
      em.open_scope(pragma + "for (int " + v + " = 0; " + v + " < " + std::to_string(ext) + "; " + v + "++) {", "}");
      em.define_range(r, v);
    }
    opened++;
  }
  std::string group;
  if (unroll == 4 && nested) {
    // A reduction in the value sets its own lane range while it is emitted,
    // so the four lanes are emitted one after another instead, each in a
    // scope of its own with the unrolled range fixed to that lane's index;
    // the fold order stays (((v0 op v1) op v2) op v3).
    em.clear_lane_range();
    const UOp& r = ranges.back();
    std::vector<std::string> lanes;
    for (int u = 0; u < 4; u++) {
      std::string t = em.fresh("lane");
      em.line(std::string(ctype(value.dtype())) + " " + t + ";");
      em.open_scope("{", "}");
      em.define_range(r, "(" + unroll_var + "*4+" + std::to_string(u) + ")");
      em.line(t + " = " + em.val(value, 0) + ";");
      em.close_scope();
      lanes.push_back(t);
    }
    group = lanes[0];
    for (int u = 1; u < 4; u++) group = combine(rop, group, lanes[u]);
  } else if (unroll == 4) {
    std::vector<std::string> lanes;
    for (int u = 0; u < 4; u++) lanes.push_back(em.val(value, u));
    group = lanes[0];
    for (int u = 1; u < 4; u++) group = combine(rop, group, lanes[u]);
  } else {
    group = em.val(value, 0);
  }
  em.line(acc + " = " + combine(rop, acc, group) + ";");
  if (unroll == 4) em.clear_lane_range();
  for (size_t i = 0; i < opened; i++) em.close_scope();
  return acc;
}

// ── Serial / fallback ───────────────────────────────────────────────────────
RenderedKernel render_serial(const KernelInfo& ki, const std::string& name) {
  Emitter em;
  int64_t T = total_outputs(ki);
  em.line("const long gid = (long)blockIdx.x * 256 + threadIdx.x;");
  em.line("if (gid >= " + std::to_string(T) + "L) return;");
  decode_outputs(em, ki, "gid", UOp());
  em.reduce_cb_ = [&](const UOp& R, int lane) {
    std::string acc = emit_serial_reduce(em, R, lane);
    em.remember_here(R, lane, acc);
    return acc;
  };
  std::string v = em.val(ki.value, 0);
  em.line(pname(ki.out_param) + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::Serial);
  rk.source = std::string(kPrelude) + signature(ki, name, 256) + " {\n" + em.code() + "}\n";
  rk.block[0] = 256;
  rk.grid[0] = static_cast<unsigned>((T + 255) / 256);
  return rk;
}

// ── Sequential: in-place updates that read their destination elsewhere ─────
// The reference compiles such a kernel to nested C loops and calls it once on
// one thread (clang.rs:28-280, cpu.rs:373-377), so each load sees the stores
// the loop order puts before it, e.g. w.assign(w + wᵀ) reads elements the
// same call has already overwritten. No parallel mapping keeps that, so one
// thread runs the kernel in that order: output loops outermost first, each
// output's value computed right before its store, every load emitted where
// it is used (no hoisting out of a loop). The innermost output loop is split
// into groups of 4 lanes where the reference's upcast pass splits it
// (upcast.rs:79-104: the last output loop, extent above 4 and a multiple of
// 4, no ALU between a reduction and the store). Within a group the
// reference evaluates the lanes' reductions, and the values no lane index
// reaches, before the first lane's store, then each lane's value and store
// in lane order; so does this kernel. Reductions fold in the reference's
// order (emit_serial_reduce).
RenderedKernel render_sequential(const KernelInfo& ki, const std::string& name) {
  Emitter em;
  em.set_no_hoist(true);
  em.reduce_cb_ = [&](const UOp& R, int lane) {
    std::string acc = emit_serial_reduce(em, R, lane);
    em.remember_here(R, lane, acc);
    return acc;
  };
  em.line("if (blockIdx.x != 0 || threadIdx.x != 0) return;");
  const size_t nr = ki.out_ranges.size();
  const bool post_reduce_alu = ki.value.op() != Op::Reduce && !ki.reduces.empty();
  const bool upcast = nr > 0 && ki.out_ext[nr - 1] > 4 && ki.out_ext[nr - 1] % 4 == 0 && !post_reduce_alu;
  for (size_t i = 0; i + (upcast ? 1 : 0) < nr; i++) {
    const UOp& r = ki.out_ranges[i];
    const std::string v = "idx" + std::to_string(r.arg().a);
    em.open_scope("#pragma unroll 1\nfor (int " + v + " = 0; " + v + " < " + std::to_string(ki.out_ext[i]) + "; " + v +
                      "++) {",
                  "}");
    em.define_range(r, v);
  }
  auto store = [&] {
    std::string v = em.val(ki.value, 0);
    em.line(pname(ki.out_param) + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
  };
  if (upcast) {
    const UOp& r = ki.out_ranges[nr - 1];
    const std::string g = "grp" + std::to_string(r.arg().a);
    em.open_scope("#pragma unroll 1\nfor (int " + g + " = 0; " + g + " < " + std::to_string(ki.out_ext[nr - 1] / 4) +
                      "; " + g + "++) {",
                  "}");
    auto lane_index = [&](int u) { return "(" + g + "*4+" + std::to_string(u) + ")"; };
    // The value's largest subexpressions that no lane index reaches, and the
    // reductions (outside other reductions) that one does.
    std::vector<UOp> invariant, lane_reduces;
    UOpSet seen;
    // Loads and reductions are leaves of this walk; it descends through ALU.
    std::function<void(const UOp&)> walk = [&](const UOp& n) {
      if (!seen.insert(n).second) return;
      if (n.op() == Op::Const || n.op() == Op::ParamScalar || n.op() == Op::Range ||
          ((n.op() == Op::Add || n.op() == Op::Mul) && n.dtype().kind == DTypeKind::I32))
        return;  // index arithmetic, rendered inline
      if (!em.depends_on(n, r.get())) {
        invariant.push_back(n);
        return;
      }
      if (n.op() == Op::Reduce) lane_reduces.push_back(n);
      if (n.op() == Op::Reduce || n.op() == Op::Load) return;
      for (auto& x : n.srcs()) walk(x);
    };
    walk(ki.value);
    for (auto& n : invariant) em.val(n, 0);
    std::vector<std::vector<std::string>> held(4);
    for (int u = 0; u < 4; u++) {
      for (auto& R : lane_reduces) {
        std::string h = em.fresh("lred");
        em.line(std::string(ctype(R.dtype())) + " " + h + ";");
        em.open_scope("{", "}");
        em.define_range(r, lane_index(u));
        std::string acc = em.val(R, 0);
        em.line(h + " = " + acc + ";");
        em.close_scope();
        held[u].push_back(h);
      }
    }
    for (int u = 0; u < 4; u++) {
      em.open_scope("{", "}");
      em.define_range(r, lane_index(u));
      for (size_t k = 0; k < lane_reduces.size(); k++) em.remember_here(lane_reduces[k], 0, held[u][k]);
      store();
      em.close_scope();
    }
    em.close_scope();
  } else {
    store();
  }
  for (size_t i = 0; i + (upcast ? 1 : 0) < nr; i++) em.close_scope();
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::Sequential);
  rk.source = std::string(kPrelude) + signature(ki, name, 64) + " {\n" + em.code() + "}\n";
  rk.block[0] = 64;
  rk.grid[0] = 1;
  return rk;
}

// ── Elementwise ─────────────────────────────────────────────────────────────
RenderedKernel render_elementwise(const KernelInfo& ki, const std::string& name) {
  Emitter em;
  em.set_nontemporal_loads(true);
  em.set_streaming_ranges(ki.out_ranges);
  UOp fast = pick_fast_output(ki);
  int64_t T = total_outputs(ki);
  int V = 1;
  int64_t fext = 1;
  if (fast) {
    for (size_t i = 0; i < ki.out_ranges.size(); i++)
      if (ki.out_ranges[i] == fast) fext = ki.out_ext[i];
    if (fext % 4 == 0) V = 4;
  }
  int64_t threads = T / V;
  em.line("const long gid = (long)blockIdx.x * " + std::to_string(kEwThreads) + " + threadIdx.x;");
  em.line("if (gid >= " + std::to_string(threads) + "L) return;");
  if (V == 4) {
    int64_t per = fext / 4;
    em.line("const int fbase = (int)(gid % " + std::to_string(per) + ") * 4;");
    em.line("const long orest = gid / " + std::to_string(per) + ";");
    em.define_range(fast, "fbase");
    decode_outputs(em, ki, "orest", fast);
    em.set_lane_range(fast, 4);
  } else {
    decode_outputs(em, ki, "gid", UOp());
  }
  std::vector<std::string> vals;
  for (int u = 0; u < V; u++) vals.push_back(em.val(ki.value, u));
  const std::string out = pname(ki.out_param);
  bool vstore = false;
  if (V == 4) {
    Affine a = affine_of(ki.out_index);
    DType dt = ki.out_param.dtype();
    vstore = a.ok && a.coef(fast) == 1 && a.c0 % 4 == 0 &&
             (dt.kind == DTypeKind::F32 || dt.kind == DTypeKind::I32);
    for (auto& t : a.terms)
      if (t.first != fast && t.second % 4 != 0) vstore = false;
    if (vstore) {
      const std::string addr = out + "+" + em.idx(ki.out_index, 0);
      const std::string four = vals[0] + ", " + vals[1] + ", " + vals[2] + ", " + vals[3];
      if (static_cast<int64_t>(T) * static_cast<int64_t>(dt.size_bytes()) >= kStreamingStoreBytes) {
        // Too large to stay in the Infinity Cache for a consumer: write it
        // past the caches instead of evicting the inputs' lines.
        const char* vt = dt.kind == DTypeKind::F32 ? "fg_f4" : "fg_i4";
        em.line(std::string("const ") + vt + " vout = {" + four + "};");
        em.line(std::string("__builtin_nontemporal_store(vout, (") + vt + "*)(" + addr + "));");
      } else {
        const char* vt = dt.kind == DTypeKind::F32 ? "float4" : "int4";
        const char* mk = dt.kind == DTypeKind::F32 ? "make_float4" : "make_int4";
        em.line(std::string("*(") + vt + "*)(" + addr + ") = " + mk + "(" + four + ");");
      }
    }
  }
  if (!vstore)
    for (int u = 0; u < V; u++) em.line(out + "[" + em.idx(ki.out_index, u) + "] = " + vals[u] + ";");
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::Elementwise);
  rk.source = std::string(kPrelude) + signature(ki, name, kEwThreads) + " {\n" + em.code() + "}\n";
  rk.block[0] = kEwThreads;
  rk.grid[0] = static_cast<unsigned>((threads + kEwThreads - 1) / kEwThreads);
  return rk;
}

// Loads inside the reduced value.
std::vector<UOp> loads_in(const UOp& v) {
  std::vector<UOp> out;
  for (auto& n : v.toposort())
    if (n.op() == Op::Load) out.push_back(n);
  return out;
}

// ── RowReduce ───────────────────────────────────────────────────────────────
RenderedKernel render_row_reduce(const KernelInfo& ki, const std::string& name) {
  const UOp& R = ki.reduces[0];
  Op rop = R.arg().rop;
  DType dt = R.dtype();
  std::vector<UOp> ranges(R.srcs().begin() + 1, R.srcs().end());
  const UOp r_in = ranges.back();
  int64_t L = range_extent(r_in);
  int T = std::min<int>(256, pow2_floor(std::max<int64_t>(1, L / 16)));
  int OPW = 256 / T;  // outputs per workgroup
  int64_t NOUT = total_outputs(ki);
  // Vector width along r_in: all lane-dependent loads unit-stride and aligned.
  int V = (L % 4 == 0) ? 4 : 1;
  if (V == 4) {
    for (auto& ld : loads_in(R.src(0))) {
      Affine a = affine_of(ld.src(0).src(1));
      int64_t c = a.ok ? a.coef(r_in) : -1;
      if (c == 0) continue;
      bool ok = a.ok && c == 1 && a.c0 % 4 == 0 &&
                (ld.dtype().kind == DTypeKind::F32 || ld.dtype().kind == DTypeKind::I32);
      for (auto& t : a.terms)
        if (t.first != r_in && t.second % 4 != 0) ok = false;
      if (!ok) V = 1;
    }
  }
  Emitter em;
  em.set_nontemporal_loads(true);
  em.set_streaming_ranges(ki.out_ranges);
  const int64_t grid = (NOUT + OPW - 1) / OPW;
  em.line("const int tid = threadIdx.x;");
  em.line("const int rlane = tid % " + std::to_string(T) + ";");
  // Whether some streamed operand (one that varies along the reduce axis) is
  // read by several outputs: the same row for every output column of a
  // narrow matmul.
  bool shared_rows = false;
  for (auto& ld : loads_in(R.src(0))) {
    const UOp& ix = ld.src(0).src(1);
    if (!em.depends_on(ix, r_in.get())) continue;
    for (auto& o : ki.out_ranges)
      if (!em.depends_on(ix, o.get())) shared_rows = true;
  }
  if (shared_rows && grid % 8 == 0) {
    // Workgroups are dispatched round-robin over the 8 XCDs: give each XCD a
    // contiguous run of outputs, so the outputs that share an input row read
    // it through one L2. (Outputs that each stream their own rows keep the
    // interleaved order, which spreads the 8 XCDs' reads over HBM better.)
    em.line("const long bid = (long)(blockIdx.x % 8) * " + std::to_string(grid / 8) + " + blockIdx.x / 8;");
  } else {
    em.line("const long bid = blockIdx.x;");
  }
  em.line("const long oid = bid * " + std::to_string(OPW) + " + tid / " + std::to_string(T) + ";");
  em.line("const bool active = oid < " + std::to_string(NOUT) + "L;");
  em.line("const long ocl = active ? oid : 0;");
  decode_outputs(em, ki, "ocl", UOp());
  std::string result;
  em.reduce_cb_ = [&](const UOp& RR, int lane) -> std::string {
    FG_CHECK(RR == R, "row reduce renders exactly one reduction");
    std::string acc = "racc";
    em.line(std::string(ctype(dt)) + " " + acc + " = " + init_lit(rop, dt) + ";");
    size_t opened = 0;
    for (size_t i = 0; i + 1 < ranges.size(); i++) {
      std::string v = "ro" + std::to_string(i);
      em.open_scope("for (int " + v + " = 0; " + v + " < " + std::to_string(range_extent(ranges[i])) + "; " + v + "++) {",
                    "}");
      em.define_range(ranges[i], v);
      opened++;
    }
    // Each thread strides the row by T*V elements. The full strides run as a
    // fixed-trip, unrolled loop so every thread's loads are in flight at once
    // (11.3 vs 12.2 us at C1); a row that is not a multiple of T*V ends with
    // one guarded partial stride.
    const int64_t stride = static_cast<int64_t>(T) * V, nfull = L / stride;
    auto fold = [&]() {
      std::string group;
      if (V == 4) {
        em.set_lane_range(r_in, 4);
        std::vector<std::string> lanes;
        for (int u = 0; u < 4; u++) lanes.push_back(em.val(R.src(0), u));
        group = combine(rop, combine(rop, combine(rop, lanes[0], lanes[1]), lanes[2]), lanes[3]);
      } else {
        group = em.val(R.src(0), 0);
      }
      em.line(acc + " = " + combine(rop, acc, group) + ";");
      if (V == 4) em.clear_lane_range();
    };
    em.open_scope("if (active) {", "}");
    opened++;
    if (nfull > 0) {
      em.open_scope(std::string(nfull <= 16 ? "#pragma unroll" : "#pragma unroll 8") + "\nfor (int rit = 0; rit < " +
                        std::to_string(nfull) + "; rit++) {",
                    "}");
      em.line("const int rj = rlane * " + std::to_string(V) + " + rit * " + std::to_string(stride) + ";");
      em.define_range(r_in, "rj");
      fold();
      em.close_scope();
    }
    if (L % stride != 0) {
      em.open_scope("{ const int rj = rlane * " + std::to_string(V) + " + " + std::to_string(nfull * stride) +
                        "; if (rj < " + std::to_string(L) + ") {",
                    "} }");
      em.define_range(r_in, "rj");
      fold();
      em.close_scope();
    }
    for (size_t i = 0; i < opened; i++) em.close_scope();
    // Tree across the T threads of this output.
    if (T > 1) {
      int tw = std::min(T, 64);
      std::string wr = wave_reduce(acc, tw, rop, dt);
      std::istringstream is(wr);
      std::string l;
      while (std::getline(is, l)) em.line(l);
    }
    if (T > 64) {
      int nw = T / 64;
      em.line(std::string("__shared__ ") + ctype(dt) + " fg_part[4];");
      em.line("if ((tid & 63) == 0) fg_part[tid >> 6] = " + acc + ";");
      em.line("__syncthreads();");
      em.line("{ const int g0 = (tid >> 6) & ~" + std::to_string(nw - 1) + "; " + acc + " = fg_part[g0];");
      for (int w = 1; w < nw; w++) em.line("  " + acc + " = " + combine(rop, acc, "fg_part[g0+" + std::to_string(w) + "]") + ";");
      em.line("}");
    }
    em.remember_here(RR, lane, acc);
    return acc;
  };
  std::string v = em.val(ki.value, 0);
  (void)result;
  em.line("if (active && rlane == 0) " + pname(ki.out_param) + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::RowReduce);
  rk.source = std::string(kPrelude) + signature(ki, name, 256) + " {\n" + em.code() + "}\n";
  rk.block[0] = 256;
  rk.grid[0] = static_cast<unsigned>((NOUT + OPW - 1) / OPW);
  return rk;
}

// ── ColumnReduce ────────────────────────────────────────────────────────────
// Two-pass column reduction. Pass 1 (`<name>_part`): workgroup (block, chunk)
// reduces rows [chunk*CH, (chunk+1)*CH) of its output block and writes one
// partial per output to scratch[chunk][out]. Pass 2 (`<name>_fin`): one thread
// per 4 outputs folds the partials in chunk order and applies the epilogue.
RenderedKernel render_column_reduce_split(const KernelInfo& ki, const std::string& name, int V, int TX, int TR,
                                          int64_t per_f, int64_t other, int64_t fext, int64_t nchunks) {
  const UOp& R = ki.reduces[0];
  Op rop = R.arg().rop;
  DType dt = R.dtype();
  const UOp r = R.src(1);
  int64_t L = range_extent(r);
  int64_t CH = (L + nchunks - 1) / nchunks;
  nchunks = (L + CH - 1) / CH;
  UOp fast = pick_fast_output(ki);
  const int64_t NOUT = fext * other;
  const std::string sig_extra = std::string(", ") + ctype(dt) + "* __restrict__ fg_scratch";
  auto sig = [&](const std::string& fn) {
    std::string s = signature(ki, fn, 256);
    return s.substr(0, s.size() - 1) + sig_extra + ")";
  };

  // Pass 1: partial sums.
  Emitter p1;
  p1.set_nontemporal_loads(true);
  p1.set_streaming_ranges(ki.out_ranges);
  p1.line("const int tid = threadIdx.x;");
  p1.line("const int tx = tid % " + std::to_string(TX) + ", tr = tid / " + std::to_string(TX) + ";");
  p1.line("const long cb = blockIdx.x % " + std::to_string(per_f * other) + ";");
  p1.line("const int chunk = (int)(blockIdx.x / " + std::to_string(per_f * other) + ");");
  p1.line("const int fbase = (int)(cb % " + std::to_string(per_f) + ") * " + std::to_string(TX * V) + " + tx * " +
          std::to_string(V) + ";");
  p1.line("const long orest = cb / " + std::to_string(per_f) + ";");
  p1.line("const bool active = fbase < " + std::to_string(fext) + ";");
  p1.line("const int fcl = active ? fbase : 0;");
  p1.define_range(fast, "fcl");
  decode_outputs(p1, ki, "orest", fast);
  if (V == 4) p1.set_lane_range(fast, 4);
  std::vector<std::string> accs(V);
  for (int u = 0; u < V; u++) {
    accs[u] = "cacc" + std::to_string(u);
    p1.line(std::string(ctype(dt)) + " " + accs[u] + " = " + init_lit(rop, dt) + ";");
  }
  p1.line("const int r0 = chunk * " + std::to_string(CH) + ";");
  p1.line("const int r1 = r0 + " + std::to_string(CH) + " < " + std::to_string(L) + " ? r0 + " + std::to_string(CH) +
          " : " + std::to_string(L) + ";");
  p1.open_scope("if (active) {", "}");
  p1.line("#pragma unroll 8");
  p1.open_scope("for (int rr = r0 + tr; rr < r1; rr += " + std::to_string(TR) + ") {", "}");
  p1.define_range(r, "rr");
  for (int u = 0; u < V; u++) p1.line(accs[u] + " = " + combine(rop, accs[u], p1.val(R.src(0), u)) + ";");
  p1.close_scope();
  p1.close_scope();
  p1.line(std::string("__shared__ ") + ctype(dt) + " fg_col[" + std::to_string(TR) + "][" + std::to_string(TX * V) + "];");
  for (int u = 0; u < V; u++)
    p1.line("fg_col[tr][tx*" + std::to_string(V) + "+" + std::to_string(u) + "] = " + accs[u] + ";");
  p1.line("__syncthreads();");
  p1.line("if (tr == 0 && active) {");
  for (int u = 0; u < V; u++) {
    std::string slot = "fg_col[q][tx*" + std::to_string(V) + "+" + std::to_string(u) + "]";
    p1.line("  " + std::string(ctype(dt)) + " s" + std::to_string(u) + " = fg_col[0][tx*" + std::to_string(V) + "+" +
            std::to_string(u) + "];");
    p1.line("  for (int q = 1; q < " + std::to_string(TR) + "; q++) s" + std::to_string(u) + " = " +
            combine(rop, "s" + std::to_string(u), slot) + ";");
    std::string guard = (V == 1 || fext % 4 != 0) ? "if (fbase + " + std::to_string(u) + " < " + std::to_string(fext) + ") " : "";
    p1.line("  " + guard + "fg_scratch[(long)chunk * " + std::to_string(NOUT) + "L + orest * " + std::to_string(fext) +
            "L + fbase + " + std::to_string(u) + "] = s" + std::to_string(u) + ";");
  }
  p1.line("}");

  // Pass 2: one wave per group of V outputs. Lane l folds chunks l, l+64, ...
  // in order, then a fixed wave tree combines the lanes (deterministic); every
  // lane evaluates the epilogue and lane 0 stores. A thread per output folding
  // all chunks serially was latency-bound (15 us for 64 chunks of 4096 sums).
  Emitter p2;
  int64_t threads = NOUT / V;  // output groups, one wave each
  p2.line("const long gid = (long)blockIdx.x * 4 + (threadIdx.x >> 6);");
  p2.line("const int lane = threadIdx.x & 63;");
  p2.line("if (gid >= " + std::to_string(threads) + "L) return;");
  int64_t per = fext / V;
  p2.line("const int fbase = (int)(gid % " + std::to_string(per) + ") * " + std::to_string(V) + ";");
  p2.line("const long orest = gid / " + std::to_string(per) + ";");
  p2.define_range(fast, "fbase");
  decode_outputs(p2, ki, "orest", fast);
  if (V == 4) p2.set_lane_range(fast, 4);
  p2.reduce_cb_ = [&](const UOp& RR, int lane) -> std::string {
    FG_CHECK(RR == R, "column reduce renders exactly one reduction");
    std::string acc = "facc" + std::to_string(lane);
    std::string lin = "orest * " + std::to_string(fext) + "L + fbase + " + std::to_string(lane);
    p2.line(std::string(ctype(dt)) + " " + acc + " = " + init_lit(rop, dt) + ";");
    p2.line("for (int c = lane; c < " + std::to_string(nchunks) + "; c += 64) " + acc + " = " +
            combine(rop, acc, "fg_scratch[(long)c * " + std::to_string(NOUT) + "L + " + lin + "]") + ";");
    p2.line(wave_reduce(acc, 64, rop, dt));
    p2.remember_here(RR, lane, acc);
    return acc;
  };
  std::vector<std::string> vals;
  for (int u = 0; u < V; u++) vals.push_back(p2.val(ki.value, u));
  for (int u = 0; u < V; u++)
    p2.line("if (lane == 0) " + pname(ki.out_param) + "[" + p2.idx(ki.out_index, u) + "] = " + vals[u] + ";");

  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::ColumnReduce);
  rk.source = std::string(kPrelude) + sig(name + "_part") + " {\n" + p1.code() + "}\n" + sig(name + "_fin") + " {\n" +
              p2.code() + "}\n";
  LaunchSpec a, b;
  a.func = name + "_part";
  a.grid[0] = static_cast<unsigned>(per_f * other * nchunks);
  a.block[0] = 256;
  b.func = name + "_fin";
  b.grid[0] = static_cast<unsigned>((threads + 3) / 4);
  b.block[0] = 256;
  rk.launches = {a, b};
  rk.scratch_bytes = static_cast<size_t>(nchunks * NOUT) * dt.size_bytes();
  rk.grid[0] = a.grid[0];
  rk.block[0] = 256;
  return rk;
}

// Workgroups a split column reduction aims for: enough loads in flight to
// stream its rows. C5's bias gradients ([8192, 4096] summed over rows):
// 1024 workgroups of 128 rows took 25.0 us; a standalone sweep of the same
// pattern ran 2048 workgroups of 64 rows in 24.5 us against 32.8 with 1024.
constexpr int64_t kColChunkTarget = 2048;

RenderedKernel render_column_reduce(const KernelInfo& ki, const std::string& name) {
  const UOp& R = ki.reduces[0];
  Op rop = R.arg().rop;
  DType dt = R.dtype();
  const UOp r = R.src(1);
  int64_t L = range_extent(r);
  UOp fast = pick_fast_output(ki);
  int64_t fext = 1;
  for (size_t i = 0; i < ki.out_ranges.size(); i++)
    if (ki.out_ranges[i] == fast) fext = ki.out_ext[i];
  int V = fext % 4 == 0 ? 4 : 1;
  int TX = std::min<int64_t>(64, std::max<int64_t>(1, pow2_floor((fext + V - 1) / V)));
  int TR = 256 / TX;
  int64_t per_f = (fext + static_cast<int64_t>(TX) * V - 1) / (static_cast<int64_t>(TX) * V);  // blocks along fast
  int64_t other = total_outputs(ki) / fext;
  // Few output blocks cannot fill the chip: split the reduce range into
  // chunks reduced by separate workgroups into scratch, then combine the
  // chunks in a fixed order in a second pass (deterministic, no atomics).
  int64_t blocks = per_f * other;
  int64_t nchunks = 1;
  if (blocks < 512) {
    nchunks = std::min<int64_t>((kColChunkTarget + blocks - 1) / blocks, L / (4 * TR));
    nchunks = std::max<int64_t>(nchunks, 1);
  }
  if (nchunks > 1) return render_column_reduce_split(ki, name, V, TX, TR, per_f, other, fext, nchunks);
  Emitter em;
  em.set_nontemporal_loads(true);
  em.set_streaming_ranges(ki.out_ranges);
  em.line("const int tid = threadIdx.x;");
  em.line("const int tx = tid % " + std::to_string(TX) + ", tr = tid / " + std::to_string(TX) + ";");
  em.line("const int fbase = (int)(blockIdx.x % " + std::to_string(per_f) + ") * " + std::to_string(TX * V) + " + tx * " +
          std::to_string(V) + ";");
  em.line("const long orest = blockIdx.x / " + std::to_string(per_f) + ";");
  em.line("const bool active = fbase < " + std::to_string(fext) + ";");
  // Inactive threads still evaluate hoisted loads: clamp them in bounds.
  em.line("const int fcl = active ? fbase : 0;");
  em.define_range(fast, "fcl");
  decode_outputs(em, ki, "orest", fast);
  em.set_lane_base_aligned(true);
  if (V == 4) em.set_lane_range(fast, 4);
  std::vector<std::string> accs(V);
  em.reduce_cb_ = [&](const UOp& RR, int lane) -> std::string {
    FG_CHECK(RR == R, "column reduce renders exactly one reduction");
    if (lane == 0) {
      for (int u = 0; u < V; u++) {
        accs[u] = "cacc" + std::to_string(u);
        em.line(std::string(ctype(dt)) + " " + accs[u] + " = " + init_lit(rop, dt) + ";");
      }
      em.open_scope("if (active) for (int rr = tr; rr < " + std::to_string(L) + "; rr += " + std::to_string(TR) + ") {", "}");
      em.define_range(r, "rr");
      for (int u = 0; u < V; u++) em.line(accs[u] + " = " + combine(rop, accs[u], em.val(R.src(0), u)) + ";");
      em.close_scope();
      em.line(std::string("__shared__ ") + ctype(dt) + " fg_col[" + std::to_string(TR) + "][" + std::to_string(TX * V) + "];");
      for (int u = 0; u < V; u++)
        em.line("fg_col[tr][tx*" + std::to_string(V) + "+" + std::to_string(u) + "] = " + accs[u] + ";");
      em.line("__syncthreads();");
      em.line("if (tr == 0) {");
      for (int u = 0; u < V; u++) {
        em.line("  " + accs[u] + " = fg_col[0][tx*" + std::to_string(V) + "+" + std::to_string(u) + "];");
        em.line("  for (int q = 1; q < " + std::to_string(TR) + "; q++) " + accs[u] + " = " +
                combine(rop, accs[u], "fg_col[q][tx*" + std::to_string(V) + "+" + std::to_string(u) + "]") + ";");
      }
      em.line("}");
      for (int u = 0; u < V; u++) em.remember_here(RR, u, accs[u]);
    }
    return accs[lane];
  };
  std::vector<std::string> vals;
  for (int u = 0; u < V; u++) vals.push_back(em.val(ki.value, u));
  for (int u = 0; u < V; u++) {
    std::string guard = "active && tr == 0";
    if (V == 1 || fext % 4 != 0) guard += " && fbase + " + std::to_string(u) + " < " + std::to_string(fext);
    em.line("if (" + guard + ") " + pname(ki.out_param) + "[" + em.idx(ki.out_index, u) + "] = " + vals[u] + ";");
  }
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::ColumnReduce);
  rk.source = std::string(kPrelude) + signature(ki, name, 256) + " {\n" + em.code() + "}\n";
  rk.block[0] = 256;
  rk.grid[0] = static_cast<unsigned>(per_f * other);
  return rk;
}

// ── GEMM (fp32 MFMA) ────────────────────────────────────────────────────────
// One GEMM operand: an elementwise expression (a bare load, or e.g. the ReLU
// of a load that the reference leaves unmaterialised) over the reduce range
// and exactly one output range. Its tile loader evaluates the expression.
struct GemmOperand {
  UOp expr;
  UOp rout;     // the output range this operand varies with
  Affine lead;  // index of its first load that moves with the reduce range
};

struct GemmMatch {
  UOp R;              // the reduction
  UOp rm, rn, rk;     // output rows, output cols, reduce range
  int64_t M = 0, N = 0, K = 0;
  GemmOperand a, b;   // a pairs with rm, b with rn
};

bool gemm_operand(const UOp& e, const UOp& rk, const KernelInfo& ki, GemmOperand* op) {
  if (e.dtype() != DType::F32()) return false;
  auto lds = loads_in(e);
  if (lds.empty()) return false;
  UOp rout;
  bool have_lead = false;
  for (auto& n : e.toposort()) {
    if (n.op() == Op::Reduce) return false;
    if (n.op() == Op::Range && n != rk) {
      if (rout && rout != n) return false;
      rout = n;
    }
  }
  for (auto& ld : lds) {
    if (ld.src(0).src(0) == ki.out_param) return false;  // in-place tiles would race
    // Kernel-scalar terms (narrow() starts, schedule.rs:217-239) may appear:
    // staging only uses the range coefficients; vector loads need every
    // scalar coefficient to be a multiple of 4, like any other term.
    Affine a = affine_of(ld.src(0).src(1));
    if (!a.ok) return false;
    if (!have_lead && a.coef(rk) != 0) {
      op->lead = a;
      have_lead = true;
    }
  }
  if (!rout || !have_lead) return false;
  op->expr = e;
  op->rout = rout;
  return true;
}

// Workgroup tile of the fp32 MFMA GEMM and the number of K splits. Each wave
// owns a (BM/WGM) x (BN/WGN) block of 32x32 MFMA tiles: TM x TN of them.
struct GemmTile {
  int BM = 256, BN = 256, BK = 32, WGM = 2, WGN = 2;
  int64_t S = 1;   // K splits (partials summed by a second pass); with stream_k, the most segments of a tile
  int64_t KC = 0;  // K per split, a multiple of BK
  int nbuf = 2;    // LDS operand stages (3: the next stage's first fragments are read before the barrier)
  // Stream-K: G workgroups each run an equal share of the (tile, k-tile)
  // iterations, crossing tile boundaries; each tile's segments are partials
  // that the second pass sums in k order.
  bool stream_k = false;
  int64_t G = 0;
  int nt() const { return 64 * WGM * WGN; }
  int tm() const { return BM / WGM / 32; }
  int tn() const { return BN / WGN / 32; }
};

// A [k][row] operand stage interleaves the rows of a wave's T MFMA tiles so
// one LDS read gives a lane its operand of several tiles. The tiles are cut
// into chunks of 4, 2 or 1 (16-, 8- or 4-byte reads); in the chunk of s tiles
// that starts at tile f, row r of tile f + i sits at wave-block row
// 32f + s*r + i. T = 5 (a 160-wide wave block) is a chunk of 4 and one of 1.
struct KmChunk {
  int first, size;
};
std::vector<KmChunk> km_chunks(int T) {
  std::vector<KmChunk> out;
  for (int f = 0; f < T;) {
    const int rest = T - f, sz = rest >= 4 ? 4 : rest >= 2 ? 2 : 1;
    out.push_back({f, sz});
    f += sz;
  }
  return out;
}

constexpr int64_t kComputeUnits = 256;  // MI355X
constexpr int64_t kLdsPerCu = 163840;   // gfx950 LDS bytes per CU
constexpr int64_t kMinSplitK = 64;      // shortest K range a split workgroup runs

// Workgroups of a tile one CU holds at once: bounded by the LDS of the two
// double-buffered operand stages (rows padded by 4 floats) and by the
// accumulators (16 VGPRs per 32x32 tile, about 128 more for staging and
// addresses, 512 per SIMD lane).
int64_t gemm_tile_residency(const GemmTile& t) {
  const int64_t lds = t.nbuf * 4 * static_cast<int64_t>(t.BM + t.BN + 8) * (t.BK + 4);
  const int64_t waves_per_simd = std::max<int64_t>(1, 512 / (16 * t.tm() * t.tn() + 128));
  const int64_t by_waves = std::max<int64_t>(1, waves_per_simd * 4 / (t.WGM * t.WGN));
  return std::max<int64_t>(1, std::min(kLdsPerCu / lds, by_waves));
}

// Tile and K splits. Measured on MI355X (fp32, same box and run for each
// comparison):
// - MFMA-bound shapes: 256x256 with four 128x128 waves and BK 32 ran 4096^3 at
//   134.8-137.6 TFLOP/s (hipBLASLt 138.9-142.8), 256x128 and 128x256 at 129,
//   128x128 at 127. The shape, k-tile and split count are chosen by estimated time:
//   rounds of resident workgroups times the MFMA time of one tile's K range
//   (padding included, at each shape's measured efficiency), plus the traffic
//   of split-K partials; or, for stream-K, each workgroup's share of the
//   k-tiles plus one more epilogue. For dW1 of the C5 MLP (4096x784, K 8192)
//   that picks 256x160 tiles as stream-K (410 + 13 us in the train step), over
//   256x160 with 3 splits on 240 CUs (430 + 10 us) and 256x256 with 4 splits
//   (484 + 14 us).
// - A side of at most 32 (N = 10 classes): one operand is streamed once, so the
//   kernel is HBM-bound. BK 16 (less LDS, more resident workgroups) and splits
//   up to about two workgroups per CU: the 8192x10 (K 4096) forward took 59 us
//   with BK 32 and 8 splits, 45 with BK 16 and 16 splits.
// - K of at most 32: the kernel is one pass over its output and epilogue
//   operands. Small tiles put many workgroups' loads and stores in flight:
//   8192x4096 with K 10 (C5's dH2, relu mask) took 91 us with 256x256 tiles, 54
//   with 128x128, 50 with 64x64; in a later same-box run 53.5 with 64x64 (four
//   waves), 51.5 with 32x64 (two), 52-53 with 128x64, 58 with 64x128 and 32x32,
//   65 with 64x32.
// FG_GEMM_TILE="BM,BN,BK,WGM,WGN,S[,NBUF]" fixes the tile, split count (0:
// stream-K over the chip's CUs) and LDS stage count (2 or 3) of every
// GEMM in the process: a tuning override for measuring alternatives to the
// choice below on one box. Read once; a malformed value fails.
// Stream-K over `iters` (tile, k-tile) iterations, tile-major with `kt`
// k-tiles per tile, on G workgroups: workgroup w runs [w*iters/G,
// (w+1)*iters/G), so iteration x belongs to workgroup ((x+1)*G - 1)/iters.
// The most segments (workgroups) any tile is split into.
int64_t stream_k_segments(int64_t ntiles, int64_t kt, int64_t G) {
  const int64_t iters = ntiles * kt;
  auto owner = [&](int64_t x) { return ((x + 1) * G - 1) / iters; };
  int64_t most = 1;
  for (int64_t t = 0; t < ntiles; t++) most = std::max(most, owner(t * kt + kt - 1) - owner(t * kt) + 1);
  return most;
}

bool gemm_tile_override(GemmTile* t) {
  static const std::vector<int64_t> v = [] {
    std::vector<int64_t> out;
    const char* e = std::getenv("FG_GEMM_TILE");
    if (!e || !*e) return out;
    std::string s(e);
    size_t p = 0;
    while (p <= s.size()) {
      size_t q = s.find(',', p);
      std::string f = s.substr(p, q == std::string::npos ? std::string::npos : q - p);
      char* end = nullptr;
      long long x = std::strtoll(f.c_str(), &end, 10);
      FG_CHECK(!f.empty() && *end == '\0' && (x > 0 || (x == 0 && out.size() == 5)),
               "FG_GEMM_TILE must be BM,BN,BK,WGM,WGN,S[,NBUF] (S 0: stream-K); got '" + s + "'");
      out.push_back(x);
      if (q == std::string::npos) break;
      p = q + 1;
    }
    FG_CHECK(out.size() == 6 || (out.size() == 7 && (out[6] == 2 || out[6] == 3)),
             "FG_GEMM_TILE must be BM,BN,BK,WGM,WGN,S[,NBUF]; got '" + s + "'");
    return out;
  }();
  if (v.empty()) return false;
  t->BM = static_cast<int>(v[0]);
  t->BN = static_cast<int>(v[1]);
  t->BK = static_cast<int>(v[2]);
  t->WGM = static_cast<int>(v[3]);
  t->WGN = static_cast<int>(v[4]);
  t->S = v[5];
  if (v.size() == 7) t->nbuf = static_cast<int>(v[6]);
  return true;
}

GemmTile choose_gemm_tile(int64_t M, int64_t N, int64_t K) {
  auto tiles = [&](const GemmTile& t) { return ((M + t.BM - 1) / t.BM) * ((N + t.BN - 1) / t.BN); };
  const int64_t smax = std::max<int64_t>(1, K / kMinSplitK);
  auto with_splits = [&](GemmTile t, int64_t S) {
    t.KC = ((K + S - 1) / S + t.BK - 1) / t.BK * t.BK;
    t.S = (K + t.KC - 1) / t.KC;
    return t;
  };
  // Stream-K on every resident workgroup slot of the chip.
  auto as_stream_k = [&](GemmTile t) {
    const int64_t kt = (K + t.BK - 1) / t.BK;
    t.stream_k = true;
    t.G = kComputeUnits * gemm_tile_residency(t);
    t.S = stream_k_segments(tiles(t), kt, t.G);
    t.KC = t.BK;
    return t;
  };
  // Worth it when every workgroup runs at least 4 k-tiles and the shares do
  // not fall on whole tiles anyway.
  auto stream_k_fits = [&](const GemmTile& t) {
    const int64_t kt = (K + t.BK - 1) / t.BK, G = kComputeUnits * gemm_tile_residency(t), iters = tiles(t) * kt;
    return iters >= 4 * G && !(iters % G == 0 && (iters / G) % kt == 0);
  };
  GemmTile forced;
  if (gemm_tile_override(&forced)) {
    if (forced.S != 0) return with_splits(forced, forced.S);
    FG_CHECK(tiles(forced) * ((K + forced.BK - 1) / forced.BK) >= kComputeUnits * gemm_tile_residency(forced),
             "FG_GEMM_TILE: stream-K needs at least one k-tile per workgroup");
    return as_stream_k(forced);
  }
  if (M <= 32 || N <= 32) {
    GemmTile t;
    auto side = [](int64_t ext, int* b, int* w) {
      if (ext <= 32) { *b = 32; *w = 1; }
      else if (ext >= 256) { *b = 256; *w = 4; }
      else if (ext >= 128) { *b = 128; *w = 4; }
      else { *b = 64; *w = 2; }
    };
    side(M, &t.BM, &t.WGM);
    side(N, &t.BN, &t.WGN);
    t.BK = 16;
    const int64_t nt = tiles(t);
    return with_splits(t, std::max<int64_t>(1, std::min(smax, (2 * kComputeUnits + nt - 1) / nt)));
  }
  if (K <= 32) return with_splits(GemmTile{32, 64, K <= 16 ? 16 : 32, 1, 2}, 1);
  constexpr double kCuFlops = 157.3e12 / kComputeUnits;  // fp32 MFMA peak per CU
  constexpr double kHbmBytes = 5.0e12;                   // sustained HBM rate for split partials
  struct Cand {
    GemmTile t;
    double eff;  // measured throughput relative to 256x256
  };
  // Each shape with BK 32 and BK 16. BK 16 pads a K that is not a multiple of
  // 32 less: the 8192x4096 forward with K 784 (49 k-tiles of 16) took 399 us
  // against 424 us with BK 32; for K 4096 BK 32 was about 2% faster.
  // 256x160 (four waves of 64x160 stacked along M, five 32-wide MFMA columns
  // each) pads a 784-wide side to 800 columns instead of 1024. C5's dW1
  // (4096x784, K 8192), timed alone: 472 us with 3 splits (240 workgroups)
  // against 526 us as 256x256 with 4; with BK 16 (two or three stages) 548 us.
  const Cand cands[] = {{{256, 256, 32, 2, 2}, 1.0},   {{256, 256, 16, 2, 2}, 0.99}, {{256, 128, 32, 2, 2}, 0.9},
                        {{256, 128, 16, 2, 2}, 0.89},  {{128, 256, 32, 2, 2}, 0.9},  {{128, 256, 16, 2, 2}, 0.89},
                        {{128, 128, 32, 2, 2}, 0.92},  {{128, 128, 16, 2, 2}, 0.91}, {{64, 64, 32, 2, 2}, 0.6},
                        {{256, 160, 32, 4, 1}, 0.97},  {{256, 160, 16, 4, 1}, 0.84}, {{160, 256, 32, 1, 4}, 0.97},
                        {{160, 256, 16, 1, 4}, 0.84}};
  GemmTile best = with_splits(GemmTile{64, 64, 32, 2, 2}, 1);
  double best_s = 1e30;
  for (const Cand& c : cands) {
    if (M < c.t.BM / 2 || N < c.t.BN / 2) continue;  // mostly padding
    const int64_t nt = tiles(c.t), res = gemm_tile_residency(c.t);
    for (int64_t s = 1; s <= smax; s++) {
      const GemmTile t = with_splits(c.t, s);
      if (t.S != s) continue;
      const int64_t rounds = (nt * t.S + kComputeUnits * res - 1) / (kComputeUnits * res);
      const double mfma = static_cast<double>(rounds * res) * 2.0 * t.BM * t.BN * t.KC / (kCuFlops * c.eff);
      const double partials = t.S > 1 ? static_cast<double>(t.S + 1) * M * N * 4.0 / kHbmBytes : 0.0;
      if (mfma + partials < best_s * 0.999) {
        best_s = mfma + partials;
        best = t;
      }
    }
    if (stream_k_fits(c.t)) {
      // Each workgroup's share of the k-tiles, plus one more epilogue when it
      // crosses into a second tile, plus the segments' partials.
      const GemmTile t = as_stream_k(c.t);
      const int64_t kt = (K + t.BK - 1) / t.BK, share = (nt * kt + t.G - 1) / t.G;
      const double mfma = static_cast<double>(share + 1) * res * 2.0 * t.BM * t.BN * t.BK / (kCuFlops * c.eff);
      const double partials = static_cast<double>(t.S + 1) * M * N * 4.0 / kHbmBytes;
      if (mfma + partials < best_s * 0.98) {
        best_s = mfma + partials;
        best = t;
      }
    }
  }
  // A 16-wide k-tile runs with three LDS stages where they fit without costing
  // a resident workgroup: its k-tiles are half as long, so the read of the next
  // stage's first fragments after each barrier weighed twice as much. Measured
  // on the 8192x4096 forward with K 784: 455-462 us against 463-464 us with two
  // stages; 4096^3 with BK 16: 1054 against 1071 us (BK 32, two stages: 1034).
  if (best.BK == 16) {
    GemmTile t3 = best;
    t3.nbuf = 3;
    const int64_t lds3 = 3 * 4 * static_cast<int64_t>(t3.BM + t3.BN + 8) * (t3.BK + 4);
    if (lds3 <= kLdsPerCu && gemm_tile_residency(t3) == gemm_tile_residency(best)) best = t3;
  }
  return best;
}

constexpr int64_t kSmallGemmMaxWork = int64_t(1) << 26;  // M*N*K
constexpr int kSmallGemmMaxGroups = 4;                   // 16-k groups per wave

bool small_gemm_fits(int64_t M, int64_t N, int64_t K) {
  GemmTile forced;
  if (gemm_tile_override(&forced)) return false;
  return M * N * K <= kSmallGemmMaxWork;
}

// Waves per workgroup: enough that no wave folds more than G groups of 16 k
// (kSmallGemmMaxGroups; FG_SMALL_GEMM_GROUPS overrides it for tuning, read
// once), at most 16 (1024 threads).
int small_gemm_waves(int64_t K) {
  static const int64_t G = [] {
    const char* e = std::getenv("FG_SMALL_GEMM_GROUPS");
    if (!e || !*e) return static_cast<int64_t>(kSmallGemmMaxGroups);
    char* end = nullptr;
    const long v = std::strtol(e, &end, 10);
    FG_CHECK(*end == '\0' && v >= 1 && v <= 64, std::string("FG_SMALL_GEMM_GROUPS must be 1 to 64; got '") + e + "'");
    return static_cast<int64_t>(v);
  }();
  const int64_t kg = (K + 15) / 16;
  return static_cast<int>(std::min<int64_t>(16, std::max<int64_t>(1, (kg + G - 1) / G)));
}

bool match_gemm(const KernelInfo& ki, GemmMatch* g) {
  if (ki.reduces.size() != 1 || ki.out_ranges.size() != 2) return false;
  const UOp& R = ki.reduces[0];
  if (R.arg().rop != Op::Add || R.srcs().size() != 2 || R.dtype() != DType::F32()) return false;
  const UOp& v = R.src(0);
  if (v.op() != Op::Mul) return false;
  const UOp& rk = R.src(1);
  GemmOperand x, y;
  if (!gemm_operand(v.src(0), rk, ki, &x) || !gemm_operand(v.src(1), rk, ki, &y)) return false;
  if (x.rout == y.rout) return false;
  Affine ao = affine_of(ki.out_index);
  if (!ao.ok) return false;
  // Tile columns follow the output range with the smaller store stride so
  // epilogue stores coalesce.
  int64_t cx = std::llabs(ao.coef(x.rout)), cy = std::llabs(ao.coef(y.rout));
  bool swap = cx < cy;
  g->R = R;
  g->rk = rk;
  g->a = swap ? y : x;
  g->b = swap ? x : y;
  g->rm = g->a.rout;
  g->rn = g->b.rout;
  g->M = range_extent(g->rm);
  g->N = range_extent(g->rn);
  g->K = range_extent(rk);
  if (std::min(g->M, g->N) < 8 || g->M * g->N * g->K < (1LL << 18)) return false;
  if (small_gemm_fits(g->M, g->N, g->K)) return true;
  if (g->M <= 32 || g->N <= 32) {
    // A narrow product pays for a 32-wide MFMA tile only when the grid fills
    // the chip; otherwise the row and column reductions serve it better.
    GemmTile t = choose_gemm_tile(g->M, g->N, g->K);
    if (((g->M + t.BM - 1) / t.BM) * ((g->N + t.BN - 1) / t.BN) * t.S < 128) return false;
  }
  return true;
}

// ── Small GEMM: one pass, the K range split over the waves of a workgroup ──
// A product too small to fill the chip with whole tiles (an MLP's 784->128
// layer at batch 256: 256x128, K 784) otherwise runs split-K: a partial pass
// plus a finishing pass, two launches of a few microseconds each, most of it
// launch and memory latency. Here each workgroup owns one 16x16 output tile
// (v_mfma_f32_16x16x4f32) and its W waves each fold a contiguous share of the
// K range, in groups of 16 k (four MFMAs: in step u, lane l supplies k =
// 16g + 4*(l/16) + u of row l%16, the same k for both operands, so a
// k-contiguous operand's four steps are one lane's four consecutive floats).
// A wave first loads all of its operands, evaluating the operand expressions
// (relu masks, transposed views) on them, then runs its MFMAs. The W partial
// tiles meet in LDS and are summed in wave order by one thread per output,
// which then runs the epilogue (bias, relu mask, SGD update). One launch, no
// scratch, a fixed fold order.
std::string block_params(const KernelInfo& ki, std::vector<std::string>* types, std::vector<std::string>* names);

RenderedKernel render_small_gemm(const KernelInfo& ki, const GemmMatch& g, const std::string& name) {
  const int64_t M = g.M, N = g.N, K = g.K;
  const int64_t KG = (K + 15) / 16, ntm = (M + 15) / 16, ntn = (N + 15) / 16;
  const int W = small_gemm_waves(K);
  const int64_t GMAX = (KG + W - 1) / W;  // groups the busiest wave folds
  // Groups loaded together: at most kSmallGemmMaxGroups, so a long K range
  // (the waves are at most 16) runs as a rolled loop of such chunks instead
  // of holding all of its operands in registers.
  const int64_t CH = std::min<int64_t>(GMAX, kSmallGemmMaxGroups);
  const bool chunked = CH < GMAX;
  const int NT = 64 * W;
  std::ostringstream s;
  // The kernel's body as a device function of its block index (fg_bid), so a
  // launch may also run it beside another kernel (render_hfused).
  std::vector<std::string> types, names;
  const std::string params = block_params(ki, &types, &names);
  s << "__device__ __forceinline__ void " << name << "_hb(" << params << ", unsigned fg_bid) {\n";
  s << "  __shared__ float fg_part[" << W << "][256];\n";
  s << "  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, r16 = lane & 15;\n";
  s << "  const int tm = (int)(fg_bid / " << ntn << "), tn = (int)(fg_bid % " << ntn << ");\n";
  s << "  const int m0 = tm * 16, n0 = tn * 16;\n";
  // This wave's groups of 16 k: [gbeg, gend).
  s << "  const int gbeg = (int)(((long)wave * " << KG << ") / " << W << "), gend = (int)(((long)(wave + 1) * " << KG
    << ") / " << W << ");\n";
  s << "  const int am = m0 + r16 < " << M << " ? m0 + r16 : " << (M - 1) << ";\n";
  s << "  const int bn = n0 + r16 < " << N << " ? n0 + r16 : " << (N - 1) << ";\n";
  s << "  const bool arow = m0 + r16 < " << M << ", brow = n0 + r16 < " << N << ";\n";
  s << "  fg_f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};\n";
  if (chunked) s << "  #pragma unroll 1\n  for (int c0 = 0; c0 < " << GMAX << "; c0 += " << CH << ") {\n";
  else s << "  {\n  constexpr int c0 = 0;\n";
  s << "  float av[" << CH << "][4], bv[" << CH << "][4];\n";
  // Loads of every group of the chunk first (all in flight together), then
  // the MFMAs.
  Emitter em;
  em.define_range(g.a.rout, "am");
  em.define_range(g.b.rout, "bn");
  em.open_scope("#pragma unroll\nfor (int gi = 0; gi < " + std::to_string(CH) + "; gi++) {", "}");
  em.line("const int kb = (gbeg + c0 + gi) * 16 + 4 * q;");
  em.line("const bool gin = gbeg + c0 + gi < gend;");
  if (K % 4 == 0) {
    // A lane's four k are all in range or all out: one clamped base, and the
    // four steps as lanes of that base (16-byte loads where k is unit-stride).
    em.line("const bool kin = gin && kb < " + std::to_string(K) + ";");
    em.line("const int kc = kin ? kb : 0;");
    em.define_range(g.rk, "kc");
    em.set_lane_range(g.rk, 4);
    for (int u = 0; u < 4; u++) {
      const std::string a = em.val(g.a.expr, u), b = em.val(g.b.expr, u);
      em.line("av[gi][" + std::to_string(u) + "] = (kin && arow) ? " + a + " : 0.0f;");
      em.line("bv[gi][" + std::to_string(u) + "] = (kin && brow) ? " + b + " : 0.0f;");
    }
    em.clear_lane_range();
  } else {
    for (int u = 0; u < 4; u++) {
      em.open_scope("{", "}");
      em.line("const bool kin = gin && kb + " + std::to_string(u) + " < " + std::to_string(K) + ";");
      em.line("const int kc = kin ? kb + " + std::to_string(u) + " : 0;");
      em.define_range(g.rk, "kc");
      const std::string a = em.val(g.a.expr, 0), b = em.val(g.b.expr, 0);
      em.line("av[gi][" + std::to_string(u) + "] = (kin && arow) ? " + a + " : 0.0f;");
      em.line("bv[gi][" + std::to_string(u) + "] = (kin && brow) ? " + b + " : 0.0f;");
      em.close_scope();
    }
  }
  em.close_scope();
  s << em.code();
  s << "  #pragma unroll\n"
       "  for (int gi = 0; gi < " << CH << "; gi++)\n"
       "    #pragma unroll\n"
       "    for (int u = 0; u < 4; u++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[gi][u], bv[gi][u], acc, 0, 0, 0);\n"
       "  }\n"
       "  // D[4*(lane/16) + e][lane%16] = acc[e]\n"
       "  #pragma unroll\n"
       "  for (int e = 0; e < 4; e++) fg_part[wave][(4 * q + e) * 16 + r16] = acc[e];\n"
       "  __syncthreads();\n"
       "  for (int o = tid; o < 256; o += " << NT << ") {\n"
       "  float sum = fg_part[0][o];\n"
       "  #pragma unroll\n"
       "  for (int w = 1; w < " << W << "; w++) sum = sum + fg_part[w][o];\n"
       "  const int grow = m0 + (o >> 4), gcol = n0 + (o & 15);\n"
       "  if (grow < " << M << " && gcol < " << N << ") {\n";
  {
    Emitter ep;
    ep.define_range(g.rm, "grow");
    ep.define_range(g.rn, "gcol");
    ep.reduce_cb_ = [&](const UOp& RR, int) -> std::string {
      FG_CHECK(RR == g.R, "gemm epilogue sees one reduction");
      return "sum";
    };
    std::string v = ep.val(ki.value, 0);
    ep.line(pname(ki.out_param) + "[" + ep.idx(ki.out_index, 0) + "] = " + v + ";");
    s << ep.code();
  }
  s << "  }\n  }\n}\n";
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::Gemm);
  rk.hbody_fn = name + "_hb";
  rk.hbody_src = s.str();
  rk.hbody_types = types;
  std::string call = rk.hbody_fn + "(";
  for (auto& n : names) call += n + ", ";
  rk.source = std::string(kPrelude) + rk.hbody_src + signature(ki, name, NT) + " {\n  " + call + "blockIdx.x);\n}\n";
  rk.block[0] = static_cast<unsigned>(NT);
  rk.grid[0] = static_cast<unsigned>(ntm * ntn);
  return rk;
}

// Helpers of the generated GEMM: vector types for 1/2/4 operands per LDS read
// and the instruction interleave of one k-tile (sched_group_barrier masks:
// 0x008 MFMA, 0x020 VMEM read, 0x100 DS read, 0x200 DS write). Group g's MFMAs
// are paired one to one with the global loads of the next stage (group 0), the
// LDS reads of group g+1, and the LDS writes of the next stage (last group), so
// those instructions issue while the MFMA pipe is busy.
const char* kGemmPrelude = R"(typedef float fg_f2 __attribute__((ext_vector_type(2)));
template <int V> struct fg_vt;
template <> struct fg_vt<1> { typedef float t; };
template <> struct fg_vt<2> { typedef fg_f2 t; };
template <> struct fg_vt<4> { typedef fg_f4 t; };
template <int mask, int n>
__device__ __forceinline__ void fg_sched_pairs() {
  if constexpr (n > 0) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(mask, 1, 0);
    fg_sched_pairs<mask, n - 1>();
  }
}
template <int G, int g, int NV, int ND, int NW, int MF>
__device__ __forceinline__ void fg_sched_k_tile() {
  constexpr int nv = g == 0 ? NV : 0, nd = g + 1 < G ? ND : 0, nw = g == G - 1 ? NW : 0;
  constexpr int rest = MF - nv - nd - nw;
  fg_sched_pairs<0x020, nv>();
  fg_sched_pairs<0x100, nd>();
  fg_sched_pairs<0x200, nw>();
  if constexpr (rest > 0) __builtin_amdgcn_sched_group_barrier(0x008, rest, 0);
  if constexpr (g + 1 < G) fg_sched_k_tile<G, g + 1, NV, ND, NW, MF>();
}
)";

// The k loop with three LDS operand stages instead of two: the stage after
// next is written while a stage is computed, so the next stage was complete
// at the previous barrier and its first fragments are read during the last
// group's MFMAs, before the barrier, instead of after it. One barrier per
// k-tile still orders every write after the reads of the stage it replaces
// (read during the k-tile before the last barrier) and before its own reads
// (after the next barrier). Needs an even number of 8-k groups per k-tile, so
// the fragment registers of the next k-tile's first group are free.
std::string gemm_three_stages(std::string src) {
  auto swap_once = [&](const std::string& from, const std::string& to) {
    const size_t p = src.find(from);
    FG_CHECK(p != std::string::npos && src.find(from, p + 1) == std::string::npos,
             "three-stage GEMM: generated text not found once");
    src.replace(p, from.size(), to);
  };
  swap_once("  // Operand stages, double-buffered, rows padded by 4 floats;",
            "  // Operand stages, three of them, rows padded by 4 floats;");
  swap_once("constexpr int SA = 2 * SA_R * SA_C, SB = 2 * SB_R * SB_C,",
            "constexpr int SA = 3 * SA_R * SA_C, SB = 3 * SB_R * SB_C,");
  swap_once("__device__ __forceinline__ void fg_sched_k_tile() {\n"
            "  constexpr int nv = g == 0 ? NV : 0, nd = g + 1 < G ? ND : 0, nw = g == G - 1 ? NW : 0;",
            "__device__ __forceinline__ void fg_sched_k_tile() {\n"
            "  constexpr int nv = g == 0 ? NV : 0, nd = ND, nw = g == G - 1 ? NW : 0;");
  swap_once(R"(  load_a(kbeg); load_b(kbeg);
  store_a(0, kbeg); store_b(0, kbeg);
  __syncthreads();
  frag(0, 0, fa[0], fb[0]);
  for (int kt = 0; kt < KT; kt++) {
    const int cur = kt & 1;
    // The last k-tile reloads itself, so the body is the same every time.
    const int knext = kbeg + (kt + 1 < KT ? kt + 1 : kt) * BK;
    load_a(knext); load_b(knext);
    #pragma unroll
    for (int g = 0; g < BK / 8; g++) {
      if (g + 1 < BK / 8) frag(cur, g + 1, fa[(g + 1) & 1], fb[(g + 1) & 1]);
)",
            R"(  static_assert((BK / 8) % 2 == 0, "three stages need an even number of 8-k groups");
  load_a(kbeg); load_b(kbeg);
  store_a(0, kbeg); store_b(0, kbeg);
  {
    const int k1 = kbeg + (1 < KT ? 1 : 0) * BK;
    load_a(k1); load_b(k1);
    store_a(1, k1); store_b(1, k1);
  }
  __syncthreads();
  frag(0, 0, fa[0], fb[0]);
  int cur = 0;
  for (int kt = 0; kt < KT; kt++) {
    const int nxt = cur == 2 ? 0 : cur + 1, nn = nxt == 2 ? 0 : nxt + 1;
    // The last k-tiles reload the last one, so the body is the same every time.
    const int knext = kbeg + (kt + 2 < KT ? kt + 2 : KT - 1) * BK;
    load_a(knext); load_b(knext);
    #pragma unroll
    for (int g = 0; g < BK / 8; g++) {
      if (g + 1 < BK / 8) frag(cur, g + 1, fa[(g + 1) & 1], fb[(g + 1) & 1]);
      else frag(nxt, 0, fa[0], fb[0]);
)");
  swap_once(R"(      if (g == BK / 8 - 1) { store_a(cur ^ 1, knext); store_b(cur ^ 1, knext); }
    }
    fg_sched_k_tile<BK / 8, 0, NV_, ND_, NW_, 4 * TM * TN>();
    __syncthreads();
    frag(cur ^ 1, 0, fa[0], fb[0]);
  }
)",
            R"(      if (g == BK / 8 - 1) { store_a(nn, knext); store_b(nn, knext); }
    }
    fg_sched_k_tile<BK / 8, 0, NV_, ND_, NW_, 4 * TM * TN>();
    __syncthreads();
    cur = nxt;
  }
)");
  return src;
}

// The main pass as stream-K: instead of one (split, tile) pair per
// workgroup, each of the G workgroups runs its share of the (tile, k-tile)
// iterations as segments of consecutive k-tiles of one tile, computing and
// storing each segment's partial sums as a split-K workgroup would. Shares
// differ by at most one k-tile, so no CU is left without work when the tiles
// do not divide into rounds.
//
// Tile order (D > 0): with equal shares, workgroups P apart (P the smallest
// multiple of the 8 XCDs with P * share a whole number of tiles' k-tiles)
// start at the same k position D = P * share / KTT tiles apart, and
// round-robin dispatch puts them on one XCD. Block index c + D*j is numbered
// c * NTILES/D + j in row-major order (column blocks fastest), so the tiles
// that one XCD's workgroups run at the same k are a few row blocks by every
// column block, and share their operand rows in that XCD's L2. D = 0 keeps
// the grouped order.
std::string gemm_stream_k(std::string src, int64_t D) {
  const std::string from = R"(  int bid = blockIdx.x;
  // Blocks are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous run of (split, tile) pairs so neighbouring tiles of one K
  // range share its L2.
  if ((NTILES_ * S_) % 8 == 0) bid = (bid % 8) * (NTILES_ * S_ / 8) + bid / 8;
#if S_ > 1
  const int ks = bid / NTILES_;
  bid = bid % NTILES_;
  const int kbeg = ks * KC_, kend = (kbeg + KC_ < K_) ? kbeg + KC_ : K_;
#else
  constexpr int kbeg = 0, kend = K_;
#endif
)";
  const std::string to = R"(  // Shares in launch order, so consecutive shares (neighbouring k-ranges
  // of one tile) run on different XCDs. Gathering them on one XCD fetched
  // 1028 MB from beyond L2 for C5's dW1 (800 in launch order with the
  // grouped tile order) and was no faster.
  const int wv = blockIdx.x;
  const long it_end = (long)(wv + 1) * ITERS_ / G_;
  for (long it = (long)wv * ITERS_ / G_; it < it_end;) {
  int bid = (int)(it / KTT_);
  const int kt0 = (int)(it % KTT_);
  const int kt1 = (it_end - it < (long)(KTT_ - kt0)) ? kt0 + (int)(it_end - it) : KTT_;
  it += kt1 - kt0;
  const int ks = wv - fg_sk_owner((long)bid * KTT_);  // the segment's place in its tile, in k order
  const int kbeg = kt0 * BK, kend = (kt1 * BK < K_) ? kt1 * BK : K_;
)";
  const size_t p = src.find(from);
  FG_CHECK(p != std::string::npos && src.find(from, p + 1) == std::string::npos,
           "stream-K GEMM: generated text not found once");
  src.replace(p, from.size(), to);
  if (D > 0) {
    const std::string grouped = R"(  const int GM = 8;
  const int group = bid / (GM * nbn), first_m = group * GM;
  const int gsz = (nbm - first_m) < GM ? (nbm - first_m) : GM;
  const int tm = first_m + (bid % (GM * nbn)) % gsz, tn = (bid % (GM * nbn)) / gsz;
)";
    const std::string by_xcd = R"(  const int sq = (bid % SK_D_) * (NTILES_ / SK_D_) + bid / SK_D_;  // the block's row-major slot
  const int tm = sq / nbn, tn = sq % nbn;
)";
    const size_t q = src.find(grouped);
    FG_CHECK(q != std::string::npos && src.find(grouped, q + 1) == std::string::npos,
             "stream-K GEMM: tile order text not found once");
    src.replace(q, grouped.size(), by_xcd);
  }
  return src;
}

// The stream-K tile order's D (see gemm_stream_k), or 0 when the shares are
// unequal or no such period divides the tiles.
int64_t stream_k_tile_period(int64_t ntiles, int64_t kt, int64_t G) {
  const int64_t iters = ntiles * kt;
  if (iters % G != 0) return 0;
  const int64_t share = iters / G;
  for (int64_t P = 8; P <= G; P += 8)
    if ((P * share) % kt == 0) {
      const int64_t D = P * share / kt;
      return ntiles % D == 0 ? D : 0;
    }
  return 0;
}

RenderedKernel render_gemm(const KernelInfo& ki, const GemmMatch& g, const std::string& name) {
  if (small_gemm_fits(g.M, g.N, g.K)) return render_small_gemm(ki, g, name);
  const int64_t M = g.M, N = g.N, K = g.K;
  const GemmTile tile = choose_gemm_tile(M, N, K);
  const int BM = tile.BM, BN = tile.BN, BK = tile.BK, WGM = tile.WGM, WGN = tile.WGN, NT = tile.nt();
  const int TM = tile.tm(), TN = tile.tn();
  const int64_t S = tile.S, KC = tile.KC, NP = (N + 3) / 4 * 4;
  const int64_t ntiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  FG_CHECK(BM % (32 * WGM) == 0 && BN % (32 * WGN) == 0 && BK % 8 == 0, "gemm tile shape does not fit the wave grid");
  FG_CHECK(TM >= 1 && TM <= 5 && TN >= 1 && TN <= 5, "gemm wave tile must be 32 to 160 wide");
  FG_CHECK(tile.nbuf == 2 || (tile.nbuf == 3 && (BK / 8) % 2 == 0), "three GEMM stages need an even number of 8-k groups");
  const bool split = S > 1 || tile.stream_k;  // partials in scratch, summed by _fin
  const int64_t KTT = (K + BK - 1) / BK;       // k-tiles per tile
  const int64_t sk_D = tile.stream_k ? stream_k_tile_period(ntiles, KTT, tile.G) : 0;
  const std::string scratch_param = split ? ", float* __restrict__ fg_scratch" : "";
  const int waves_per_eu = static_cast<int>(std::max<int64_t>(1, gemm_tile_residency(tile) * NT / 256));
  auto sig = [&](const std::string& fn, int block, bool main) {
    std::string s = signature(ki, fn, block);
    s = s.substr(0, s.size() - 1) + scratch_param + ")";
    if (main) {
      const std::string lb = "__launch_bounds__(" + std::to_string(block) + ") ";
      s.replace(s.find(lb), lb.size(),
                lb + "__attribute__((amdgpu_waves_per_eu(" + std::to_string(waves_per_eu) + "))) ");
    }
    return s;
  };
  const std::string main_name = split ? name + "_part" : name;

  // How each operand reaches LDS. Mode 0: 4 consecutive k per thread (unit
  // stride along k: 16-byte loads), staged [row][k]. Mode 1: 4 consecutive rows
  // per thread (unit stride along m/n), staged [k][row] with the rows of tile i
  // interleaved (tile i row r is wave row T*r+i), so one LDS read gives a lane
  // its operand for all T tiles. Mode 2: one element per load, staged along
  // whichever index moves faster in memory.
  struct Stage {
    int md = 2;
    bool km = false;
    int groups = 0, per = 0, V = 1;
    bool k_fast = true;
    std::vector<UOp> lds;
  };
  auto plan = [&](const GemmOperand& op, int BX, int64_t ext) {
    Stage st;
    const int64_t so = op.lead.coef(op.rout), sk = op.lead.coef(g.rk);
    if (sk == 1 && K % 4 == 0) st.md = 0;
    else if (so == 1 && ext % 4 == 0) st.md = 1;
    st.k_fast = std::llabs(sk) <= std::llabs(so);
    st.km = st.md == 1 || (st.md == 2 && !st.k_fast);
    st.V = st.md == 2 ? 1 : 4;
    st.groups = st.md == 2 ? BX * BK : BX * BK / 4;
    st.per = (st.groups + NT - 1) / NT;
    st.lds = loads_in(op.expr);
    return st;
  };
  const Stage sa = plan(g.a, BM, M), sb = plan(g.b, BN, N);
  const int NV = sa.per * static_cast<int>(sa.lds.size()) + sb.per * static_cast<int>(sb.lds.size());
  const int ND = (sa.km ? 4 * static_cast<int>(km_chunks(TM).size()) : TM) +
                 (sb.km ? 4 * static_cast<int>(km_chunks(TN).size()) : TN);
  const int NW = sa.per + sb.per;

  std::ostringstream s;
  s << kPrelude << kGemmPrelude;
  s << "#define M_ " << M << "\n#define N_ " << N << "\n#define K_ " << K << "\n#define NP_ " << NP << "\n";
  s << "#define S_ " << S << "\n#define KC_ " << KC << "\n#define NTILES_ " << ntiles << "\n";
  s << "#define BM " << BM << "\n#define BN " << BN << "\n#define BK " << BK << "\n";
  s << "#define NT " << NT << "\n#define WGN " << WGN << "\n#define TM " << TM << "\n#define TN " << TN << "\n";
  s << "#define A_KM " << (sa.km ? 1 : 0) << "\n#define B_KM " << (sb.km ? 1 : 0) << "\n";
  s << "#define NV_ " << NV << "\n#define ND_ " << ND << "\n#define NW_ " << NW << "\n";
  if (tile.stream_k) {
    s << "#define G_ " << tile.G << "\n#define KTT_ " << KTT << "\n#define ITERS_ " << ntiles * KTT << "L\n";
    if (sk_D > 0) s << "#define SK_D_ " << sk_D << "\n";
    s << "// Stream-K: the workgroup that runs (tile, k-tile) iteration x.\n"
         "__device__ __forceinline__ int fg_sk_owner(long x) { return (int)(((x + 1) * G_ - 1) / ITERS_); }\n";
  }
  s << sig(main_name, NT, true) << " {\n";
  s << R"(  // Operand stages, double-buffered, rows padded by 4 floats; then per-wave
  // 32 x WN staging tiles for the epilogue.
  constexpr int WM = BM / (NT / 64 / WGN), WN = BN / WGN;
  // A [row][k] stage of 16-wide k-tiles is unpadded, its 16-byte chunks
  // XOR-swizzled by row: chunk c of row r sits at c ^ ((r >> 2) & 3). The 16
  // lanes a fragment read serves at once (16 rows, one chunk, over 64 banks)
  // and the 8 lanes of a stage write (two rows, over 32) then fall on distinct
  // banks: PMC SQ_LDS_BANK_CONFLICT 0 for C5's K = 784 forward, against
  // 6.5e6 cycles per dispatch with rows padded to 20 floats (which put two
  // rows' writes on the same banks) and with c ^ ((r >> 1) & 3) (which put
  // rows r and r + 8 of a read on the same banks).
#define FG_SWZ(r, c) (BK == 16 ? ((c) ^ ((((r) >> 2) & 3) << 2)) : (c))
#if A_KM
  constexpr int SA_R = BK, SA_C = BM + 4;
#else
  constexpr int SA_R = BM, SA_C = BK == 16 ? BK : BK + 4;
#endif
#if B_KM
  constexpr int SB_R = BK, SB_C = BN + 4;
#else
  constexpr int SB_R = BN, SB_C = BK == 16 ? BK : BK + 4;
#endif
  constexpr int SA = 2 * SA_R * SA_C, SB = 2 * SB_R * SB_C, EPS = WN + 4, SE = (NT / 64) * 32 * EPS;
  __shared__ __attribute__((aligned(16))) float smem[(SA + SB) > SE ? (SA + SB) : SE];
  float (*As)[SA_R][SA_C] = reinterpret_cast<float (*)[SA_R][SA_C]>(smem);
  float (*Bs)[SB_R][SB_C] = reinterpret_cast<float (*)[SB_R][SB_C]>(smem + SA);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5, r32 = lane & 31;
  const int nbm = (M_ + BM - 1) / BM, nbn = (N_ + BN - 1) / BN;
  int bid = blockIdx.x;
  // Blocks are dispatched round-robin over the 8 XCDs; give each XCD a
  // contiguous run of (split, tile) pairs so neighbouring tiles of one K
  // range share its L2.
  if ((NTILES_ * S_) % 8 == 0) bid = (bid % 8) * (NTILES_ * S_ / 8) + bid / 8;
#if S_ > 1
  const int ks = bid / NTILES_;
  bid = bid % NTILES_;
  const int kbeg = ks * KC_, kend = (kbeg + KC_ < K_) ? kbeg + KC_ : K_;
#else
  constexpr int kbeg = 0, kend = K_;
#endif
  const int GM = 8;
  const int group = bid / (GM * nbn), first_m = group * GM;
  const int gsz = (nbm - first_m) < GM ? (nbm - first_m) : GM;
  const int tm = first_m + (bid % (GM * nbn)) % gsz, tn = (bid % (GM * nbn)) / gsz;
  const int m0 = tm * BM, n0 = tn * BN;
  const int wm = (wave / WGN) * WM, wn = (wave % WGN) * WN;
  floatx16 acc[TM][TN];
  #pragma unroll
  for (int i = 0; i < TM; i++)
    #pragma unroll
    for (int j = 0; j < TN; j++)
      #pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
)";
  // Global -> register loaders. load_X issues the operand's raw loads; store_X
  // evaluates the operand expression (relu recompute, masks) on them when it
  // writes the next stage to LDS, late in the k-tile, so the loads stay in
  // flight under the MFMAs. Out-of-range elements load from a clamped, valid
  // address and are replaced by 0 with a select: the k-tile body has no
  // branches, so its instructions can be interleaved as one region.
  std::set<std::string> rsrc_declared;
  auto loader = [&](const char* X, const GemmOperand& op, const Stage& st, int BX, int64_t ext, const char* dim) {
    const int V = st.V, per = st.per;
    const bool guard = st.groups % NT != 0;
    // Bounds checks only where a tile can overhang: rows when the extent is not
    // a multiple of the tile, k when K is not a multiple of BK (the K splits
    // are multiples of BK). Statically in-range loads keep their plain
    // addresses, which saves registers in the large tiles.
    const bool row_check = ext % BX != 0, k_check = K % BK != 0;
    // Raw buffer loads where every load of the operand allows them: a 32-bit
    // byte offset per lane that is the same in every k-tile, and the k-tile's
    // start in the scalar offset, so the k loop computes no addresses and
    // holds one register per load instead of a 64-bit address. Each load must
    // read a 4-byte element of a buffer under 2 GiB at an affine index whose
    // terms are all ranges or constants with non-negative coefficients (the
    // per-lane part is then a valid offset on its own; a kernel scalar, such
    // as a narrow() start, could be negative for all the renderer knows), and
    // k must need no bounds check (the k-tile's start is not clamped). Measured on C5's kernels alone (same box, same bits): the
    // 8192x4096, K 4096 products 1.4-2.0% faster (forward with the relu of its
    // input, dH with the relu mask, dW with the SGD update), dW1's stream-K
    // pass 1.7%, the K 784 forward within 0.6%.
    bool bufl = !k_check;
    for (auto& ld : st.lds) {
      const UOp& ix = ld.src(0);
      const DTypeKind dk = ld.dtype().kind;
      if (dk != DTypeKind::F32 && dk != DTypeKind::I32) bufl = false;
      if (ix.src(0).op() != Op::ParamBuffer || ix.src(0).arg().b * 4 >= (int64_t(1) << 31)) bufl = false;
      Affine a = affine_of(ix.src(1));
      if (!a.ok || a.c0 < 0) bufl = false;
      for (auto& t : a.terms)
        if (t.second < 0 || t.first.op() != Op::Range) bufl = false;
    }
    std::map<const UOpInner*, std::string> rsrc;
    std::ostringstream decl;
    if (bufl)
      for (auto& ld : st.lds) {
        const UOp& pb = ld.src(0).src(0);
        const std::string nm = "fg_rs_" + pname(pb);
        rsrc[pb.get()] = nm;
        if (rsrc_declared.insert(nm).second)
          decl << "  const __amdgpu_buffer_rsrc_t " << nm << " = __builtin_amdgcn_make_buffer_rsrc((void*)" << pname(pb)
               << ", (short)0, " << pb.arg().b * 4 << ", 0x00020000);\n";
      }
    auto reg = [&](size_t i, const std::string& slot) { return "r" + std::string(X) + std::to_string(i) + "[" + slot + "]"; };
    auto slot = [&](int u) { return V == 1 ? std::string("j") : "4*j+" + std::to_string(u); };
    auto coords = [&]() {
      std::ostringstream c;
      c << "      const int idx = tid + NT * j;\n";
      if (st.md == 0) c << "      const int r = idx / (BK / 4), kk = (idx % (BK / 4)) * 4;\n";
      else if (st.md == 1) c << "      const int kk = idx / (" << BX << " / 4), r = (idx % (" << BX << " / 4)) * 4;\n";
      else if (st.k_fast) c << "      const int r = idx / BK, kk = idx % BK;\n";
      else c << "      const int kk = idx / " << BX << ", r = idx % " << BX << ";\n";
      c << "      const int gr = " << dim << "0 + r, gk = k0 + kk;\n";
      std::string cond;
      if (guard) cond += "idx < " + std::to_string(st.groups);
      if (row_check) cond += (cond.empty() ? "" : " && ") + std::string("gr < ") + std::to_string(ext);
      if (k_check) cond += (cond.empty() ? "" : " && ") + std::string("gk < kend");
      if (cond.empty()) {
        c << "      constexpr bool in = true;\n      const int grc = gr, gkc = gk;\n";
      } else {
        c << "      const bool in = " << cond << ";\n";
        c << "      const int grc = in ? gr : 0, gkc = in ? gk : 0;\n";
      }
      return c.str();
    };
    auto setup = [&](Emitter& em, bool loads) {
      // 64-bit index arithmetic: the per-j address offsets are then constants
      // the compiler folds into the loads, instead of 32-bit sums it must
      // recompute and sign-extend (which alone cost 80+ spilled VGPRs in the
      // 256x256 tile).
      em.define_range(op.rout, "(long)grc");
      if (loads && bufl) {
        em.define_range(g.rk, "(long)kk");
        em.set_buffer_loads(rsrc, g.rk, "k0");
      } else {
        em.define_range(g.rk, "(long)gkc");
      }
      if (st.md == 0) em.set_lane_range(g.rk, 4);
      else if (st.md == 1) em.set_lane_range(op.rout, 4);
    };
    auto indent = [](const std::string& code, const char* pre) {
      std::ostringstream o;
      std::istringstream is(code);
      std::string ln;
      while (std::getline(is, ln)) o << pre << ln << "\n";
      return o.str();
    };
    std::ostringstream l;
    l << decl.str();
    for (size_t i = 0; i < st.lds.size(); i++)
      l << "  " << ctype(st.lds[i].dtype()) << " r" << X << i << "[" << per * V << "];\n";
    l << "  auto load_" << X << " = [&](int k0) {\n";
    l << "    #pragma unroll\n    for (int j = 0; j < " << per << "; j++) {\n" << coords();
    {
      Emitter em;
      setup(em, true);
      std::ostringstream body;
      for (size_t i = 0; i < st.lds.size(); i++)
        for (int u = 0; u < V; u++) body << reg(i, slot(u)) << " = " << em.val(st.lds[i], u) << ";\n";
      l << indent(em.code() + body.str(), "      ");
    }
    l << "    }\n  };\n";
    const char* SX = X[0] == 'a' ? "As" : "Bs";
    l << "  auto store_" << X << " = [&](int buf, int k0) {\n";
    l << "    #pragma unroll\n    for (int j = 0; j < " << per << "; j++) {\n" << coords();
    {
      Emitter em;
      setup(em, false);
      em.load_cb_ = [&](const UOp& ld, int u) -> std::string {
        for (size_t i = 0; i < st.lds.size(); i++)
          if (st.lds[i] == ld) return reg(i, slot(u));
        return std::string();
      };
      std::vector<std::string> vals;
      for (int u = 0; u < V; u++) vals.push_back(em.val(op.expr, u));
      std::ostringstream body;
      for (int u = 0; u < V; u++) body << "v[" << u << "] = in ? " << vals[u] << " : 0.0f;\n";
      l << "      float v[" << V << "];\n";
      if (!(st.lds.size() == 1 && op.expr == st.lds[0])) {
        // The operand is an expression of its loads (a relu recomputed, a
        // mask): pass the raw registers through an empty asm here, so the
        // expression's instructions cannot be scheduled ahead of this point.
        // Without it the scheduler put some of them right after the k-tile's
        // first loads, each behind a wait for those loads to arrive: the C5
        // forward with relu(H) as its operand ran 1990 us against 1830 us for
        // the plain product of the same shape.
        std::string regs;
        for (size_t i = 0; i < st.lds.size(); i++)
          for (int u = 0; u < V; u++) regs += (regs.empty() ? "" : ", ") + std::string("\"+v\"(") + reg(i, slot(u)) + ")";
        l << "      asm volatile(\"\" : " << regs << ");\n";
      }
      l << indent(em.code() + body.str(), "      ");
    }
    const std::string sguard = guard ? "if (idx < " + std::to_string(st.groups) + ") " : "";
    if (st.md == 0) {
      l << "      " << sguard << "*(fg_f4*)(&" << SX << "[buf][r][FG_SWZ(r, kk)]) = fg_f4{v[0], v[1], v[2], v[3]};\n";
    } else if (st.md == 1) {
      l << "      " << sguard << "*(fg_f4*)(&" << SX << "[buf][kk][r]) = fg_f4{v[0], v[1], v[2], v[3]};\n";
    } else if (st.km) {
      l << "      " << sguard << SX << "[buf][kk][r] = v[0];\n";
    } else {
      l << "      " << sguard << SX << "[buf][r][FG_SWZ(r, kk)] = v[0];\n";
    }
    l << "    }\n  };\n";
    return l.str();
  };
  s << loader("a", g.a, sa, BM, M, "m");
  s << loader("b", g.b, sb, BN, N, "n");
  // [k][row] stages: one LDS read of each chunk's interleaved rows per MFMA step.
  auto km_frag = [&](const char* stage, const char* w, const char* fr, int T) {
    std::ostringstream f;
    f << "    #pragma unroll\n    for (int t = 0; t < 4; t++) {\n";
    for (const KmChunk& c : km_chunks(T)) {
      f << "      {\n        const typename fg_vt<" << c.size << ">::t v = *(const typename fg_vt<" << c.size
        << ">::t*)&" << stage << "[buf][8 * g + 4 * h + t][" << w << " + " << 32 * c.first << " + " << c.size
        << " * r32];\n";
      f << "        #pragma unroll\n        for (int i = 0; i < " << c.size << "; i++) " << fr << "[" << c.first
        << " + i][t] = ((const float*)&v)[i];\n      }\n";
    }
    f << "    }\n";
    return f.str();
  };
  // Wave-block position of row r of tile i in a [k][row] stage.
  auto km_pos = [&](int T, const std::string& i, const std::string& r) {
    std::string e = "0";
    const auto ch = km_chunks(T);
    for (size_t c = ch.size(); c-- > 0;) {
      const std::string here = std::to_string(32 * ch[c].first) + " + " + std::to_string(ch[c].size) + " * " + r +
                               " + (" + i + " - " + std::to_string(ch[c].first) + ")";
      e = c + 1 == ch.size() ? here : "(" + i + " < " + std::to_string(ch[c].first + ch[c].size) + " ? " + here + " : " + e + ")";
    }
    return e;
  };
  // Epilogue staging of a [k][row] B operand's columns: one LDS write per chunk.
  auto km_stage = [&]() {
    std::ostringstream f;
    for (const KmChunk& c : km_chunks(TN)) {
      f << "      {\n        typename fg_vt<" << c.size << ">::t v;\n";
      f << "        #pragma unroll\n        for (int j = 0; j < " << c.size << "; j++) ((float*)&v)[j] = acc[i]["
        << c.first << " + j][e];\n";
      f << "        *(typename fg_vt<" << c.size << ">::t*)(wst + rr * EPS + " << 32 * c.first << " + " << c.size
        << " * r32) = v;\n      }\n";
    }
    return f.str();
  };
  s << R"(  // K schedule: in group g (8 k), MFMA step t, lane half h uses k = 8g + 4h + t.
  float fa[2][TM][4], fb[2][TN][4];
  auto frag = [&](int buf, int g, float (&fra)[TM][4], float (&frb)[TN][4]) {
#if A_KM
)" << km_frag("As", "wm", "fra", TM) << R"(#else
    #pragma unroll
    for (int i = 0; i < TM; i++) {
      const fg_f4 v = *(const fg_f4*)&As[buf][wm + 32 * i + r32][FG_SWZ(wm + 32 * i + r32, 8 * g + 4 * h)];
      fra[i][0] = v.x; fra[i][1] = v.y; fra[i][2] = v.z; fra[i][3] = v.w;
    }
#endif
#if B_KM
)" << km_frag("Bs", "wn", "frb", TN) << R"(#else
    #pragma unroll
    for (int j = 0; j < TN; j++) {
      const fg_f4 v = *(const fg_f4*)&Bs[buf][wn + 32 * j + r32][FG_SWZ(wn + 32 * j + r32, 8 * g + 4 * h)];
      frb[j][0] = v.x; frb[j][1] = v.y; frb[j][2] = v.z; frb[j][3] = v.w;
    }
#endif
  };
  const int KT = (kend - kbeg + BK - 1) / BK;
  load_a(kbeg); load_b(kbeg);
  store_a(0, kbeg); store_b(0, kbeg);
  __syncthreads();
  frag(0, 0, fa[0], fb[0]);
  for (int kt = 0; kt < KT; kt++) {
    const int cur = kt & 1;
    // The last k-tile reloads itself, so the body is the same every time.
    const int knext = kbeg + (kt + 1 < KT ? kt + 1 : kt) * BK;
    load_a(knext); load_b(knext);
    #pragma unroll
    for (int g = 0; g < BK / 8; g++) {
      if (g + 1 < BK / 8) frag(cur, g + 1, fa[(g + 1) & 1], fb[(g + 1) & 1]);
      #pragma unroll
      for (int t = 0; t < 4; t++)
        #pragma unroll
        for (int i = 0; i < TM; i++)
          #pragma unroll
          for (int j = 0; j < TN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[g & 1][i][t], fb[g & 1][j][t], acc[i][j], 0, 0, 0);
      if (g == BK / 8 - 1) { store_a(cur ^ 1, knext); store_b(cur ^ 1, knext); }
    }
    fg_sched_k_tile<BK / 8, 0, NV_, ND_, NW_, 4 * TM * TN>();
    __syncthreads();
    frag(cur ^ 1, 0, fa[0], fb[0]);
  }
  // Epilogue: each wave stages the 32 x WN accumulators of tile row i in its
  // own LDS tile (32x32 MFMA layout: element e of lane l is row
  // 8*(e/4) + 4*(l/32) + e%4, column l%32 of its tile), then reads them back as
  // rows of float4, so epilogue operands load and outputs store 16 bytes per
  // lane.
  __syncthreads();
  float* wst = smem + wave * (32 * EPS);
  #pragma unroll
  for (int i = 0; i < TM; i++) {
    #pragma unroll
    for (int e = 0; e < 16; e++) {
      const int rr = 8 * (e >> 2) + 4 * h + (e & 3);
#if B_KM
)" << km_stage() << R"(#else
      #pragma unroll
      for (int j = 0; j < TN; j++) wst[rr * EPS + 32 * j + r32] = acc[i][j][e];
#endif
    }
    __syncthreads();
    #pragma unroll
    for (int q = 0; q < WN / 8; q++) {
      const int ch = lane + 64 * q, rr = ch / (WN / 4), cc = (ch % (WN / 4)) * 4;
      const fg_f4 gv = *(const fg_f4*)(wst + rr * EPS + cc);
#if A_KM
      const int grow = m0 + wm + )" << km_pos(TM, "i", "rr") << R"(;
#else
      const int grow = m0 + wm + 32 * i + rr;
#endif
      const int gcol = n0 + wn + cc;
      if (grow < M_ && gcol < N_) {
)";
  // Everything outside the reduction, for the four columns gcol..gcol+3 of
  // row grow whose sums are in gv.
  auto epilogue = [&]() {
    static const char* kComp[4] = {"gv.x", "gv.y", "gv.z", "gv.w"};
    Emitter em;
    em.define_range(g.rm, "grow");
    const std::string out = pname(ki.out_param);
    if (N % 4 == 0) {
      // Every column group lies inside the tile: lanes along the columns.
      em.define_range(g.rn, "gcol");
      em.set_lane_range(g.rn, 4);
      em.reduce_cb_ = [&](const UOp& RR, int lane) -> std::string {
        FG_CHECK(RR == g.R, "gemm epilogue sees one reduction");
        return kComp[lane];
      };
      std::vector<std::string> vals;
      for (int u = 0; u < 4; u++) vals.push_back(em.val(ki.value, u));
      Affine ao = affine_of(ki.out_index);
      bool vstore = ao.ok && ao.coef(g.rn) == 1 && ao.c0 % 4 == 0 &&
                    ki.out_param.dtype().kind == DTypeKind::F32;
      for (auto& t : ao.terms)
        if (t.first != g.rn && t.second % 4 != 0) vstore = false;
      if (vstore) {
        em.line("*(float4*)(" + out + "+" + em.idx(ki.out_index, 0) + ") = make_float4(" + vals[0] + ", " + vals[1] +
                ", " + vals[2] + ", " + vals[3] + ");");
      } else {
        for (int u = 0; u < 4; u++) em.line(out + "[" + em.idx(ki.out_index, u) + "] = " + vals[u] + ";");
      }
    } else {
      // Ragged last column group: one guarded column at a time.
      for (int u = 0; u < 4; u++) {
        const std::string col = "(gcol+" + std::to_string(u) + ")";
        em.open_scope("if (" + col + " < N_) {", "}");
        em.define_range(g.rn, col);
        em.reduce_cb_ = [&, u](const UOp& RR, int) -> std::string {
          FG_CHECK(RR == g.R, "gemm epilogue sees one reduction");
          return kComp[u];
        };
        std::string v = em.val(ki.value, 0);
        em.line(out + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
        em.close_scope();
      }
    }
    return em.code();
  };
  auto indent = [](const std::string& code, const std::string& pre) {
    std::ostringstream o;
    std::istringstream is(code);
    std::string l;
    while (std::getline(is, l)) o << pre << l << "\n";
    return o.str();
  };
  if (!split) {
    s << indent(epilogue(), "        ");
  } else {
    // Raw partial sums of this K range; the epilogue runs after they are summed.
    s << "        *(fg_f4*)(fg_scratch + ((long)ks * M_ + grow) * NP_ + gcol) = gv;\n";
  }
  s << "      }\n    }\n    __syncthreads();\n  }\n";
  if (tile.stream_k) s << "  }\n";  // the workgroup's next segment
  s << "}\n";
  if (split) {
    // Second pass: one thread per 4 columns of a row sums the partials in
    // split order (stream-K: the tile's segments, in k order), then runs the
    // epilogue.
    s << sig(name + "_fin", 256, false) << " {\n";
    s << R"(  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)M_ * (NP_ / 4)) return;
  const int grow = (int)(gid / (NP_ / 4)), gcol = (int)(gid % (NP_ / 4)) * 4;
  fg_f4 gv = *(const fg_f4*)(fg_scratch + (long)grow * NP_ + gcol);
)";
    if (tile.stream_k && sk_D > 0) {
      // The tile's block index (the inverse of the main pass's row-major
      // slot), then how many workgroups its k-tiles were split over.
      s << R"(  const int nbn = (N_ + BN - 1) / BN, sq = (grow / BM) * nbn + gcol / BN;
  const long t0 = (long)((sq % (NTILES_ / SK_D_)) * SK_D_ + sq / (NTILES_ / SK_D_)) * KTT_;
  const int nseg = fg_sk_owner(t0 + KTT_ - 1) - fg_sk_owner(t0) + 1;
  for (int ks = 1; ks < nseg; ks++) {)";
    } else if (tile.stream_k) {
      // The tile's block index (the inverse of the main pass's grouped
      // order), then how many workgroups its k-tiles were split over.
      s << R"(  const int nbm = (M_ + BM - 1) / BM, nbn = (N_ + BN - 1) / BN, GM = 8;
  const int tm = grow / BM, tn = gcol / BN, group = tm / GM, first_m = group * GM;
  const int gsz = (nbm - first_m) < GM ? (nbm - first_m) : GM;
  const long t0 = (long)(group * GM * nbn + tn * gsz + (tm - first_m)) * KTT_;
  const int nseg = fg_sk_owner(t0 + KTT_ - 1) - fg_sk_owner(t0) + 1;
  for (int ks = 1; ks < nseg; ks++) {)";
    } else {
      s << "  for (int ks = 1; ks < S_; ks++) {";
    }
    s << R"(
    const fg_f4 p = *(const fg_f4*)(fg_scratch + ((long)ks * M_ + grow) * NP_ + gcol);
    gv.x = gv.x + p.x; gv.y = gv.y + p.y; gv.z = gv.z + p.z; gv.w = gv.w + p.w;
  }
  if (gcol < N_) {
)";
    s << indent(epilogue(), "    ");
    s << "  }\n}\n";
  }
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::Gemm);
  rk.source = s.str();
  if (tile.nbuf == 3) rk.source = gemm_three_stages(rk.source);
  rk.block[0] = static_cast<unsigned>(NT);
  rk.grid[0] = static_cast<unsigned>(tile.stream_k ? tile.G : ntiles * S);
  if (tile.stream_k) rk.source = gemm_stream_k(rk.source, sk_D);
  if (split) {
    LaunchSpec a, b;
    a.func = name + "_part";
    a.grid[0] = rk.grid[0];
    a.block[0] = static_cast<unsigned>(NT);
    b.func = name + "_fin";
    b.grid[0] = static_cast<unsigned>((M * (NP / 4) + 255) / 256);
    b.block[0] = 256;
    rk.launches = {a, b};
    rk.scratch_bytes = static_cast<size_t>(S * M * NP) * sizeof(float);
  }
  return rk;
}

// ── Block: a small kernel in one workgroup ──────────────────────────────────
// A kernel with few outputs and little work per output (an MLP's class-axis
// softmax pieces and loss, small bias and weight gradients) is bound by its
// launch, not by the chip: in a graph each launch costs about 2 us of device
// time whatever it does. Such a kernel runs as one 1024-thread workgroup
// whose body is a device function, so a replayed sequence can run several of
// them back to back in one launch (render_block_batch), separated by
// workgroup barriers. The body has three forms:
// - one output per thread, reductions serial in the reference's order
//   (elementwise and serial kernels, and reductions of at most 32 elements);
// - row reductions: G consecutive lanes per output stride the reduce range,
//   then a DPP/swizzle tree over the G lanes;
// - column reductions: consecutive lanes take consecutive outputs, TR row
//   groups split the reduce range, and LDS folds the groups in order.
// The reduction forms walk their outputs in rounds of a fixed trip count, so
// their barriers and lane exchanges run in uniform control flow. A kernel computes the same bits
// whether it runs alone or in a batch: the body is the same code.
// One workgroup has one CU's memory parallelism: a body is cheap only while
// each thread folds few terms. Measured on the C4 train step: a run of five
// [256, 10] kernels whose first computed 2560 outputs of 128 terms each took
// 48 us in one workgroup, against about 15 us as five launches; the loss
// kernels (256 outputs of 10 terms) take well under a launch's cost.
constexpr int kBlockThreads = 1024;
constexpr int64_t kBlockMaxOutputs = 4096;
constexpr int64_t kBlockMaxReduce = 1024;
constexpr int64_t kBlockMaxWork = int64_t(1) << 16;  // terms folded, all outputs: 64 per thread

// Terms a reduction folds per output: its extent, times the terms of any
// reduction recomputed inside its value.
int64_t reduce_terms(const UOp& R) {
  int64_t l = 1;
  for (size_t i = 1; i < R.srcs().size(); i++) l *= range_extent(R.src(i));
  int64_t inner = 0;
  for (auto& n : R.src(0).toposort())
    if (n.op() == Op::Reduce) {
      int64_t m = 1;
      for (size_t i = 1; i < n.srcs().size(); i++) m *= range_extent(n.src(i));
      inner += m;
    }
  return l * (1 + inner);
}

bool block_eligible(const KernelInfo& ki, KernelClass base) {
  if (base == KernelClass::Gemm || base == KernelClass::NarrowGemm || base == KernelClass::Sequential) return false;
  const int64_t T = total_outputs(ki);
  if (T > kBlockMaxOutputs) return false;
  std::set<const UOpInner*> nested;
  for (auto& R : ki.reduces)
    for (auto& n : R.src(0).toposort())
      if (n.op() == Op::Reduce) nested.insert(n.get());
  int64_t terms = 0;
  for (auto& R : ki.reduces) {
    int64_t l = 1;
    for (size_t i = 1; i < R.srcs().size(); i++) l *= range_extent(R.src(i));
    if (l > kBlockMaxReduce) return false;
    if (!nested.count(R.get())) terms += reduce_terms(R);
  }
  return T * std::max<int64_t>(terms, 1) <= kBlockMaxWork;
}

// Parameter list of a block body: no __restrict__, since a batched launch
// passes a buffer one stage writes to a later stage that reads it.
std::string block_params(const KernelInfo& ki, std::vector<std::string>* types, std::vector<std::string>* names) {
  std::ostringstream os;
  bool first = true;
  for (auto& [slot, p] : ki.params) {
    std::string t = p.op() == Op::ParamBuffer ? std::string(p == ki.out_param ? "" : "const ") + ctype(p.dtype()) + "*"
                                              : std::string(ctype(p.dtype()));
    os << (first ? "" : ", ") << t << " data" << slot;
    first = false;
    types->push_back(t);
    names->push_back("data" + std::to_string(slot));
  }
  return os.str();
}

RenderedKernel render_block(const KernelInfo& ki, KernelClass base, const std::string& name) {
  const int64_t T = total_outputs(ki);
  const std::string NT = std::to_string(kBlockThreads);
  Emitter em;
  const UOp* R = ki.reduces.size() == 1 ? &ki.reduces[0] : nullptr;
  // Innermost reduce range; a reduction whose ranges were all of extent 1
  // has none left and folds a single term.
  int64_t Lin = 1;
  if (R && R->srcs().size() >= 2) Lin = range_extent(R->srcs().back());
  const bool serial_form = !R || base == KernelClass::Serial || base == KernelClass::Elementwise || Lin <= 32;
  auto store = [&](const std::string& guard) {
    std::string v = em.val(ki.value, 0);
    em.line(guard + pname(ki.out_param) + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
  };
  if (serial_form) {
    em.open_scope("for (long gid = threadIdx.x; gid < " + std::to_string(T) + "L; gid += " + NT + ") {", "}");
    decode_outputs(em, ki, "gid", UOp());
    em.reduce_cb_ = [&](const UOp& RR, int lane) {
      std::string acc = emit_serial_reduce(em, RR, lane);
      em.pin_here(RR);
      em.remember_here(RR, lane, acc);
      return acc;
    };
    store("");
    em.close_scope();
  } else if (base == KernelClass::ColumnReduce && R->srcs().size() == 2) {
    // Consecutive lanes take consecutive outputs (the memory's fast axis), TR
    // row groups split the reduce range (unrolled, loads in flight together),
    // and the TR partials are folded through LDS in row-group order.
    // TR ~ sqrt(L) balances the loads and the fold.
    const UOp r = R->src(1);
    int TR = 2;
    while (TR < 32 && static_cast<int64_t>(TR) * TR < Lin) TR *= 2;
    const int TX = kBlockThreads / TR;
    const int64_t rounds = (T + TX - 1) / TX, trips = (Lin + TR - 1) / TR;
    const Op rop = R->arg().rop;
    const DType dt = R->dtype();
    em.line("const int tx = threadIdx.x % " + std::to_string(TX) + ", tr = threadIdx.x / " + std::to_string(TX) + ";");
    em.line(std::string("__shared__ ") + ctype(dt) + " fg_blk[" + std::to_string(TR) + "][" + std::to_string(TX) + "];");
    em.open_scope("for (int rnd = 0; rnd < " + std::to_string(rounds) + "; rnd++) {", "}");
    em.line("const long oid = (long)rnd * " + std::to_string(TX) + " + tx;");
    em.line("const bool active = oid < " + std::to_string(T) + "L;");
    em.line("const long ocl = active ? oid : 0;");
    decode_outputs(em, ki, "ocl", UOp());
    em.reduce_cb_ = [&](const UOp& RR, int lane) -> std::string {
      FG_CHECK(RR == *R, "block column reduce renders exactly one reduction");
      std::string acc = em.fresh("bacc");
      em.line(std::string(ctype(dt)) + " " + acc + " = " + init_lit(rop, dt) + ";");
      size_t opened = 0;
      em.open_scope("if (active) {", "}");
      opened++;
      em.open_scope("#pragma unroll\nfor (int bit = 0; bit < " + std::to_string(trips) + "; bit++) {", "}");
      opened++;
      em.line("const int rr = tr + bit * " + std::to_string(TR) + ";");
      if (Lin % TR != 0) {
        em.open_scope("if (rr < " + std::to_string(Lin) + ") {", "}");
        opened++;
      }
      em.define_range(r, "rr");
      em.line(acc + " = " + combine(rop, acc, em.val(R->src(0), 0)) + ";");
      for (size_t i = 0; i < opened; i++) em.close_scope();
      em.line("fg_blk[tr][tx] = " + acc + ";");
      em.line("__syncthreads();");
      em.line(acc + " = fg_blk[0][tx];");
      em.line("#pragma unroll");
      em.line("for (int q = 1; q < " + std::to_string(TR) + "; q++) " + acc + " = " + combine(rop, acc, "fg_blk[q][tx]") +
              ";");
      em.line("__syncthreads();");
      em.pin_here(RR);
      em.remember_here(RR, lane, acc);
      return acc;
    };
    store("if (active && tr == 0) ");
    em.close_scope();
  } else {
    // Row reductions: G consecutive lanes per output stride the innermost
    // reduce range (outer reduce ranges loop serially), fully unrolled so a
    // lane's loads are in flight together, then a DPP/swizzle tree over the G
    // lanes. G ~ sqrt(L) balances the two.
    std::vector<UOp> ranges(R->srcs().begin() + 1, R->srcs().end());
    const UOp r_in = ranges.back();
    int G = 2;
    while (G < 64 && static_cast<int64_t>(G) * G < Lin) G *= 2;
    const int64_t per_round = kBlockThreads / G, rounds = (T + per_round - 1) / per_round;
    const int64_t trips = (Lin + G - 1) / G;
    const Op rop = R->arg().rop;
    const DType dt = R->dtype();
    em.line("const int lg = threadIdx.x % " + std::to_string(G) + ";");
    em.open_scope("for (int rnd = 0; rnd < " + std::to_string(rounds) + "; rnd++) {", "}");
    em.line("const long oid = (long)rnd * " + std::to_string(per_round) + " + threadIdx.x / " + std::to_string(G) + ";");
    em.line("const bool active = oid < " + std::to_string(T) + "L;");
    em.line("const long ocl = active ? oid : 0;");
    decode_outputs(em, ki, "ocl", UOp());
    em.reduce_cb_ = [&](const UOp& RR, int lane) -> std::string {
      FG_CHECK(RR == *R, "block reduction renders exactly one reduction");
      std::string acc = em.fresh("bacc");
      em.line(std::string(ctype(dt)) + " " + acc + " = " + init_lit(rop, dt) + ";");
      size_t opened = 0;
      em.open_scope("if (active) {", "}");
      opened++;
      for (size_t i = 0; i + 1 < ranges.size(); i++) {
        std::string v = "bro" + std::to_string(i);
        em.open_scope("for (int " + v + " = 0; " + v + " < " + std::to_string(range_extent(ranges[i])) + "; " + v + "++) {",
                      "}");
        em.define_range(ranges[i], v);
        opened++;
      }
      em.open_scope("#pragma unroll\nfor (int bit = 0; bit < " + std::to_string(trips) + "; bit++) {", "}");
      opened++;
      em.line("const int rj = lg + bit * " + std::to_string(G) + ";");
      if (Lin % G != 0) {
        em.open_scope("if (rj < " + std::to_string(Lin) + ") {", "}");
        opened++;
      }
      em.define_range(r_in, "rj");
      em.line(acc + " = " + combine(rop, acc, em.val(R->src(0), 0)) + ";");
      for (size_t i = 0; i < opened; i++) em.close_scope();
      std::string wr = wave_reduce(acc, G, rop, dt);
      std::istringstream is(wr);
      std::string l;
      while (std::getline(is, l)) em.line(l);
      em.pin_here(RR);
      em.remember_here(RR, lane, acc);
      return acc;
    };
    store("if (active && lg == 0) ");
    em.close_scope();
  }
  RenderedKernel rk;
  std::vector<std::string> names;
  const std::string params = block_params(ki, &rk.stage_types, &names);
  rk.stage_fn = name + "_body";
  rk.stage_src = "__device__ __forceinline__ void " + rk.stage_fn + "(" + params + ") {\n" + em.code() + "}\n";
  std::string call = rk.stage_fn + "(";
  for (size_t i = 0; i < names.size(); i++) call += (i ? ", " : "") + names[i];
  call += ");";
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::Block);
  rk.source = std::string(kPrelude) + rk.stage_src + "extern \"C\" __global__ void __launch_bounds__(" + NT + ") " + name +
              "(" + params + ") {\n  " + call + "\n}\n";
  rk.block[0] = kBlockThreads;
  rk.grid[0] = 1;
  return rk;
}

// ── Narrow GEMM (VALU, HBM-bound) ───────────────────────────────────────────
// A product with one output side of at most kNarrow elements (the 10 classes
// of an MLP's last layer) streams its wide operand once and does only
// kNarrow FMAs per wide element: an HBM-bound kernel, for which a 32-wide
// MFMA tile is mostly padding. Two layouts, by which way the wide operand is
// contiguous:
// - rows: the wide operand is contiguous along k (out[w, n] = sum_k
//   W[w, k] N[n, k], the forward x·Wᵀ). The lanes of a workgroup stride k by
//   four floats, so every load is a coalesced 16-byte load that streams a row
//   once. The narrow operand's float4 at (n, k) is held in registers for the
//   whole launch when it fits (render_narrow_rows_cached), else loaded once
//   per group of 4 rows. Each accumulator is then summed across the wave by a
//   fixed DPP/swizzle tree, and the totals go through LDS to the lanes that
//   run the epilogue.
// - cols: the wide operand is contiguous along the wide output (out[n, w] =
//   sum_k N[k, n] W[k, w], the weight gradient dZᵀ·H). Lanes own V
//   consecutive wide outputs and loop over k, where the narrow values are the
//   same for every lane. The k range is split over workgroups into scratch
//   partials that a finishing pass sums in split order before the epilogue.
// Both fold in a fixed order, so results are deterministic. The products are
// accumulated with fused multiply-adds (one rounding per term, as the MFMA
// GEMM's are): these kernels are bound by HBM, and unfused they spent as long
// on separate multiplies and adds as on their loads.
constexpr int64_t kNarrow = 16;

struct NarrowPlan {
  bool rows = false;       // the rows layout (else cols)
  UOp rw, rn;              // wide and narrow output ranges
  GemmOperand wide, nar;   // their operands
  int64_t W = 0, NN = 0, K = 0;
};

bool narrow_plan(const GemmMatch& g, NarrowPlan* np) {
  const bool a_narrow = g.M <= kNarrow, b_narrow = g.N <= kNarrow;
  if (a_narrow == b_narrow) return false;
  np->rw = a_narrow ? g.rn : g.rm;
  np->rn = a_narrow ? g.rm : g.rn;
  np->wide = a_narrow ? g.b : g.a;
  np->nar = a_narrow ? g.a : g.b;
  np->W = a_narrow ? g.N : g.M;
  np->NN = a_narrow ? g.M : g.N;
  np->K = g.K;
  const int64_t sk = np->wide.lead.coef(g.rk), sw = np->wide.lead.coef(np->rw);
  if (sk == 1 && np->K % 4 == 0) np->rows = true;
  else if (sw == 1) np->rows = false;
  else return false;
  return np->W >= 256 && np->K >= 64;
}

// The rows layout with the narrow operand held in registers. Thread t owns k
// positions 4t + 1024j (j < JT) and keeps the narrow operand's float4 at each
// of them for every n (NN x JT x 4 floats), so the narrow operand is read once
// per workgroup instead of once per row group. Workgroups are persistent over
// R consecutive rows, folded one at a time; the raw loads of the row D ahead
// are in flight while a row is folded (a ring of D register buffers), and the
// wide operand's expression (a recomputed relu, say) is evaluated on them when
// the row is folded, so no instruction waits on a load before its row's turn.
// Each thread folds the same terms in the same order as the layout below, and
// the sums run through the same trees, so the results are the same bits.
// Measured on the C5 L3 forward shape (8192x10, K 4096, relu recomputed), in
// a standalone A/B over rotated cold buffers: 27.7 us against 45-49 us for the
// row-group layout, 39.8 us for that layout with its sums batched; 256 or 1024
// workgroups, or a ring of 1 or 4 rows, were slower.
constexpr int64_t kNarrowRowGroups = 512;
constexpr int kNarrowRowDepth = 2;

bool narrow_rows_cached_fits(const NarrowPlan& np) {
  const int64_t JT = (np.K + 1023) / 1024;
  const int64_t nloads = static_cast<int64_t>(loads_in(np.wide.expr).size());
  // The workgroup's sums stay in LDS until its last row: 4 x R x NN floats,
  // at most 64 KB.
  const int64_t rows = (np.W + kNarrowRowGroups - 1) / kNarrowRowGroups;
  // About 200 VGPRs in all keeps two waves per SIMD.
  return np.NN * JT * 4 <= 160 && kNarrowRowDepth * nloads * JT * 4 <= 64 && rows * np.NN <= 4096;
}

RenderedKernel render_narrow_rows_cached(const KernelInfo& ki, const GemmMatch& g, const NarrowPlan& np,
                                         const std::string& name) {
  const int NN = static_cast<int>(np.NN);
  const int64_t W = np.W, K = np.K, JT = (K + 1023) / 1024;
  const int64_t groups = std::min<int64_t>(kNarrowRowGroups, W);
  const int64_t R = (W + groups - 1) / groups;
  const int64_t grid = (W + R - 1) / R;
  const int D = kNarrowRowDepth;
  const bool kguard = K % 1024 != 0;
  const std::vector<UOp> lds = loads_in(np.wide.expr);
  const std::string Ws = std::to_string(W), Rs = std::to_string(R), Ks = std::to_string(K);
  auto kname = [](int64_t j) { return "k" + std::to_string(j); };
  auto reg = [](int d, size_t i, int64_t j) {
    return "w" + std::to_string(d) + "_" + std::to_string(i) + "_" + std::to_string(j);
  };
  auto nb = [](int n, int64_t j) { return "nb" + std::to_string(n) + "_" + std::to_string(j); };
  auto open_k = [&](Emitter& e, int64_t j) {
    e.open_scope(kguard ? "if (" + kname(j) + " < " + Ks + ") {" : "{", "}");
    e.define_range(g.rk, kname(j));
    e.set_lane_range(g.rk, 4);
  };
  auto close_k = [](Emitter& e) {
    e.clear_lane_range();
    e.close_scope();
  };

  Emitter em;
  em.set_nontemporal_loads(true);
  em.set_streaming_ranges({np.rw});
  em.line("const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;");
  em.line("const long base = (long)blockIdx.x * " + Rs + ";");
  em.line("__shared__ float fg_nt[4][" + std::to_string(R * NN) + "];");
  for (int64_t j = 0; j < JT; j++) em.line("const int " + kname(j) + " = " + std::to_string(j * 1024) + " + tid * 4;");
  // The narrow operand at this thread's k positions (0 past the end of k).
  for (int64_t j = 0; j < JT; j++) {
    for (int n = 0; n < NN; n++) em.line("float " + nb(n, j) + "[4] = {0.0f, 0.0f, 0.0f, 0.0f};");
    open_k(em, j);
    for (int n = 0; n < NN; n++) {
      em.open_scope("{", "}");
      em.define_range(np.rn, std::to_string(n));
      for (int u = 0; u < 4; u++) em.line(nb(n, j) + "[" + std::to_string(u) + "] = " + em.val(np.nar.expr, u) + ";");
      em.close_scope();
    }
    close_k(em);
  }
  // The ring: raw values of every load of the wide operand's expression.
  for (int d = 0; d < D; d++)
    for (size_t i = 0; i < lds.size(); i++)
      for (int64_t j = 0; j < JT; j++) em.line(std::string(ctype(lds[i].dtype())) + " " + reg(d, i, j) + "[4];");
  // Issue the loads of wide row `row` (clamped to the last row) into buffer d.
  auto load_row = [&](int d, const std::string& row) {
    em.open_scope("{", "}");
    em.line("const long lr = " + row + ";");
    em.line("const int wrow = (int)(lr < " + Ws + "L ? lr : " + std::to_string(W - 1) + "L);");
    em.define_range(np.rw, "wrow");
    for (int64_t j = 0; j < JT; j++) {
      open_k(em, j);
      for (size_t i = 0; i < lds.size(); i++)
        for (int u = 0; u < 4; u++)
          em.line(reg(d, i, j) + "[" + std::to_string(u) + "] = " + em.val(lds[i], u) + ";");
      close_k(em);
    }
    em.close_scope();
  };
  // Fold local row `rl` from buffer d; lane 0 of each wave leaves the wave's
  // sums in fg_nt.
  auto fold_row = [&](int d, const std::string& rl) {
    em.open_scope("{", "}");
    em.line("const long lr = base + " + rl + ";");
    em.line("const int wrow = (int)(lr < " + Ws + "L ? lr : " + std::to_string(W - 1) + "L);");
    em.define_range(np.rw, "wrow");
    for (int n = 0; n < NN; n++) em.line("float acc" + std::to_string(n) + " = 0.0f;");
    int64_t cur_j = 0;
    em.load_cb_ = [&](const UOp& ld, int u) -> std::string {
      for (size_t i = 0; i < lds.size(); i++)
        if (lds[i] == ld) return reg(d, i, cur_j) + "[" + std::to_string(u) + "]";
      return std::string();
    };
    for (int64_t j = 0; j < JT; j++) {
      cur_j = j;
      open_k(em, j);
      std::vector<std::string> a;
      for (int u = 0; u < 4; u++) a.push_back(em.val(np.wide.expr, u));
      for (int n = 0; n < NN; n++) {
        const std::string acc = "acc" + std::to_string(n), b = nb(n, j);
        em.line(acc + " = __builtin_fmaf(" + a[3] + ", " + b + "[3], __builtin_fmaf(" + a[2] + ", " + b +
                "[2], __builtin_fmaf(" + a[1] + ", " + b + "[1], __builtin_fmaf(" + a[0] + ", " + b + "[0], " + acc +
                "))));");
      }
      close_k(em);
    }
    em.load_cb_ = nullptr;
    for (int n = 0; n < NN; n++) {
      std::istringstream is(wave_reduce("acc" + std::to_string(n), 64, Op::Add, DType::F32()));
      std::string l;
      while (std::getline(is, l)) em.line(l);
    }
    em.open_scope("if (lane == 0) {", "}");
    for (int n = 0; n < NN; n++)
      em.line("fg_nt[wave][(" + rl + ") * " + std::to_string(NN) + " + " + std::to_string(n) + "] = acc" +
              std::to_string(n) + ";");
    em.close_scope();
    em.close_scope();
  };
  for (int d = 0; d < D; d++) load_row(d, "base + " + std::to_string(d));
  em.open_scope("for (int ib = 0; ib < " + Rs + "; ib += " + std::to_string(D) + ") {", "}");
  for (int d = 0; d < D; d++) {
    const std::string rl = "(ib + " + std::to_string(d) + ")";
    const std::string ahead = "(ib + " + std::to_string(d + D) + ")";
    em.open_scope(R % D != 0 ? "if (" + rl + " < " + Rs + ") {" : "{", "}");
    fold_row(d, rl);
    load_row(d, "base + (" + ahead + " < " + Rs + " ? " + ahead + " : " + std::to_string(R - 1) + ")");
    em.close_scope();
  }
  em.close_scope();
  // The four waves' sums in wave order, then the epilogue.
  em.line("__syncthreads();");
  em.open_scope("for (int o = tid; o < " + std::to_string(R * NN) + "; o += 256) {", "}");
  em.line("const long orow = base + o / " + std::to_string(NN) + ";");
  em.open_scope("if (orow < " + Ws + "L) {", "}");
  em.line("const int ow = (int)orow, on = o % " + std::to_string(NN) + ";");
  em.line("const float tot = ((fg_nt[0][o] + fg_nt[1][o]) + fg_nt[2][o]) + fg_nt[3][o];");
  em.define_range(np.rw, "ow");
  em.define_range(np.rn, "on");
  em.reduce_cb_ = [&](const UOp& RR, int) -> std::string {
    FG_CHECK(RR == g.R, "narrow gemm epilogue sees one reduction");
    return "tot";
  };
  std::string v = em.val(ki.value, 0);
  em.line(pname(ki.out_param) + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
  em.close_scope();
  em.close_scope();
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::NarrowGemm);
  rk.source = std::string(kPrelude) + signature(ki, name, 256) + " {\n" + em.code() + "}\n";
  rk.block[0] = 256;
  rk.grid[0] = static_cast<unsigned>(grid);
  return rk;
}

RenderedKernel render_narrow_rows(const KernelInfo& ki, const GemmMatch& g, const NarrowPlan& np,
                                  const std::string& name) {
  // A workgroup owns RB wide rows. Thread t owns k positions 4t + 1024j
  // (j < JT); for a group of JG blocks it first issues the 16-byte loads of all
  // RB rows, then folds them with the narrow operand's float4 at each (n, k),
  // so a workgroup's whole share of the wide operand is in flight at once.
  const int NN = static_cast<int>(np.NN);
  const int RB = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(4, 48 / np.NN)));
  const int64_t W = np.W, K = np.K, JT = (K + 1023) / 1024;
  const int JG = static_cast<int>(std::min<int64_t>(JT, 4));
  Emitter em;
  em.set_nontemporal_loads(true);
  em.set_streaming_ranges({np.rw});
  em.line("const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;");
  em.line("const long row0 = (long)blockIdx.x * " + std::to_string(RB) + ";");
  for (int r = 0; r < RB; r++) {
    em.line("const int wr" + std::to_string(r) + " = (int)(row0 + " + std::to_string(r) + " < " + std::to_string(W) +
            "L ? row0 + " + std::to_string(r) + " : " + std::to_string(W - 1) + ");");
    for (int n = 0; n < NN; n++) em.line("float acc" + std::to_string(r) + "_" + std::to_string(n) + " = 0.0f;");
  }
  em.open_scope("for (int jg = 0; jg < " + std::to_string(JT) + "; jg += " + std::to_string(JG) + ") {", "}");
  // The wide operand's values for the group (rows past the end read the
  // last row; k past the end contributes nothing).
  for (int j = 0; j < JG; j++) {
    const std::string kj = "k" + std::to_string(j);
    em.line("const int " + kj + " = (jg + " + std::to_string(j) + ") * 1024 + tid * 4;");
    for (int r = 0; r < RB; r++) em.line("float a" + std::to_string(r) + "_" + std::to_string(j) + "[4] = {0.0f, 0.0f, 0.0f, 0.0f};");
    em.open_scope("if (" + kj + " < " + std::to_string(K) + ") {", "}");
    em.define_range(g.rk, kj);
    em.set_lane_range(g.rk, 4);
    for (int r = 0; r < RB; r++) {
      em.open_scope("{", "}");
      em.define_range(np.rw, "wr" + std::to_string(r));
      for (int u = 0; u < 4; u++)
        em.line("a" + std::to_string(r) + "_" + std::to_string(j) + "[" + std::to_string(u) + "] = " +
                em.val(np.wide.expr, u) + ";");
      em.close_scope();
    }
    em.clear_lane_range();
    em.close_scope();
  }
  for (int j = 0; j < JG; j++) {
    const std::string kj = "k" + std::to_string(j);
    em.open_scope("if (" + kj + " < " + std::to_string(K) + ") {", "}");
    em.define_range(g.rk, kj);
    em.set_lane_range(g.rk, 4);
    for (int n = 0; n < NN; n++) {
      em.open_scope("{", "}");
      em.define_range(np.rn, std::to_string(n));
      std::vector<std::string> b;
      for (int u = 0; u < 4; u++) b.push_back(em.val(np.nar.expr, u));
      for (int r = 0; r < RB; r++) {
        const std::string acc = "acc" + std::to_string(r) + "_" + std::to_string(n);
        const std::string a = "a" + std::to_string(r) + "_" + std::to_string(j);
        em.line(acc + " = __builtin_fmaf(" + a + "[3], " + b[3] + ", __builtin_fmaf(" + a + "[2], " + b[2] +
                ", __builtin_fmaf(" + a + "[1], " + b[1] + ", __builtin_fmaf(" + a + "[0], " + b[0] + ", " + acc + "))));");
      }
      em.close_scope();
    }
    em.clear_lane_range();
    em.close_scope();
  }
  em.close_scope();
  // Sums over the workgroup: a fixed DPP/swizzle tree in each wave, then the
  // four waves in order through LDS. Every tree runs before the one branch
  // that stores the totals, so the trees' lane exchanges overlap; a store
  // branch after each tree serialised their latencies (17% of the kernel).
  const int outs = RB * NN;
  em.line("__shared__ float fg_nt[4][" + std::to_string(outs) + "];");
  for (int r = 0; r < RB; r++)
    for (int n = 0; n < NN; n++) {
      const std::string acc = "acc" + std::to_string(r) + "_" + std::to_string(n);
      std::istringstream is(wave_reduce(acc, 64, Op::Add, DType::F32()));
      std::string l;
      while (std::getline(is, l)) em.line(l);
    }
  em.open_scope("if (lane == 0) {", "}");
  for (int r = 0; r < RB; r++)
    for (int n = 0; n < NN; n++)
      em.line("fg_nt[wave][" + std::to_string(r * NN + n) + "] = acc" + std::to_string(r) + "_" + std::to_string(n) + ";");
  em.close_scope();
  em.line("__syncthreads();");
  em.open_scope("if (tid < " + std::to_string(outs) + ") {", "}");
  em.line("const long orow = row0 + tid / " + std::to_string(NN) + ";");
  em.open_scope("if (orow < " + std::to_string(W) + "L) {", "}");
  em.line("const int ow = (int)orow, on = tid % " + std::to_string(NN) + ";");
  em.line("const float tot = ((fg_nt[0][tid] + fg_nt[1][tid]) + fg_nt[2][tid]) + fg_nt[3][tid];");
  em.define_range(np.rw, "ow");
  em.define_range(np.rn, "on");
  em.reduce_cb_ = [&](const UOp& RR, int) -> std::string {
    FG_CHECK(RR == g.R, "narrow gemm epilogue sees one reduction");
    return "tot";
  };
  std::string v = em.val(ki.value, 0);
  em.line(pname(ki.out_param) + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
  em.close_scope();
  em.close_scope();
  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::NarrowGemm);
  rk.source = std::string(kPrelude) + signature(ki, name, 256) + " {\n" + em.code() + "}\n";
  rk.block[0] = 256;
  rk.grid[0] = static_cast<unsigned>((W + RB - 1) / RB);
  return rk;
}

RenderedKernel render_narrow_cols(const KernelInfo& ki, const GemmMatch& g, const NarrowPlan& np,
                                  const std::string& name) {
  const int NN = static_cast<int>(np.NN);
  const int64_t W = np.W, K = np.K;
  // V wide outputs per lane (16-byte loads when the wide extent allows).
  const int V = W % 4 == 0 ? 4 : 1;
  const int64_t cols_per_wg = 64 * V, cblocks = (W + cols_per_wg - 1) / cols_per_wg;
  // k splits: about 1024 workgroups, each wave running at least 16 k. The
  // partials (S x NN x W floats) stay under a tenth of the wide operand.
  int64_t S = std::max<int64_t>(1, std::min<int64_t>((1024 + cblocks - 1) / cblocks, K / 64));
  const int64_t KC = ((K + S - 1) / S + 3) / 4 * 4;  // per workgroup, a multiple of the 4 waves
  S = (K + KC - 1) / KC;
  const int64_t KW = KC / 4;                         // per wave
  const bool split = S > 1;
  const std::string sig_extra = split ? ", float* __restrict__ fg_scratch" : "";
  auto sig = [&](const std::string& fn) {
    std::string s = signature(ki, fn, 256);
    return s.substr(0, s.size() - 1) + sig_extra + ")";
  };
  // Output (n, w)'s epilogue with its sum in `sum`.
  auto epilogue = [&](Emitter& em, const std::string& n, const std::string& w, const std::string& sum) {
    em.define_range(np.rn, n);
    em.define_range(np.rw, w);
    em.reduce_cb_ = [&g, sum](const UOp& RR, int) -> std::string {
      FG_CHECK(RR == g.R, "narrow gemm epilogue sees one reduction");
      return sum;
    };
    std::string v = em.val(ki.value, 0);
    em.line(pname(ki.out_param) + "[" + em.idx(ki.out_index, 0) + "] = " + v + ";");
  };

  Emitter em;
  em.set_nontemporal_loads(true);
  em.set_streaming_ranges({np.rw});
  // The wave index as a wave-uniform value: k is then uniform across lanes, so
  // the narrow operand's loads are scalar loads.
  em.line("const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);");
  em.line("const long cb = blockIdx.x % " + std::to_string(cblocks) + ";");
  em.line("const int ks = (int)(blockIdx.x / " + std::to_string(cblocks) + ");");
  em.line("const long wl = cb * " + std::to_string(cols_per_wg) + " + lane * " + std::to_string(V) + ";");
  em.line("const bool active = wl < " + std::to_string(W) + "L;");
  em.line("const int w0 = active ? (int)wl : 0;");
  em.line("const int kw0 = ks * " + std::to_string(KC) + " + wave * " + std::to_string(KW) + ";");
  em.line("const int kw1 = kw0 + " + std::to_string(KW) + " < " + std::to_string(K) + " ? kw0 + " + std::to_string(KW) +
          " : " + std::to_string(K) + ";");
  for (int n = 0; n < NN; n++)
    for (int u = 0; u < V; u++) em.line("float acc" + std::to_string(n) + "_" + std::to_string(u) + " = 0.0f;");
  em.define_range(np.rw, "w0");
  // Batches of KB rows: the batch's wide loads are issued before its FMAs.
  constexpr int KB = 8;
  em.open_scope("for (int kb = kw0; kb < kw1; kb += " + std::to_string(KB) + ") {", "}");
  for (int q = 0; q < KB; q++) {
    const std::string kq = "kq" + std::to_string(q);
    em.line("const int " + kq + " = kb + " + std::to_string(q) + " < kw1 ? kb + " + std::to_string(q) + " : kw1 - 1;");
    em.line("float wv" + std::to_string(q) + "[" + std::to_string(V) + "];");
    em.open_scope("{", "}");
    em.define_range(g.rk, kq);
    if (V > 1) em.set_lane_range(np.rw, V);
    for (int u = 0; u < V; u++)
      em.line("wv" + std::to_string(q) + "[" + std::to_string(u) + "] = " + em.val(np.wide.expr, u) + ";");
    em.clear_lane_range();
    em.close_scope();
  }
  for (int q = 0; q < KB; q++) {
    const std::string kq = "kq" + std::to_string(q);
    em.open_scope("if (kb + " + std::to_string(q) + " < kw1) {", "}");
    em.define_range(g.rk, kq);
    for (int n = 0; n < NN; n++) {
      em.open_scope("{", "}");
      em.define_range(np.rn, std::to_string(n));
      const std::string b = em.val(np.nar.expr, 0);
      for (int u = 0; u < V; u++) {
        const std::string acc = "acc" + std::to_string(n) + "_" + std::to_string(u);
        em.line(acc + " = __builtin_fmaf(" + b + ", wv" + std::to_string(q) + "[" + std::to_string(u) + "], " + acc + ");");
      }
      em.close_scope();
    }
    em.close_scope();
  }
  em.close_scope();
  // The four waves' sums, in wave order, through LDS.
  const int per_wg = NN * static_cast<int>(cols_per_wg);
  em.line("__shared__ float fg_nc[4][" + std::to_string(per_wg) + "];");
  for (int n = 0; n < NN; n++)
    for (int u = 0; u < V; u++)
      em.line("fg_nc[wave][" + std::to_string(n) + " * " + std::to_string(cols_per_wg) + " + lane * " + std::to_string(V) +
              " + " + std::to_string(u) + "] = acc" + std::to_string(n) + "_" + std::to_string(u) + ";");
  em.line("__syncthreads();");
  em.open_scope("for (int o = threadIdx.x; o < " + std::to_string(per_wg) + "; o += 256) {", "}");
  em.line("const int on = o / " + std::to_string(cols_per_wg) + ";");
  em.line("const long owl = cb * " + std::to_string(cols_per_wg) + " + o % " + std::to_string(cols_per_wg) + ";");
  em.open_scope("if (owl < " + std::to_string(W) + "L) {", "}");
  em.line("const int ow = (int)owl;");
  em.line("const float tot = ((fg_nc[0][o] + fg_nc[1][o]) + fg_nc[2][o]) + fg_nc[3][o];");
  if (split) {
    em.line("fg_scratch[((long)ks * " + std::to_string(NN) + " + on) * " + std::to_string(W) + "L + ow] = tot;");
  } else {
    epilogue(em, "on", "ow", "tot");
  }
  em.close_scope();
  em.close_scope();

  RenderedKernel rk;
  rk.name = name;
  rk.kind = kernel_class_name(KernelClass::NarrowGemm);
  const std::string main_name = split ? name + "_part" : name;
  rk.source = std::string(kPrelude) + sig(main_name) + " {\n" + em.code() + "}\n";
  rk.block[0] = 256;
  rk.grid[0] = static_cast<unsigned>(cblocks * S);
  if (split) {
    // Finishing pass: one thread per output sums the S partials in split
    // order, then runs the epilogue.
    Emitter fin;
    const int64_t outs = np.NN * W;
    fin.line("const long gid = (long)blockIdx.x * 256 + threadIdx.x;");
    fin.line("if (gid >= " + std::to_string(outs) + "L) return;");
    fin.line("const int on = (int)(gid / " + std::to_string(W) + "), ow = (int)(gid % " + std::to_string(W) + ");");
    fin.line("float tot = fg_scratch[gid];");
    fin.line("for (int s = 1; s < " + std::to_string(S) + "; s++) tot = tot + fg_scratch[(long)s * " + std::to_string(outs) +
             "L + gid];");
    epilogue(fin, "on", "ow", "tot");
    rk.source += sig(name + "_fin") + " {\n" + fin.code() + "}\n";
    LaunchSpec a, b;
    a.func = name + "_part";
    a.grid[0] = rk.grid[0];
    a.block[0] = 256;
    b.func = name + "_fin";
    b.grid[0] = static_cast<unsigned>((outs + 255) / 256);
    b.block[0] = 256;
    rk.launches = {a, b};
    rk.scratch_bytes = static_cast<size_t>(S * outs) * sizeof(float);
  }
  return rk;
}

// Whether an in-place kernel reads its destination at an index other than
// the one it stores to (the reference executes such a kernel sequentially).
// A reduction whose value holds another reduction over the same Range node:
// the ranges intern to one node (same axis, kind and extent), so the inner
// loop's loads would be the outer loop's and fold the wrong elements. The
// reference never nests reductions in one kernel (schedule.rs materialises
// nested reduces); the HIP schedule's fusions must not either.
bool nests_reduce_over_same_range(const UOp& kernel) {
  for (auto& n : kernel.toposort()) {
    if (n.op() != Op::Reduce || n.srcs().size() < 2) continue;
    UOpSet outer(n.srcs().begin() + 1, n.srcs().end());
    for (auto& m : n.src(0).toposort())
      if (m.op() == Op::Reduce)
        for (size_t i = 1; i < m.srcs().size(); i++)
          if (outer.count(m.src(i))) return true;
  }
  return false;
}

bool reads_dest_elsewhere(const KernelInfo& ki) {
  for (auto& ld : loads_in(ki.value)) {
    if (ld.src(0).src(0) != ki.out_param) continue;
    if (ld.src(0).src(1) != ki.out_index) return true;
  }
  return false;
}

}  // namespace

// The class a kernel would have on its own size (no block promotion).
KernelClass base_class(const UOp& kernel) {
  KernelInfo ki = analyze_kernel(kernel);
  if (reads_dest_elsewhere(ki)) return KernelClass::Sequential;
  if (ki.reduces.empty()) return KernelClass::Elementwise;
  if (ki.reduces.size() > 1) return KernelClass::Serial;
  GemmMatch g;
  const GpuPasses& on = gpu_passes();
  if ((on.mfma || on.narrow) && match_gemm(ki, &g)) {
    // A narrow product whose wide operand streams along k runs in one pass
    // as VALU rows; otherwise a small product takes the one-pass small GEMM
    // before the narrow columns' two passes.
    NarrowPlan np;
    const bool narrow = on.narrow && narrow_plan(g, &np);
    if (narrow && np.rows) return KernelClass::NarrowGemm;
    if (on.mfma && small_gemm_fits(g.M, g.N, g.K)) return KernelClass::Gemm;
    if (narrow) return KernelClass::NarrowGemm;
    if (on.mfma) return KernelClass::Gemm;
  }
  const UOp& R = ki.reduces[0];
  // A reduction nested in another reduction's value renders serially.
  for (auto& n : R.src(0).toposort())
    if (n.op() == Op::Reduce) return KernelClass::Serial;
  if (R.srcs().size() < 2) return KernelClass::Serial;
  for (auto& ld : loads_in(R.src(0)))
    if (!affine_of(ld.src(0).src(1)).ok) return KernelClass::Serial;
  const UOp r_in = R.srcs().back();
  UOp fast = pick_fast_output(ki);
  int row = 0, col = 0;
  for (auto& ld : loads_in(R.src(0))) {
    Affine a = affine_of(ld.src(0).src(1));
    if (a.coef(r_in) == 1) row++;
    else if (fast && a.coef(fast) == 1) col++;
  }
  if (!fast || row >= col) return KernelClass::RowReduce;
  if (R.srcs().size() == 2) return KernelClass::ColumnReduce;
  return KernelClass::Serial;
}

KernelClass classify_kernel(const UOp& kernel) {
  const KernelClass base = base_class(kernel);
  if (gpu_passes().block && block_eligible(analyze_kernel(kernel), base)) return KernelClass::Block;
  return base;
}

RenderedKernel render_hip(const UOp& kernel, const std::string& name, int force_class) {
  KernelInfo ki = analyze_kernel(kernel);
  // Kernel indexes are int32, as rangeify builds them (schedule/indexing.rs:
  // 42-62 multiplies i32 ranges by i32 strides). A buffer of 2^31 or more
  // elements would wrap: refuse it rather than index out of bounds.
  for (auto& [slot, p] : ki.params)
    if (p.op() == Op::ParamBuffer)
      FG_CHECK(p.arg().b < (int64_t(1) << 31), "buffer data" + std::to_string(slot) + " has " +
                                                   std::to_string(p.arg().b) +
                                                   " elements; kernel indexes are int32 (at most 2^31-1 elements)");
  FG_CHECK(total_outputs(ki) < (int64_t(1) << 31), "kernel has " + std::to_string(total_outputs(ki)) +
                                                         " outputs; kernel indexes are int32 (at most 2^31-1)");
  FG_CHECK(!nests_reduce_over_same_range(kernel),
           "kernel nests a reduction inside another over the same range; it must be materialised first");
  std::vector<std::pair<int, DType>> params;
  for (auto& [slot, p] : ki.params) params.emplace_back(slot, p.dtype());
  if (total_outputs(ki) == 0) {
    // An output axis of extent 0: no element to compute, as the reference's
    // loop nest runs no iteration. One launch that does nothing keeps the
    // sequence uniform (the classes' launch shapes assume an output).
    RenderedKernel rk;
    rk.name = name + "_empty";
    rk.kind = "empty";
    rk.source = std::string(kPrelude) + signature(ki, rk.name, 64) + " {}\n";
    rk.block[0] = 64;
    rk.grid[0] = 1;
    rk.params = params;
    rk.out_slot = static_cast<int>(ki.out_param.arg().a);
    rk.out_count = 0;
    return rk;
  }
  // An in-place update that reads its destination at another index has one
  // valid order, the reference's sequential one, whatever class is asked for.
  KernelClass k = reads_dest_elsewhere(ki)  ? KernelClass::Sequential
                  : force_class >= 0        ? static_cast<KernelClass>(force_class)
                                            : classify_kernel(kernel);
  if (!ki.reduces.empty() && k == KernelClass::Elementwise) k = KernelClass::Serial;
  // The symbol carries the lowering class so profiles name what ran.
  static const char* suffix[] = {"_gemm", "_ew", "_rowred", "_colred", "_serial", "_ngemm", "_blk", "_seq"};
  const std::string sym = name + suffix[static_cast<int>(k)];
  RenderedKernel rk;
  switch (k) {
    case KernelClass::Gemm: {
      GemmMatch g;
      FG_CHECK(match_gemm(ki, &g), "kernel does not match the MFMA GEMM pattern");
      rk = render_gemm(ki, g, sym);
      break;
    }
    case KernelClass::NarrowGemm: {
      GemmMatch g;
      NarrowPlan np;
      FG_CHECK(match_gemm(ki, &g) && narrow_plan(g, &np), "kernel does not match the narrow GEMM pattern");
      if (!np.rows) rk = render_narrow_cols(ki, g, np, sym);
      else if (narrow_rows_cached_fits(np)) rk = render_narrow_rows_cached(ki, g, np, sym);
      else rk = render_narrow_rows(ki, g, np, sym);
      break;
    }
    case KernelClass::Elementwise: rk = render_elementwise(ki, sym); break;
    case KernelClass::RowReduce: rk = render_row_reduce(ki, sym); break;
    case KernelClass::ColumnReduce: rk = render_column_reduce(ki, sym); break;
    case KernelClass::Serial: rk = render_serial(ki, sym); break;
    case KernelClass::Sequential: rk = render_sequential(ki, sym); break;
    case KernelClass::Block: {
      const KernelClass base = base_class(kernel);
      FG_CHECK(block_eligible(ki, base), "kernel is too large for one workgroup");
      rk = render_block(ki, base, sym);
      break;
    }
  }
  rk.params = params;
  rk.out_slot = static_cast<int>(ki.out_param.arg().a);
  for (auto& ld : loads_in(ki.value)) rk.reads_output = rk.reads_output || ld.src(0).src(0) == ki.out_param;
  rk.out_count = static_cast<size_t>(total_outputs(ki));
  return rk;
}

// Kernel symbols are named by a hash of their source, so the same kernel gets
// the same name (and the same cached code object) in every process.
RenderedKernel render_hip_stable(const UOp& kernel) {
  static const std::string kPlaceholder = "FGKERNELNAME";
  RenderedKernel rk = render_hip(kernel, kPlaceholder);
  uint64_t h = 1469598103934665603ULL;
  for (unsigned char c : rk.source) {
    h ^= c;
    h *= 1099511628211ULL;
  }
  char hex[32];
  std::snprintf(hex, sizeof(hex), "k%012llx", static_cast<unsigned long long>(h & 0xffffffffffffULL));
  auto replace_all = [&](std::string& s) {
    for (size_t p = s.find(kPlaceholder); p != std::string::npos; p = s.find(kPlaceholder, p))
      s.replace(p, kPlaceholder.size(), hex);
  };
  replace_all(rk.source);
  replace_all(rk.name);
  replace_all(rk.stage_fn);
  replace_all(rk.stage_src);
  replace_all(rk.hbody_fn);
  replace_all(rk.hbody_src);
  for (auto& l : rk.launches) replace_all(l.func);
  return rk;
}

// The batch's part of a launch: stage bodies appended to `src` (each body
// once), parameters a<first_arg>... appended to `params`, and the statements
// that run the stages (LDS hand-off arrays, barriers, stage calls, copies of
// forwarded outputs, the read-back) appended to `body`.
static void batch_part(const std::vector<const RenderedKernel*>& stages, bool read_back, const BatchForwarding* fwd,
                       size_t first_arg, std::set<std::string>& defined, std::ostringstream& src,
                       std::ostringstream& params, std::ostringstream& body) {
  size_t nargs = 0;
  for (auto* st : stages) nargs += st->stage_types.size();
  FG_CHECK(!fwd || fwd->arg_buffer.size() == nargs, "batch forwarding: one entry per argument");
  if (fwd) {
    for (size_t k = 0; k < fwd->dtypes.size(); k++)
      body << "  __shared__ __attribute__((aligned(16))) " << ctype(fwd->dtypes[k]) << " fg_fwd" << k << "["
           << fwd->numels[k] << "];\n";
  }
  size_t n = first_arg, j_all = 0;
  for (size_t i = 0; i < stages.size(); i++) {
    const RenderedKernel& st = *stages[i];
    FG_CHECK(!st.stage_fn.empty(), "kernel " + st.name + " is not a block kernel");
    if (defined.insert(st.stage_fn).second) src << st.stage_src;
    const bool barrier = fwd && !fwd->barrier.empty() ? fwd->barrier[i] != 0 : i > 0;
    if (barrier) body << "  __syncthreads();\n";
    body << "  " << st.stage_fn << "(";
    for (size_t j = 0; j < st.stage_types.size(); j++, n++, j_all++) {
      params << (n ? ", " : "") << st.stage_types[j] << " a" << n;
      const int k = fwd ? fwd->arg_buffer[j_all] : -1;
      body << (j ? ", " : "") << (k >= 0 ? "fg_fwd" + std::to_string(k) : "a" + std::to_string(n));
    }
    body << ");\n";
  }
  if (fwd && !fwd->dtypes.empty()) {
    // The forwarded outputs reach their buffers once every stage has run.
    body << "  __syncthreads();\n";
    for (size_t k = 0; k < fwd->dtypes.size(); k++)
      body << "  for (int i = threadIdx.x; i < " << fwd->numels[k] << "; i += " << kBlockThreads << ") a"
           << first_arg + fwd->out_arg[k] << "[i] = fg_fwd" << k << "[i];\n";
  }
  if (read_back) {
    params << ", unsigned int* rb_dst, const unsigned int* rb_src, int rb_words";
    body << "  __syncthreads();\n"
         << "  for (int i = threadIdx.x; i < rb_words; i += " << kBlockThreads << ") rb_dst[i] = rb_src[i];\n";
  }
}

// Names a rendered launch by a hash of its source (the placeholder replaced).
static void name_by_hash(RenderedKernel& rk, const std::string& placeholder, const char* cls) {
  uint64_t h = 1469598103934665603ULL;
  for (unsigned char c : rk.source) {
    h ^= c;
    h *= 1099511628211ULL;
  }
  char hex[40];
  std::snprintf(hex, sizeof(hex), "k%012llx_%s", static_cast<unsigned long long>(h & 0xffffffffffffULL), cls);
  for (size_t p = rk.source.find(placeholder); p != std::string::npos; p = rk.source.find(placeholder, p))
    rk.source.replace(p, placeholder.size(), hex);
  rk.name = hex;
}

RenderedKernel render_block_batch(const std::vector<const RenderedKernel*>& stages, bool read_back,
                                  const BatchForwarding* fwd) {
  FG_CHECK(stages.size() >= (read_back ? 1u : 2u), "a batch runs at least two block kernels");
  static const std::string kPlaceholder = "FGBATCHNAME";
  std::ostringstream src, params, body;
  src << kPrelude;
  std::set<std::string> defined;
  batch_part(stages, read_back, fwd, 0, defined, src, params, body);
  src << "extern \"C\" __global__ void __launch_bounds__(" << kBlockThreads << ") " << kPlaceholder << "("
      << params.str() << ") {\n" << body.str() << "}\n";
  RenderedKernel rk;
  rk.source = src.str();
  name_by_hash(rk, kPlaceholder, "batch");
  rk.kind = "block_batch";
  rk.block[0] = kBlockThreads;
  return rk;
}

RenderedKernel render_hbatch(const std::vector<const RenderedKernel*>& hb,
                             const std::vector<const RenderedKernel*>& stages, bool read_back,
                             const BatchForwarding* fwd) {
  FG_CHECK(!hb.empty() && hb.size() <= 2 && !stages.empty(), "render_hbatch: one or two kernels and a batch");
  static const std::string kPlaceholder = "FGHBATCHNAME";
  std::ostringstream src, params, body, dispatch;
  src << kPrelude;
  std::set<std::string> defined;
  size_t n = 0;
  unsigned g0 = 0;
  dispatch << "  if (blockIdx.x != 0u) {\n    const unsigned fg_hbid = blockIdx.x - 1u;\n";
  for (size_t i = 0; i < hb.size(); i++) {
    const RenderedKernel& k = *hb[i];
    FG_CHECK(!k.hbody_fn.empty() && k.launches.empty() && k.scratch_bytes == 0,
             "render_hbatch: " + k.name + " has no block-index body");
    FG_CHECK(k.block[1] == 1 && k.block[2] == 1 && k.grid[1] == 1 && k.grid[2] == 1 && k.block[0] % 64 == 0 &&
                 k.block[0] <= static_cast<unsigned>(kBlockThreads),
             "render_hbatch: " + k.name + " is not a 1-D launch of whole waves within a block kernel's workgroup");
    FG_CHECK(k.source.find(k.hbody_fn + "(") != std::string::npos,
             "render_hbatch: a body is not the one its kernel calls");
    if (defined.insert(k.hbody_fn).second) src << k.hbody_src;
    else
      FG_CHECK(hb[0]->hbody_src == k.hbody_src, "render_hbatch: two different bodies named " + k.hbody_fn);
    std::ostringstream call;
    call << k.hbody_fn << "(";
    for (auto& t : k.hbody_types) {
      params << (n ? ", " : "") << t << " a" << n;
      call << "a" << n++ << ", ";
    }
    // Waves past the kernel's own workgroup size end at once; the body's
    // barriers count the waves that run it.
    const std::string run = "if (threadIdx.x < " + std::to_string(k.block[0]) + "u) " + call.str();
    if (i + 1 < hb.size())
      dispatch << "    if (fg_hbid < " << g0 + k.grid[0] << "u) { " << run << "fg_hbid - " << g0 << "u); }\n    else ";
    else
      dispatch << (i ? "{ " : "    { ") << run << "fg_hbid - " << g0 << "u); }\n";
    g0 += k.grid[0];
  }
  dispatch << "    return;\n  }\n";
  batch_part(stages, read_back, fwd, n, defined, src, params, body);
  src << "extern \"C\" __global__ void __launch_bounds__(" << kBlockThreads << ") " << kPlaceholder << "("
      << params.str() << ") {\n" << dispatch.str() << body.str() << "}\n";
  RenderedKernel rk;
  rk.source = src.str();
  name_by_hash(rk, kPlaceholder, "hbatch");
  rk.kind = "hbatch";
  rk.block[0] = kBlockThreads;
  rk.grid[0] = 1 + g0;
  return rk;
}

RenderedKernel render_hfused(const RenderedKernel& a, const RenderedKernel& b) {
  FG_CHECK(!a.hbody_fn.empty() && !b.hbody_fn.empty(), "render_hfused: kernels without a block-index body");
  // Bodies are emitted once per name: one name must mean one body.
  FG_CHECK(a.hbody_fn != b.hbody_fn || a.hbody_src == b.hbody_src,
           "render_hfused: two different bodies named " + a.hbody_fn);
  FG_CHECK(a.source.find(a.hbody_fn + "(") != std::string::npos &&
               b.source.find(b.hbody_fn + "(") != std::string::npos,
           "render_hfused: a body is not the one its kernel calls");
  FG_CHECK(a.block[0] == b.block[0] && a.block[1] == 1 && a.block[2] == 1 && b.block[1] == 1 && b.block[2] == 1 &&
               a.grid[1] == 1 && a.grid[2] == 1 && b.grid[1] == 1 && b.grid[2] == 1,
           "render_hfused: the kernels' launch shapes differ");
  static const std::string kPlaceholder = "FGHFUSEDNAME";
  std::ostringstream src, params, call_a, call_b;
  src << kPrelude << a.hbody_src;
  if (b.hbody_fn != a.hbody_fn) src << b.hbody_src;
  size_t n = 0;
  call_a << a.hbody_fn << "(";
  for (auto& t : a.hbody_types) {
    params << (n ? ", " : "") << t << " a" << n;
    call_a << "a" << n++ << ", ";
  }
  call_b << b.hbody_fn << "(";
  for (auto& t : b.hbody_types) {
    params << (n ? ", " : "") << t << " a" << n;
    call_b << "a" << n++ << ", ";
  }
  src << "extern \"C\" __global__ void __launch_bounds__(" << a.block[0] << ") " << kPlaceholder << "(" << params.str()
      << ") {\n  if (blockIdx.x < " << a.grid[0] << "u) " << call_a.str() << "blockIdx.x);\n  else " << call_b.str()
      << "blockIdx.x - " << a.grid[0] << "u);\n}\n";
  RenderedKernel rk;
  rk.source = src.str();
  uint64_t h = 1469598103934665603ULL;
  for (unsigned char c : rk.source) {
    h ^= c;
    h *= 1099511628211ULL;
  }
  char hex[40];
  std::snprintf(hex, sizeof(hex), "k%012llx_pair", static_cast<unsigned long long>(h & 0xffffffffffffULL));
  for (size_t p = rk.source.find(kPlaceholder); p != std::string::npos; p = rk.source.find(kPlaceholder, p))
    rk.source.replace(p, kPlaceholder.size(), hex);
  rk.name = hex;
  rk.kind = "pair";
  rk.block[0] = a.block[0];
  rk.grid[0] = a.grid[0] + b.grid[0];
  return rk;
}

bool kernels_independent(const std::vector<const RenderedKernel*>& kernels,
                         const std::vector<std::vector<BatchArg>>& args, const std::vector<size_t>& a,
                         const std::vector<size_t>& b) {
  auto sets = [&](const std::vector<size_t>& side, std::set<const void*>& reads, std::set<const void*>& writes) {
    for (size_t i : side) {
      FG_CHECK(i < kernels.size() && i < args.size(), "kernels_independent: position out of range");
      const RenderedKernel& m = *kernels[i];
      for (size_t j = 0; j < args[i].size(); j++) {
        if (!args[i][j].id) continue;
        const bool out = j < m.params.size() && m.params[j].first == m.out_slot;
        (out ? writes : reads).insert(args[i][j].id);
        if (out) reads.insert(args[i][j].id);
      }
    }
  };
  std::set<const void*> ra, wa, rb, wb;
  sets(a, ra, wa);
  sets(b, rb, wb);
  for (const void* w : wa)
    if (rb.count(w) || wb.count(w)) return false;
  for (const void* w : wb)
    if (ra.count(w)) return false;
  return true;
}

bool hbatch_member(const RenderedKernel& k) {
  return !k.hbody_fn.empty() && k.launches.empty() && k.scratch_bytes == 0 && k.block[1] == 1 && k.block[2] == 1 &&
         k.grid[1] == 1 && k.grid[2] == 1 && k.block[0] % 64 == 0 && k.block[0] <= static_cast<unsigned>(kBlockThreads);
}

std::vector<HBatchRun> hbatch_runs(const std::vector<const RenderedKernel*>& kernels,
                                   const std::vector<std::vector<BatchArg>>& args,
                                   const std::vector<std::pair<size_t, size_t>>& groups,
                                   const std::vector<size_t>& pair_firsts, size_t extra) {
  FG_CHECK(kernels.size() == args.size(), "hbatch_runs: one argument list per kernel");
  const size_t n = kernels.size();
  // The sequence's launch units in order: (first, count, group index or -1).
  struct Unit {
    size_t first, count;
    long group;
  };
  std::vector<Unit> units;
  for (size_t i = 0; i < n;) {
    long g = -1;
    for (size_t k = 0; k < groups.size(); k++)
      if (groups[k].first == i) g = static_cast<long>(k);
    if (g >= 0) {
      units.push_back({i, groups[g].second, g});
      i += groups[g].second;
    } else if (std::find(pair_firsts.begin(), pair_firsts.end(), i) != pair_firsts.end() && i + 1 < n) {
      units.push_back({i, 2, -1});
      i += 2;
    } else {
      units.push_back({i, 1, -1});
      i++;
    }
  }
  auto hb_unit = [&](const Unit& u) {
    if (u.group >= 0) return false;
    for (size_t j = u.first; j < u.first + u.count; j++)
      if (!hbatch_member(*kernels[j])) return false;
    return true;
  };
  auto nargs = [&](const Unit& u) {
    size_t t = 0;
    for (size_t j = u.first; j < u.first + u.count; j++) t += args[j].size();
    return t;
  };
  std::vector<bool> used(units.size(), false);
  std::vector<HBatchRun> out;
  for (size_t u = 0; u < units.size(); u++) {
    if (units[u].group < 0) continue;
    for (long d : {-1L, 1L}) {
      const long v = static_cast<long>(u) + d;
      if (v < 0 || v >= static_cast<long>(units.size()) || used[v] || !hb_unit(units[v])) continue;
      if (nargs(units[u]) + nargs(units[v]) + extra > FG_MAX_LAUNCH_ARGS) continue;
      std::vector<size_t> hb, st;
      for (size_t j = units[v].first; j < units[v].first + units[v].count; j++) hb.push_back(j);
      for (size_t j = units[u].first; j < units[u].first + units[u].count; j++) st.push_back(j);
      if (!kernels_independent(kernels, args, hb, st)) continue;
      used[u] = used[v] = true;
      out.push_back({hb, static_cast<size_t>(units[u].group)});
      break;
    }
  }
  std::sort(out.begin(), out.end(),
            [](const HBatchRun& a, const HBatchRun& b) { return a.hb.front() < b.hb.front(); });
  return out;
}

std::vector<size_t> pair_runs(const std::vector<const RenderedKernel*>& kernels,
                              const std::vector<std::vector<BatchArg>>& args, const std::vector<bool>& excluded) {
  FG_CHECK(kernels.size() == args.size() && kernels.size() == excluded.size(), "pair_runs: one entry per kernel");
  const size_t n = kernels.size();
  auto pairable = [&](size_t i) {
    const RenderedKernel& m = *kernels[i];
    return !excluded[i] && !m.hbody_fn.empty() && m.launches.empty() && m.scratch_bytes == 0;
  };
  auto sets = [&](size_t i, std::set<const void*>& reads, std::set<const void*>& writes) {
    const RenderedKernel& m = *kernels[i];
    for (size_t j = 0; j < args[i].size(); j++) {
      if (!args[i][j].id) continue;
      const bool out = j < m.params.size() && m.params[j].first == m.out_slot;
      (out ? writes : reads).insert(args[i][j].id);
      if (out) reads.insert(args[i][j].id);
    }
  };
  std::vector<size_t> firsts;
  for (size_t i = 0; i + 1 < n; i++) {
    if (!pairable(i) || !pairable(i + 1)) continue;
    const RenderedKernel &a = *kernels[i], &b = *kernels[i + 1];
    if (a.block[0] != b.block[0] || args[i].size() + args[i + 1].size() > FG_MAX_LAUNCH_ARGS) continue;
    std::set<const void*> ra, wa, rb, wb;
    sets(i, ra, wa);
    sets(i + 1, rb, wb);
    bool indep = true;
    for (const void* w : wa) indep = indep && !rb.count(w) && !wb.count(w);
    for (const void* w : wb) indep = indep && !ra.count(w);
    if (!indep) continue;
    firsts.push_back(i);
    i++;
  }
  return firsts;
}

BatchForwarding batch_forwarding(const std::vector<const RenderedKernel*>& stages,
                                 const std::vector<std::vector<BatchArg>>& args) {
  FG_CHECK(stages.size() == args.size(), "batch_forwarding: one argument list per stage");
  BatchForwarding f;
  auto out_param = [&](size_t j, size_t q) {
    const RenderedKernel& m = *stages[j];
    return q < m.params.size() && m.params[q].first == m.out_slot && args[j][q].id;
  };
  std::map<const void*, int> writers;
  for (size_t j = 0; j < stages.size(); j++)
    for (size_t q = 0; q < args[j].size(); q++)
      if (out_param(j, q)) writers[args[j][q].id]++;
  std::map<const void*, int> lds;  // buffer -> its LDS array, once its writer has run
  size_t bytes = 0;
  for (size_t j = 0; j < stages.size(); j++) {
    const RenderedKernel& m = *stages[j];
    const size_t base = f.arg_buffer.size();
    f.arg_buffer.resize(base + args[j].size(), -1);
    for (size_t q = 0; q < args[j].size(); q++) {
      auto it = args[j][q].id ? lds.find(args[j][q].id) : lds.end();
      if (it != lds.end()) f.arg_buffer[base + q] = it->second;
    }
    for (size_t q = 0; q < args[j].size(); q++) {
      if (!out_param(j, q)) continue;
      const DType dt = m.params[q].second;
      const size_t numel = args[j][q].numel, sz = numel * dt.size_bytes();
      const bool kind_ok = dt == DType::F32() || dt == DType::I32() || dt == DType::Bool();
      if (writers[args[j][q].id] != 1 || m.reads_output || m.out_count != numel || !kind_ok ||
          bytes + sz > kBatchForwardBytes)
        continue;
      bytes += (sz + 15) / 16 * 16;
      const int k = static_cast<int>(f.dtypes.size());
      f.dtypes.push_back(dt);
      f.numels.push_back(numel);
      f.out_arg.push_back(static_cast<int>(base + q));
      f.arg_buffer[base + q] = k;
      lds[args[j][q].id] = k;
    }
  }
  // Barriers only where a stage depends on one run since the last barrier.
  std::set<const void*> reads, writes;
  std::set<std::string> bodies;
  for (size_t j = 0; j < stages.size(); j++) {
    const RenderedKernel& m = *stages[j];
    std::set<const void*> rj, wj;
    for (size_t q = 0; q < args[j].size(); q++) {
      if (!args[j][q].id) continue;
      const bool out = q < m.params.size() && m.params[q].first == m.out_slot;
      (out ? wj : rj).insert(args[j][q].id);
      if (out && m.reads_output) rj.insert(args[j][q].id);
    }
    bool dep = bodies.count(m.stage_fn) > 0;
    for (const void* x : rj) dep = dep || writes.count(x);
    for (const void* x : wj) dep = dep || writes.count(x) || reads.count(x);
    f.barrier.push_back(j > 0 && dep ? 1 : 0);
    if (j > 0 && dep) {
      reads.clear();
      writes.clear();
      bodies.clear();
    }
    reads.insert(rj.begin(), rj.end());
    writes.insert(wj.begin(), wj.end());
    bodies.insert(m.stage_fn);
  }
  return f;
}

std::vector<std::pair<size_t, size_t>> block_batch_runs(const std::vector<bool>& is_block,
                                                        const std::vector<size_t>& nargs) {
  FG_CHECK(is_block.size() == nargs.size(), "block_batch_runs: one argument count per launch");
  std::vector<std::pair<size_t, size_t>> runs;
  for (size_t i = 0; i < is_block.size();) {
    if (!is_block[i]) {
      i++;
      continue;
    }
    size_t n = 1, total = nargs[i];
    while (i + n < is_block.size() && n < kMaxBatchStages && is_block[i + n] &&
           total + nargs[i + n] <= FG_MAX_LAUNCH_ARGS) {
      total += nargs[i + n];
      n++;
    }
    if (n >= 2) runs.emplace_back(i, n);
    i += n;
  }
  return runs;
}

}  // namespace fg
