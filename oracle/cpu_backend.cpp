// TEST INFRASTRUCTURE — the parity oracle. Only tests/, __graft_entry__.smoke()
// and bench.py's cpu_baseline leg load this library; the product never does.
//
// A CPU device that restates the reference's clang backend
// (src/device/cpu.rs) behind the same Device interface the HIP device
// implements, so one program realises on `cpu` (oracle) and `hip` (product)
// by switching the device, as in the reference:
//   optimize  = upcast -> unroll -> symbolic (src/optimize/mod.rs:116-141,
//               upcast.rs:79-177, unroll.rs:41-119), honouring OPT
//               (mod.rs:85-112)
//   render    = C with one statement per op, the reference's operator
//               spellings and accumulation order (codegen/clang.rs:28-280,
//               expand.rs + devectorize.rs lane semantics: UPCAST lanes get
//               their own accumulators; each REDUCE step folds the UNROLL lanes
//               left to right and adds the group: devectorize.rs:206-214,
//               274-347)
//   compile   = clang -shared -O3 -march=native + dlopen (cpu.rs:151-208)
//   execute   = one call on the calling thread (cpu.rs:328-380)
//
// One deliberate divergence from the reference: when an UNROLL axis id is
// smaller than the UPCAST axis id (a column reduction whose output is
// upcast), devectorize.rs:147-179 groups lanes along the upcast axis instead
// of the unrolled one (it assumes contracted axes are innermost). The oracle
// folds along the unrolled axis, i.e. computes the mathematically defined sum.
#include <dlfcn.h>
#include <unistd.h>

#include <algorithm>
#include <charconv>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <sstream>

#include "device.hpp"
#include "ir.hpp"
#include "schedule.hpp"
#include "tensor.hpp"

namespace fg {
namespace oracle {

// ── OPT parsing (src/optimize/mod.rs:85-112) ────────────────────────────────
struct OptConfig {
  bool symbolic = true, upcast = true, unroll = true;
};

OptConfig parse_opt(const char* raw) {
  OptConfig all;
  if (!raw) return all;
  std::string s(raw);
  auto trim = [](std::string x) {
    size_t a = x.find_first_not_of(" \t\n"), b = x.find_last_not_of(" \t\n");
    return a == std::string::npos ? std::string() : x.substr(a, b - a + 1);
  };
  s = trim(s);
  if (s.empty() || s == "1" || s == "on" || s == "all") return all;
  OptConfig none{false, false, false};
  if (s == "0" || s == "off" || s == "none") return none;
  std::stringstream ss(s);
  std::string item;
  while (std::getline(ss, item, ',')) {
    item = trim(item);
    if (item == "symbolic") none.symbolic = true;
    else if (item == "upcast") none.upcast = true;
    else if (item == "unroll") none.unroll = true;
  }
  return none;
}

bool const_i32(const UOp& n, int64_t* v) {  // optimize/mod.rs:47-52
  if (n.arg().kind != Arg::Kind::Int || n.dtype() != DType::I32()) return false;
  *v = n.arg().a;
  return true;
}

bool range_kind_is(const UOp& n, std::initializer_list<AxisKind> ks) {
  if (n.arg().kind != Arg::Kind::Range) return false;
  for (auto k : ks)
    if (n.arg().range_kind() == k) return true;
  return false;
}

// ── upcast (src/optimize/upcast.rs) ─────────────────────────────────────────
constexpr int64_t kUpcast = 4;

bool has_post_reduce_store_alu(const UOp& root) {  // upcast.rs:67-75
  for (auto& n : root.toposort()) {
    if (n.op() != Op::Store || n.srcs().size() != 2) continue;
    const UOp& v = n.src(1);
    if (v.op() == Op::Reduce) continue;
    for (auto& x : v.toposort())
      if (x.op() == Op::Reduce) return true;
  }
  return false;
}

UOp select_upcast_range(const UOp& root) {  // upcast.rs:79-103
  auto order = root.toposort();
  for (auto& n : order)
    if (range_kind_is(n, {AxisKind::Upcast})) return UOp();
  if (has_post_reduce_store_alu(root)) return UOp();
  std::vector<UOp> rs;
  for (auto& n : order)
    if (range_kind_is(n, {AxisKind::Loop, AxisKind::Global, AxisKind::Local, AxisKind::Thread})) rs.push_back(n);
  std::stable_sort(rs.begin(), rs.end(), [](const UOp& a, const UOp& b) { return a.arg().a < b.arg().a; });
  rs.erase(std::unique(rs.begin(), rs.end()), rs.end());
  if (rs.empty()) return UOp();
  UOp r = rs.back();
  if (r.arg().range_kind() != AxisKind::Loop || r.srcs().size() != 1) return UOp();
  int64_t size;
  if (!const_i32(r.src(0), &size) || size <= kUpcast || size % kUpcast != 0) return UOp();
  return r;
}

UOp upcast_loops(const UOp& root) {  // upcast.rs:108-177
  UOp target = select_upcast_range(root);
  if (!target) return root;
  return graph_rewrite(root, [&](const UOp& end) -> UOp {
    if (end.op() != Op::End || end.srcs().size() < 2 || end.src(0) != target) return UOp();
    const UOp& range = end.src(0);
    int64_t size;
    if (!const_i32(range.src(0), &size) || size <= kUpcast || size % kUpcast != 0) return UOp();
    DeviceId d = range.device();
    int64_t axis = range.arg().a;
    UOp outer = UOp::make_new(Op::Range, DType::I32(), {UOp::const_int(size / kUpcast, DType::I32(), d)},
                              Arg::range(axis, AxisKind::Global));
    UOp inner = UOp::make_new(Op::Range, DType::I32(), {UOp::const_int(kUpcast, DType::I32(), d)},
                              Arg::range(axis, AxisKind::Upcast));
    UOp expanded = UOp::add(UOp::mul(outer, UOp::const_int(kUpcast, DType::I32(), d)), inner);
    UOpMap<UOp> rep{{range, expanded}};
    std::vector<UOp> srcs{inner};
    for (size_t i = 1; i < end.srcs().size(); i++) srcs.push_back(substitute_with_map(end.src(i), rep));
    UOp up = UOp::make_new(Op::End, DType::Void(), srcs, Arg::none());
    return UOp::make_new(Op::End, DType::Void(), {outer, up}, Arg::none());
  });
}

// ── unroll (src/optimize/unroll.rs:41-119) ──────────────────────────────────
constexpr int64_t kUnroll = 4;

UOp split_reduce_unroll(const UOp& reduce) {
  if (reduce.op() != Op::Reduce || reduce.srcs().size() < 2) return UOp();
  for (size_t i = 1; i < reduce.srcs().size(); i++)
    if (range_kind_is(reduce.src(i), {AxisKind::Unroll})) return UOp();
  size_t idx = 0;
  for (size_t i = reduce.srcs().size(); i-- > 1;)
    if (range_kind_is(reduce.src(i), {AxisKind::Reduce})) {
      idx = i;
      break;
    }
  if (idx == 0) return UOp();
  const UOp& range = reduce.src(idx);
  if (range.srcs().size() != 1) return UOp();
  int64_t size;
  if (!const_i32(range.src(0), &size) || size <= kUnroll || size % kUnroll != 0) return UOp();
  DeviceId d = range.device();
  int64_t axis = range.arg().a;
  UOp outer = UOp::make_new(Op::Range, DType::I32(), {UOp::const_int(size / kUnroll, DType::I32(), d)},
                            Arg::range(axis, AxisKind::Reduce));
  UOp inner = UOp::make_new(Op::Range, DType::I32(), {UOp::const_int(kUnroll, DType::I32(), d)},
                            Arg::range(axis, AxisKind::Unroll));
  UOp expanded = UOp::add(UOp::mul(outer, UOp::const_int(kUnroll, DType::I32(), d)), inner);
  UOp value = substitute_with_map(reduce.src(0), UOpMap<UOp>{{range, expanded}});
  std::vector<UOp> srcs{value};
  for (size_t i = 1; i < reduce.srcs().size(); i++) {
    if (i == idx) {
      srcs.push_back(outer);
      srcs.push_back(inner);
    } else {
      srcs.push_back(reduce.src(i));
    }
  }
  return UOp::make_new(Op::Reduce, reduce.dtype(), srcs, reduce.arg());
}

UOp reference_optimize(const UOp& kernel, const OptConfig& cfg) {  // optimize/mod.rs:125-141
  UOp cur = kernel;
  if (cfg.upcast) cur = upcast_loops(cur);
  if (cfg.unroll) cur = graph_rewrite(cur, split_reduce_unroll);
  if (cfg.symbolic) cur = graph_rewrite(cur, symbolic_simple);
  return cur;
}

// ── C emitter ───────────────────────────────────────────────────────────────
// Renders the optimized kernel as scalar C. Lanes: an UPCAST range contributes
// output lanes (each with its own statements and accumulators); an UNROLL range
// contributes the lanes folded per reduction step.

// Float literals as the reference prints them (clang.rs:93-115): shortest
// round-trip decimal of the f64 value with an `f` suffix for f32.
std::string c_float(double v, DType dt) {
  if (std::isinf(v)) return v > 0 ? "INFINITY" : "(-INFINITY)";
  if (std::isnan(v)) return "NAN";
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof(buf), v);
  std::string s(buf, r.ptr);
  if (s.find_first_of(".eE") == std::string::npos) s += ".0";
  if (dt.kind == DTypeKind::F32) s += "f";
  return s;
}

std::string c_const(const UOp& c) {
  const Arg& a = c.arg();
  switch (a.kind) {
    case Arg::Kind::Float: return c_float(a.f, c.dtype());
    case Arg::Kind::Int: return std::to_string(a.a);
    case Arg::Kind::Bool: return a.a ? "1" : "0";
    default: fail("Const with unexpected arg");
  }
}

struct CEmit {
  std::ostringstream out;
  int depth = 1;
  int val_count = 0, alu_count = 0;
  UOp up_range, un_range;  // active lane ranges
  // cache: (node, up lane or -1, unroll lane or -1) -> C name
  std::map<std::tuple<const UOpInner*, int, int>, std::string> cache;
  std::map<const UOpInner*, std::string> loop_var;
  std::map<std::pair<const UOpInner*, const UOpInner*>, bool> dep;

  std::string ind() const { return std::string(static_cast<size_t>(depth) * 2, ' '); }

  bool depends(const UOp& n, const UOp& r) {
    if (!r) return false;
    auto k = std::make_pair(n.get(), r.get());
    auto it = dep.find(k);
    if (it != dep.end()) return it->second;
    bool d = n == r;
    for (auto& s : n.srcs())
      if (!d && depends(s, r)) d = true;
    dep[k] = d;
    return d;
  }

  std::string idx(const UOp& e, int ul, int nl) {
    switch (e.op()) {
      case Op::Const: return c_const(e);
      case Op::ParamScalar: return "data" + std::to_string(e.arg().a);
      case Op::Range: {
        if (e == up_range) return std::to_string(ul);
        if (e == un_range) return std::to_string(nl);
        auto it = loop_var.find(e.get());
        FG_CHECK(it != loop_var.end(), "oracle: range used outside its loop");
        return it->second;
      }
      case Op::Add: return "(" + idx(e.src(0), ul, nl) + "+" + idx(e.src(1), ul, nl) + ")";
      case Op::Mul: return "(" + idx(e.src(0), ul, nl) + "*" + idx(e.src(1), ul, nl) + ")";
      default: return val(e, ul, nl);
    }
  }

  std::string val(const UOp& n, int ul, int nl) {
    int ku = depends(n, up_range) ? ul : -1;
    int kn = depends(n, un_range) ? nl : -1;
    auto key = std::make_tuple(n.get(), ku, kn);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    std::string name;
    switch (n.op()) {
      case Op::Const: return c_const(n);
      case Op::ParamScalar: return "data" + std::to_string(n.arg().a);
      case Op::Range: return idx(n, ul, nl);
      case Op::Load: {
        const UOp& ix = n.src(0);
        std::string addr = "(data" + std::to_string(ix.src(0).arg().a) + "+" + idx(ix.src(1), ul, nl) + ")";
        name = "val" + std::to_string(val_count++);
        out << ind() << n.dtype().c_type() << " " << name << " = *" << addr << ";\n";
        break;
      }
      case Op::Reduce:
        name = reduce(n, ul);
        break;
      default: {
        if ((n.op() == Op::Add || n.op() == Op::Mul) && n.dtype().kind == DTypeKind::I32 && is_index(n))
          return idx(n, ul, nl);
        std::vector<std::string> s;
        for (auto& x : n.srcs()) s.push_back(val(x, ul, nl));
        std::string e;
        switch (n.op()) {  // clang.rs:216-227
          case Op::Neg: e = "(-" + s[0] + ")"; break;
          case Op::Exp2: e = "exp2(" + s[0] + ")"; break;
          case Op::Log2: e = "log2(" + s[0] + ")"; break;
          case Op::Sqrt: e = "__builtin_sqrtf(" + s[0] + ")"; break;
          case Op::Reciprocal: e = "(1/" + s[0] + ")"; break;
          case Op::Add: e = "(" + s[0] + "+" + s[1] + ")"; break;
          case Op::Mul: e = "(" + s[0] + "*" + s[1] + ")"; break;
          case Op::Max: e = "((" + s[0] + ">" + s[1] + ")?" + s[0] + ":" + s[1] + ")"; break;
          case Op::CmpLt: e = "(" + s[0] + "<" + s[1] + ")"; break;
          case Op::Where: e = "(" + s[0] + "?" + s[1] + ":" + s[2] + ")"; break;
          default: fail(std::string("oracle cannot render ") + op_name(n.op()));
        }
        name = "alu" + std::to_string(alu_count++);
        out << ind() << n.dtype().c_type() << " " << name << " = " << e << ";\n";
      }
    }
    cache[key] = name;
    return name;
  }

  static bool is_index(const UOp& n) {
    if (n.op() == Op::Range || n.op() == Op::Const || n.op() == Op::ParamScalar) return true;
    if (n.op() == Op::Add || n.op() == Op::Mul) return is_index(n.src(0)) && is_index(n.src(1));
    return false;
  }

  // Reduce lowering for one output lane (devectorize.rs:274-347): accumulator
  // init, loops over the REDUCE ranges in source order, and per step
  // acc = acc op (((v0 op v1) op v2) op v3) over the UNROLL lanes.
  std::string reduce(const UOp& R, int ul) {
    std::vector<int> lanes{ul};
    return reduce_lanes(R, lanes)[0];
  }

  // One reduction loop nest computing the accumulators of several UPCAST
  // lanes together (one accumulator per lane, as devectorize.rs:289-322).
  std::vector<std::string> reduce_lanes(const UOp& R, const std::vector<int>& uls) {
    Op rop = R.arg().rop;
    std::string init = rop == Op::Add ? c_float(0.0, R.dtype()) : "(-INFINITY)";
    if (R.dtype().kind != DTypeKind::F32) init = rop == Op::Add ? "0" : "(-2147483647-1)";
    std::vector<std::string> accs;
    for (size_t i = 0; i < uls.size(); i++) {
      accs.push_back("acc" + std::to_string(alu_count++));
      out << ind() << R.dtype().c_type() << " " << accs.back() << " = " << init << ";\n";
    }
    UOp unr;
    std::vector<UOp> loops;
    for (size_t i = 1; i < R.srcs().size(); i++) {
      const UOp& r = R.src(i);
      if (range_kind_is(r, {AxisKind::Unroll})) unr = r;
      else loops.push_back(r);
    }
    auto saved = cache;
    for (auto& r : loops) {
      std::string v = "ridx" + std::to_string(r.arg().a);
      if (loop_var.count(r.get())) v += "_" + std::to_string(depth);
      out << ind() << "for (int " << v << " = 0; " << v << " < " << idx(r.src(0), uls[0], 0) << "; " << v
          << "++) {\n";
      loop_var[r.get()] = v;
      depth++;
    }
    for (size_t li = 0; li < uls.size(); li++) {
      int ul = uls[li];
      UOp prev_un = un_range;
      std::string group;
      if (unr) {
        un_range = unr;
        int64_t n;
        FG_CHECK(const_i32(unr.src(0), &n), "unroll range must have a constant bound");
        std::vector<std::string> lanes;
        for (int64_t u = 0; u < n; u++) lanes.push_back(val(R.src(0), ul, static_cast<int>(u)));
        // horizontal_reduce: one node per fold step, left to right.
        group = lanes[0];
        for (size_t u = 1; u < lanes.size(); u++) {
          std::string g = "alu" + std::to_string(alu_count++);
          out << ind() << R.dtype().c_type() << " " << g << " = " << combine(rop, group, lanes[u]) << ";\n";
          group = g;
        }
      } else {
        group = val(R.src(0), ul, -1);
      }
      un_range = prev_un;
      std::string upd = "alu" + std::to_string(alu_count++);
      out << ind() << R.dtype().c_type() << " " << upd << " = " << combine(rop, accs[li], group) << ";\n";
      out << ind() << accs[li] << " = " << upd << ";\n";
    }
    for (size_t i = 0; i < loops.size(); i++) {
      depth--;
      out << ind() << "}\n";
      loop_var.erase(loops[loops.size() - 1 - i].get());
    }
    cache = saved;  // values computed inside the loops are out of scope now
    return accs;
  }

  static std::string combine(Op rop, const std::string& a, const std::string& b) {
    if (rop == Op::Add) return "(" + a + "+" + b + ")";
    return "((" + a + ">" + b + ")?" + a + ":" + b + ")";
  }

  // Effects: End chains and Stores.
  void effect(const UOp& e, int ul) {
    if (e.op() == Op::Sink) {
      for (auto& s : e.srcs()) effect(s, ul);
      return;
    }
    if (e.op() == Op::End) {
      const UOp& r = e.src(0);
      if (range_kind_is(r, {AxisKind::Upcast})) {
        int64_t n;
        FG_CHECK(const_i32(r.src(0), &n), "upcast range must have a constant bound");
        UOp prev = up_range;
        up_range = r;
        // Reductions feeding the lanes share one loop nest with one
        // accumulator per lane.
        std::vector<int> uls;
        for (int64_t u = 0; u < n; u++) uls.push_back(static_cast<int>(u));
        for (size_t i = 1; i < e.srcs().size(); i++) {
          for (auto& x : e.src(i).toposort()) {
            if (x.op() != Op::Reduce || !depends(x, r)) continue;
            if (cache.count(std::make_tuple(x.get(), 0, -1))) continue;
            auto accs = reduce_lanes(x, uls);
            for (size_t u = 0; u < uls.size(); u++) cache[std::make_tuple(x.get(), uls[u], -1)] = accs[u];
          }
        }
        for (int64_t u = 0; u < n; u++)
          for (size_t i = 1; i < e.srcs().size(); i++) effect(e.src(i), static_cast<int>(u));
        up_range = prev;
        return;
      }
      std::string v = (range_kind_is(r, {AxisKind::Reduce, AxisKind::GroupReduce}) ? "ridx" : "idx") +
                      std::to_string(r.arg().a);
      out << ind() << "for (int " << v << " = 0; " << v << " < " << idx(r.src(0), ul, -1) << "; " << v << "++) {\n";
      loop_var[r.get()] = v;
      depth++;
      auto saved = cache;
      for (size_t i = 1; i < e.srcs().size(); i++) effect(e.src(i), ul);
      cache = saved;
      depth--;
      out << ind() << "}\n";
      loop_var.erase(r.get());
      return;
    }
    FG_CHECK(e.op() == Op::Store, std::string("oracle: unexpected effect ") + op_name(e.op()));
    const UOp& ix = e.src(0);
    std::string v = val(e.src(1), ul, -1);
    out << ind() << "*(data" << ix.src(0).arg().a << "+" << idx(ix.src(1), ul, -1) << ") = " << v << ";\n";
  }
};

struct CParam {
  int slot;
  DType dtype;
  bool buffer;
};

std::vector<CParam> collect_params(const UOp& sink) {
  std::map<int, CParam> ps;
  for (auto& n : sink.toposort()) {
    if (n.op() == Op::ParamBuffer) ps[static_cast<int>(n.arg().a)] = {static_cast<int>(n.arg().a), n.dtype(), true};
    if (n.op() == Op::ParamScalar) ps[static_cast<int>(n.arg().a)] = {static_cast<int>(n.arg().a), n.dtype(), false};
  }
  std::vector<CParam> out;
  for (auto& kv : ps) out.push_back(kv.second);
  return out;
}

std::string render_c(const UOp& sink, const std::string& name) {
  auto params = collect_params(sink);
  std::ostringstream src;
  src << "#include <math.h>\nvoid " << name << "(";
  for (size_t i = 0; i < params.size(); i++) {
    if (i) src << ", ";
    if (params[i].buffer) src << params[i].dtype.c_type() << "* restrict data" << params[i].slot;
    else src << params[i].dtype.c_type() << " data" << params[i].slot;
  }
  src << ") {\n";
  CEmit em;
  em.effect(sink, -1);
  src << em.out.str() << "}\n";
  // Uniform entry point: the reference marshals through libffi (cpu.rs:338-377).
  src << "void " << name << "__entry(void** a) {\n  " << name << "(";
  for (size_t i = 0; i < params.size(); i++) {
    if (i) src << ", ";
    if (params[i].buffer) src << "(" << params[i].dtype.c_type() << "*)a[" << i << "]";
    else src << "*(" << params[i].dtype.c_type() << "*)a[" << i << "]";
  }
  src << ");\n}\n";
  return src.str();
}

// ── compile (cpu.rs:151-208) ────────────────────────────────────────────────
struct CpuProgram : Program {
  void* lib = nullptr;
  void (*entry)(void**) = nullptr;
  ~CpuProgram() override {
    if (lib) dlclose(lib);
  }
};

std::string run_clang(const std::string& source, std::string* so_path) {
  char cdir[] = "/tmp/fg_oracle_XXXXXX";
  FG_CHECK(mkdtemp(cdir) != nullptr, "failed to create temp dir");
  std::string dir = cdir;
  std::string c = dir + "/k.c", so = dir + "/k.so", log = dir + "/log.txt";
  {
    std::ofstream f(c);
    f << source;
  }
  const char* cc = std::getenv("FG_ORACLE_CC");
  std::string clang = cc ? cc : "clang";
  std::string cmd = clang + " -shared -fPIC -O3 -march=native -o " + so + " " + c + " -lm > " + log + " 2>&1";
  int rc = std::system(cmd.c_str());
  std::ifstream lf(log);
  std::stringstream ls;
  ls << lf.rdbuf();
  *so_path = so;
  if (rc != 0) return "clang compilation failed:\n" + ls.str();
  return "";
}

class CpuDevice : public Device {
 public:
  DeviceId id() const override { return DeviceId::Cpu; }

  // Off by default: the reference's kernel partition. On, the CPU device
  // runs the HIP device's value-preserving fusions (schedule.cpp), so a test
  // can compare the fused and the reference partition on one device, where
  // every kernel keeps the reference's lowering and accumulation order.
  bool fuse = false;
  bool fuse_elementwise() const override { return fuse; }
  // Test-only: skip kernel execution, so a host-side profile of the front end
  // (graph building, scheduling, plan replay) is not buried under the
  // kernels' CPU time. Results are then meaningless.
  bool dry_run = false;

  Buffer allocate(DType dtype, size_t numel) override {  // cpu.rs:277-280
    Buffer b = reserve_buffer(dtype, numel);
    realize_storage(*b, true);
    b->known_zero = true;
    return b;
  }

  void realize_storage(BufferInner& b, bool zero) override {
    if (b.realized) return;
    size_t n = std::max<size_t>(b.nbytes(), 1);
    b.storage = zero ? std::calloc(1, n) : std::malloc(n);
    FG_CHECK(b.storage != nullptr, "oracle: host allocation failed");
    b.realized = true;
  }

  void release(BufferInner& b) override {
    std::free(b.storage);
    b.storage = nullptr;
    b.realized = false;
  }

  void copy_from_host(const Buffer& b, const void* src, size_t nbytes) override {  // cpu.rs:282-302
    FG_CHECK(b->device == DeviceId::Cpu, "CPU backend received non-CPU buffer " + std::to_string(b->id));
    b->ensure_allocated();
    FG_CHECK(nbytes == b->nbytes(),
             "copy_from_host: expected " + std::to_string(b->nbytes()) + " bytes, got " + std::to_string(nbytes));
    if (nbytes) std::memcpy(b->storage, src, nbytes);
    b->known_zero = false;
  }

  std::vector<uint8_t> copy_to_host(const Buffer& b) override {  // cpu.rs:304-316
    FG_CHECK(b->device == DeviceId::Cpu, "CPU backend received non-CPU buffer " + std::to_string(b->id));
    FG_CHECK(b->realized, "copy_to_host called on unrealized or non-CPU buffer");
    std::vector<uint8_t> out(b->nbytes());
    if (!out.empty()) std::memcpy(out.data(), b->storage, out.size());
    return out;
  }

  UOp optimize(const UOp& rangeified) override {
    return reference_optimize(rangeified, parse_opt(std::getenv("OPT")));
  }

  RenderedKernel render(const UOp& optimized, const std::string& name) override {
    RenderedKernel rk;
    rk.name = name;
    rk.kind = "clang";
    rk.source = render_c(optimized, name);
    return rk;
  }

  std::shared_ptr<Program> compile(const RenderedKernel& rk, size_t num_args) override {
    std::string so;
    std::string err = run_clang(rk.source, &so);
    FG_CHECK(err.empty(), "compile failed: " + err);
    auto p = std::make_shared<CpuProgram>();
    p->lib = dlopen(so.c_str(), RTLD_NOW | RTLD_LOCAL);
    FG_CHECK(p->lib != nullptr, std::string("failed to load shared library: ") + dlerror());
    p->entry = reinterpret_cast<void (*)(void**)>(dlsym(p->lib, (rk.name + "__entry").c_str()));
    FG_CHECK(p->entry != nullptr, "symbol '" + rk.name + "' not found");
    p->num_args = num_args;
    p->meta = rk;
    return p;
  }

  void execute(Program& prog, std::vector<KernelArg>& args) override {  // cpu.rs:328-380
    auto& p = static_cast<CpuProgram&>(prog);
    FG_CHECK(args.size() == p.num_args,
             "expected " + std::to_string(p.num_args) + " kernel args, got " + std::to_string(args.size()));
    std::vector<void*> ptrs(args.size());
    std::vector<int32_t> ints(args.size());
    std::vector<float> flts(args.size());
    std::vector<uint8_t> bools(args.size());
    for (size_t i = 0; i < args.size(); i++) {
      switch (args[i].kind) {
        case KernelArg::Kind::Buffer:
          FG_CHECK(args[i].buffer->device == DeviceId::Cpu && args[i].buffer->realized,
                   "CPU backend received unrealized or non-CPU buffer");
          ptrs[i] = args[i].buffer->storage;
          break;
        case KernelArg::Kind::I32: ints[i] = args[i].i; ptrs[i] = &ints[i]; break;
        case KernelArg::Kind::F32: flts[i] = args[i].f; ptrs[i] = &flts[i]; break;
        case KernelArg::Kind::Bool: bools[i] = args[i].b ? 1 : 0; ptrs[i] = &bools[i]; break;
      }
    }
    if (!dry_run) p.entry(ptrs.data());
  }
};

}  // namespace oracle
}  // namespace fg

extern "C" {

static fg::oracle::CpuDevice* g_cpu_device = nullptr;

// Register the oracle CPU device as device 0 ("cpu").
int fg_oracle_register(void) {
  if (!g_cpu_device) {
    g_cpu_device = new fg::oracle::CpuDevice();
    fg::register_device(fg::DeviceId::Cpu, g_cpu_device);
  }
  return 0;
}

// Skip (1) or run (0) kernels on the CPU device: for host-side profiling of
// the front end only. Returns the previous setting.
int fg_oracle_set_dry_run(int on) {
  fg_oracle_register();
  int prev = g_cpu_device->dry_run ? 1 : 0;
  g_cpu_device->dry_run = on != 0;
  return prev;
}

// Schedule the CPU device's realisations with (1) or without (0) the HIP
// device's fusions; returns the previous setting.
int fg_oracle_set_fuse(int on) {
  fg_oracle_register();
  int prev = g_cpu_device->fuse ? 1 : 0;
  g_cpu_device->fuse = on != 0;
  return prev;
}

}  // extern "C"

// Same layout as the front end's handle (ferrograd_amd/csrc/capi.cpp).
struct fg_tensor {
  fg::Tensor t;
};

extern "C" {

// Schedule `roots` with the reference's rules (no fusion) and return, as JSON,
// the oracle C source of every kernel: {"kernels": ["...", ...]}. Two calls:
// buf == NULL plans and reports the size; a second call copies the result.
int fg_oracle_plan_c(fg_tensor** roots, int n, char* buf, size_t len, size_t* needed) {
  static std::string last;
  if (buf) {
    size_t m = len ? std::min(len - 1, last.size()) : 0;
    if (len) {
      std::memcpy(buf, last.data(), m);
      buf[m] = '\0';
    }
    if (needed) *needed = last.size() + 1;
    return 0;
  }
  try {
    std::vector<fg::UOp> rs;
    fg::UOpSet seen;
    for (int i = 0; i < n; i++) {
      if (roots[i]->t.is_realized()) continue;
      fg::UOp u = roots[i]->t.uop();
      if (seen.insert(u).second) rs.push_back(u);
    }
    std::ostringstream os;
    os << "{\"kernels\": [";
    if (!rs.empty()) {
      auto plan = fg::schedule_many(rs, fg::ScheduleOptions{});
      for (size_t i = 0; i < plan.items.size(); i++) {
        fg::UOp k = fg::oracle::reference_optimize(fg::rangeify(plan.items[i].sink),
                                                   fg::oracle::parse_opt(std::getenv("OPT")));
        std::string src = fg::oracle::render_c(k, "kernel_" + std::to_string(i));
        os << (i ? ", " : "") << "\"";
        for (char c : src) {
          if (c == '"') os << "\\\"";
          else if (c == '\\') os << "\\\\";
          else if (c == '\n') os << "\\n";
          else os << c;
        }
        os << "\"";
      }
    }
    os << "]}";
    last = os.str();
    if (needed) *needed = last.size() + 1;
    return 0;
  } catch (const std::exception& e) {
    last = std::string("{\"error\": \"") + e.what() + "\"}";
    if (needed) *needed = last.size() + 1;
    return 1;
  }
}

}  // extern "C"
