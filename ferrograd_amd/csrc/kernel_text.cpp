// Text form of a rangeified kernel (the format is described in kernel_text.hpp).
#include "kernel_text.hpp"

#include <cerrno>
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <unordered_map>

namespace fg {

namespace {

constexpr const char* kHeader = "fg-kernel 1";
constexpr int kNumOps = static_cast<int>(Op::Gep) + 1;
constexpr int kNumAxisKinds = static_cast<int>(AxisKind::Thread) + 1;

std::string join(const std::vector<int64_t>& v) {
  std::string s;
  for (size_t i = 0; i < v.size(); i++) s += (i ? "," : "") + std::to_string(v[i]);
  return s;
}

std::string arg_text(const Arg& a) {
  switch (a.kind) {
    case Arg::Kind::None: return "-";
    case Arg::Kind::Device: return std::string("device:") + device_name(static_cast<DeviceId>(a.a));
    case Arg::Kind::Int: return "int:" + std::to_string(a.a);
    case Arg::Kind::Bool: return std::string("bool:") + (a.a ? "1" : "0");
    case Arg::Kind::Float: {
      uint64_t bits;
      std::memcpy(&bits, &a.f, 8);
      char buf[32];
      std::snprintf(buf, sizeof(buf), "float:%016" PRIx64, bits);
      return buf;
    }
    case Arg::Kind::Range:
      return "range:" + std::to_string(a.a) + ":" + axis_kind_name(static_cast<AxisKind>(a.b));
    case Arg::Kind::ParamBuffer: return "param:" + std::to_string(a.a) + ":" + std::to_string(a.b);
    case Arg::Kind::ParamScalar: return "scalar:" + std::to_string(a.a);
    case Arg::Kind::Index: return "index:" + std::to_string(a.a);
    case Arg::Kind::Reduce: return std::string("reduce:") + op_name(a.rop) + ":" + join(a.v);
    case Arg::Kind::Axes: return "axes:" + join(a.v);
    case Arg::Kind::Shape: return "shape:" + join(a.v);
    case Arg::Kind::Bounds: return "bounds:" + join(a.v);
    case Arg::Kind::Lanes: return "lanes:" + join(a.v);
    case Arg::Kind::Variable:
      FG_CHECK(a.name.find_first_of(": \t\n") == std::string::npos,
               "kernel_to_text: variable name '" + a.name + "' holds a separator");
      return "var:" + a.name + ":" + std::to_string(a.b) + ":" + std::to_string(a.c);
    case Arg::Kind::Buffer:
      fail("kernel_to_text: the kernel still holds a device Buffer; kernels refer to memory by ParamBuffer slot");
  }
  fail("kernel_to_text: unknown arg kind");
}

[[noreturn]] void bad(size_t line, const std::string& what) {
  fail("fg-kernel text line " + std::to_string(line) + ": " + what);
}

bool parse_i64(const std::string& s, int64_t* out) {
  if (s.empty()) return false;
  char* end = nullptr;
  errno = 0;
  long long v = std::strtoll(s.c_str(), &end, 10);
  if (errno != 0 || *end != '\0') return false;
  *out = v;
  return true;
}

std::vector<std::string> split(const std::string& s, char sep) {
  std::vector<std::string> out;
  size_t p = 0;
  while (true) {
    size_t q = s.find(sep, p);
    out.push_back(s.substr(p, q == std::string::npos ? std::string::npos : q - p));
    if (q == std::string::npos) return out;
    p = q + 1;
  }
}

std::vector<int64_t> parse_list(const std::string& s, size_t line) {
  std::vector<int64_t> v;
  if (s.empty()) return v;
  for (auto& tok : split(s, ',')) {
    int64_t x;
    if (!parse_i64(tok, &x)) bad(line, "bad integer '" + tok + "' in list '" + s + "'");
    v.push_back(x);
  }
  return v;
}

bool parse_op(const std::string& s, Op* op) {
  for (int i = 0; i < kNumOps; i++)
    if (s == op_name(static_cast<Op>(i))) {
      *op = static_cast<Op>(i);
      return true;
    }
  return false;
}

DType parse_dtype(const std::string& s, size_t line) {
  std::string base = s;
  uint16_t lanes = 1;
  size_t x = s.find('x');
  if (x != std::string::npos) {
    int64_t n;
    if (!parse_i64(s.substr(x + 1), &n) || n < 1 || n > 65535) bad(line, "bad vector width in dtype '" + s + "'");
    base = s.substr(0, x);
    lanes = static_cast<uint16_t>(n);
  }
  DTypeKind k;
  if (base == "f32") k = DTypeKind::F32;
  else if (base == "i32") k = DTypeKind::I32;
  else if (base == "bool") k = DTypeKind::Bool;
  else if (base == "void") k = DTypeKind::Void;
  else bad(line, "unknown dtype '" + s + "'");
  return DType(k, lanes);
}

Arg parse_arg(const std::string& s, size_t line) {
  if (s == "-") return Arg::none();
  size_t c = s.find(':');
  if (c == std::string::npos) bad(line, "bad arg '" + s + "'");
  const std::string kind = s.substr(0, c), rest = s.substr(c + 1);
  auto fields = split(rest, ':');
  auto need = [&](size_t n) {
    if (fields.size() != n) bad(line, "arg '" + s + "' needs " + std::to_string(n) + " fields");
  };
  auto i64 = [&](const std::string& f) {
    int64_t v;
    if (!parse_i64(f, &v)) bad(line, "bad integer '" + f + "' in arg '" + s + "'");
    return v;
  };
  if (kind == "device") {
    need(1);
    if (rest == "hip") return Arg::device(DeviceId::Hip);
    if (rest == "cpu") return Arg::device(DeviceId::Cpu);
    bad(line, "unknown device '" + rest + "'");
  }
  if (kind == "int") { need(1); return Arg::integer(i64(rest)); }
  if (kind == "bool") {
    need(1);
    if (rest != "0" && rest != "1") bad(line, "bad bool '" + rest + "'");
    return Arg::boolean(rest == "1");
  }
  if (kind == "float") {
    need(1);
    if (rest.size() != 16 || rest.find_first_not_of("0123456789abcdefABCDEF") != std::string::npos)
      bad(line, "float arg needs 16 hex digits, got '" + rest + "'");
    uint64_t bits = std::strtoull(rest.c_str(), nullptr, 16);
    double f;
    std::memcpy(&f, &bits, 8);
    return Arg::flt(f);
  }
  if (kind == "range") {
    need(2);
    for (int k = 0; k < kNumAxisKinds; k++)
      if (fields[1] == axis_kind_name(static_cast<AxisKind>(k))) return Arg::range(i64(fields[0]), static_cast<AxisKind>(k));
    bad(line, "unknown axis kind '" + fields[1] + "'");
  }
  if (kind == "param") { need(2); return Arg::param_buffer(i64(fields[0]), i64(fields[1])); }
  if (kind == "scalar") { need(1); return Arg::param_scalar(i64(rest)); }
  if (kind == "index") { need(1); return Arg::index(i64(rest)); }
  if (kind == "reduce") {
    need(2);
    Op rop;
    if (!parse_op(fields[0], &rop)) bad(line, "unknown reduce op '" + fields[0] + "'");
    Arg a = Arg::reduce(rop, {});
    a.v = parse_list(fields[1], line);
    return a;
  }
  if (kind == "axes" || kind == "shape" || kind == "bounds" || kind == "lanes") {
    need(1);
    Arg a;
    a.kind = kind == "axes" ? Arg::Kind::Axes : kind == "shape" ? Arg::Kind::Shape
             : kind == "bounds" ? Arg::Kind::Bounds : Arg::Kind::Lanes;
    a.v = parse_list(rest, line);
    if (a.kind == Arg::Kind::Lanes && a.v.size() % 2) bad(line, "lanes need pairs");
    return a;
  }
  if (kind == "var") {
    need(3);
    Arg a;
    a.kind = Arg::Kind::Variable;
    a.name = fields[0];
    a.b = i64(fields[1]);
    a.c = i64(fields[2]);
    return a;
  }
  bad(line, "unknown arg kind '" + kind + "'");
}

}  // namespace

std::string kernel_to_text(const UOp& sink) {
  auto order = sink.toposort();
  std::unordered_map<const void*, size_t> id;
  std::ostringstream os;
  os << kHeader << "\n";
  for (size_t i = 0; i < order.size(); i++) {
    const UOp& n = order[i];
    os << op_name(n.op()) << " " << n.dtype().str() << " " << arg_text(n.arg());
    if (n.has_tag()) os << " #" << n.tag();
    for (auto& s : n.srcs()) os << " " << id.at(s.get());
    os << "\n";
    id[n.get()] = i;
  }
  return os.str();
}

UOp kernel_from_text(const std::string& text) {
  std::istringstream is(text);
  std::string ln;
  if (!std::getline(is, ln) || ln != kHeader) fail("fg-kernel text must start with '" + std::string(kHeader) + "'");
  std::vector<UOp> nodes;
  size_t line = 1;
  while (std::getline(is, ln)) {
    line++;
    if (ln.empty()) continue;
    std::istringstream ls(ln);
    std::string op_s, dt_s, arg_s, tok;
    if (!(ls >> op_s >> dt_s >> arg_s)) bad(line, "needs '<Op> <dtype> <arg>'");
    Op op;
    if (!parse_op(op_s, &op)) bad(line, "unknown op '" + op_s + "'");
    DType dt = parse_dtype(dt_s, line);
    Arg arg = parse_arg(arg_s, line);
    bool has_tag = false;
    uint64_t tag = 0;
    std::vector<UOp> srcs;
    while (ls >> tok) {
      if (tok[0] == '#') {
        if (has_tag || !srcs.empty()) bad(line, "a tag comes once, before the sources");
        errno = 0;
        char* end = nullptr;
        tag = std::strtoull(tok.c_str() + 1, &end, 10);
        if (errno != 0 || *end != '\0' || tok.size() < 2) bad(line, "bad tag '" + tok + "'");
        has_tag = true;
        continue;
      }
      int64_t s;
      if (!parse_i64(tok, &s) || s < 0 || static_cast<size_t>(s) >= nodes.size())
        bad(line, "source '" + tok + "' is not an earlier node");
      srcs.push_back(nodes[static_cast<size_t>(s)]);
    }
    if (op == Op::Device) {
      if (arg.kind != Arg::Kind::Device || !srcs.empty()) bad(line, "Device takes a device arg and no sources");
    } else {
      if (srcs.empty()) bad(line, std::string(op_name(op)) + " needs sources (leaves take a Device source)");
      for (auto& s : srcs)
        if (s.device() != srcs[0].device()) bad(line, "sources on different devices");
    }
    nodes.push_back(UOp::make(op, dt, std::move(srcs), std::move(arg), has_tag, tag));
  }
  if (nodes.empty() || nodes.back().op() != Op::Sink) fail("fg-kernel text must end with the kernel's Sink");
  return nodes.back();
}

}  // namespace fg
