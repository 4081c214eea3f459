// C-ABI of the tensor front end (include/ferrograd.h).
#include "../../include/ferrograd.h"

#include <cstdlib>
#include <cstring>
#include <sstream>
#include <string>

#include "gpu_lower.hpp"
#include "kernel_text.hpp"
#include "schedule.hpp"
#include "tensor.hpp"

struct fg_tensor {
  fg::Tensor t;
};
struct fg_linear {
  fg::Linear l;
};
struct fg_sgd {
  fg::Sgd s;
};

namespace {

thread_local std::string g_err;

template <class F>
int guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return 1;
  }
}

fg::DType to_dtype(int d) {
  switch (d) {
    case FG_F32: return fg::DType::F32();
    case FG_I32: return fg::DType::I32();
    case FG_BOOL: return fg::DType::Bool();
    default: fg::fail("unknown dtype code " + std::to_string(d));
  }
}

int from_dtype(fg::DType d) {
  switch (d.kind) {
    case fg::DTypeKind::F32: return FG_F32;
    case fg::DTypeKind::I32: return FG_I32;
    case fg::DTypeKind::Bool: return FG_BOOL;
    default: return -1;
  }
}

fg::DeviceId to_dev(int d) {
  FG_CHECK(d == FG_DEV_CPU || d == FG_DEV_HIP, "unknown device code " + std::to_string(d));
  return static_cast<fg::DeviceId>(d);
}

fg::Shape to_shape(const int64_t* s, int n) {
  fg::Shape out;
  for (int i = 0; i < n; i++) {
    FG_CHECK(s[i] >= 0, "negative dimension");
    out.push_back(static_cast<size_t>(s[i]));
  }
  return out;
}

std::vector<size_t> to_axes(const int64_t* a, int n) {
  std::vector<size_t> out;
  for (int i = 0; i < n; i++) {
    FG_CHECK(a[i] >= 0, "negative axis");
    out.push_back(static_cast<size_t>(a[i]));
  }
  return out;
}

fg_tensor* wrap(const fg::Tensor& t) { return new fg_tensor{t}; }

std::string json_escape(const std::string& s) {
  std::string o;
  o.reserve(s.size() + 16);
  for (char c : s) {
    switch (c) {
      case '"': o += "\\\""; break;
      case '\\': o += "\\\\"; break;
      case '\n': o += "\\n"; break;
      case '\t': o += "\\t"; break;
      default: o += c;
    }
  }
  return o;
}

}  // namespace

extern "C" {

const char* fg_last_error(void) { return g_err.c_str(); }

int fg_tensor_from_data(int device, int dtype, const void* data, size_t nbytes, const int64_t* shape, int ndim,
                        fg_tensor** out) {
  return guard([&] {
    *out = wrap(fg::Tensor::from_bytes(data, nbytes, to_shape(shape, ndim), to_dtype(dtype), to_dev(device)));
  });
}

int fg_tensor_zeros(int device, int dtype, const int64_t* shape, int ndim, fg_tensor** out) {
  return guard([&] { *out = wrap(fg::Tensor::zeros(to_shape(shape, ndim), to_dev(device), to_dtype(dtype))); });
}

int fg_tensor_ones(int device, int dtype, const int64_t* shape, int ndim, fg_tensor** out) {
  return guard([&] { *out = wrap(fg::Tensor::ones(to_shape(shape, ndim), to_dev(device), to_dtype(dtype))); });
}

int fg_idx_images(const char* path, int device, fg_tensor** out) {
  return guard([&] { *out = wrap(fg::idx_images(path, to_dev(device))); });
}

int fg_idx_labels(const char* path, uint8_t* out, size_t capacity, size_t* count) {
  return guard([&] {
    std::vector<uint8_t> labels = fg::idx_labels(path);
    *count = labels.size();
    if (out) {
      FG_CHECK(capacity >= labels.size(), "fg_idx_labels: buffer holds " + std::to_string(capacity) + " labels, file has " +
                                              std::to_string(labels.size()));
      std::memcpy(out, labels.data(), labels.size());
    }
  });
}

int fg_tensor_free(fg_tensor* t) {
  delete t;
  return 0;
}

int fg_tensor_unary(fg_tensor* t, int op, fg_tensor** out) {
  return guard([&] {
    const fg::Tensor& x = t->t;
    switch (op) {
      case FG_UNARY_NEG: *out = wrap(x.neg()); break;
      case FG_UNARY_RECIPROCAL: *out = wrap(x.reciprocal()); break;
      case FG_UNARY_EXP2: *out = wrap(x.exp2()); break;
      case FG_UNARY_LOG2: *out = wrap(x.log2()); break;
      case FG_UNARY_SQRT: *out = wrap(x.sqrt()); break;
      case FG_UNARY_RELU: *out = wrap(x.relu()); break;
      case FG_UNARY_EXP: *out = wrap(x.exp()); break;
      case FG_UNARY_LOG: *out = wrap(x.log()); break;
      case FG_UNARY_CONTIGUOUS: *out = wrap(x.contiguous()); break;
      case FG_UNARY_DETACH: *out = wrap(x.detach()); break;
      case FG_UNARY_ALIAS: *out = wrap(x); break;
      default: fg::fail("unknown unary op " + std::to_string(op));
    }
  });
}

int fg_tensor_binary(fg_tensor* a, fg_tensor* b, int op, fg_tensor** out) {
  return guard([&] {
    switch (op) {
      case FG_BINARY_ADD: *out = wrap(a->t.add(b->t)); break;
      case FG_BINARY_MUL: *out = wrap(a->t.mul(b->t)); break;
      case FG_BINARY_SUB: *out = wrap(a->t.sub(b->t)); break;
      case FG_BINARY_MATMUL: *out = wrap(a->t.matmul(b->t)); break;
      case FG_BINARY_CROSS_ENTROPY: *out = wrap(a->t.cross_entropy(b->t)); break;
      default: fg::fail("unknown binary op " + std::to_string(op));
    }
  });
}

int fg_tensor_reduce(fg_tensor* t, int op, const int64_t* axes, int n, fg_tensor** out) {
  return guard([&] {
    auto ax = to_axes(axes, n);
    if (op == FG_REDUCE_SUM) *out = wrap(t->t.sum(ax));
    else if (op == FG_REDUCE_MAX) *out = wrap(t->t.max(ax));
    else fg::fail("unknown reduce op " + std::to_string(op));
  });
}

int fg_tensor_movement(fg_tensor* t, int op, const int64_t* arg, int n, fg_tensor** out) {
  return guard([&] {
    switch (op) {
      case FG_MOVE_RESHAPE: *out = wrap(t->t.reshape(to_shape(arg, n))); break;
      case FG_MOVE_PERMUTE: *out = wrap(t->t.permute(to_axes(arg, n))); break;
      case FG_MOVE_EXPAND: *out = wrap(t->t.expand(to_shape(arg, n))); break;
      default: fg::fail("unknown movement op " + std::to_string(op));
    }
  });
}

int fg_tensor_narrow(fg_tensor* t, int64_t dim, int64_t start, int64_t len, fg_tensor** out) {
  return guard([&] {
    FG_CHECK(dim >= 0 && start >= 0 && len >= 0, "narrow: negative argument");
    *out = wrap(t->t.narrow(static_cast<size_t>(dim), static_cast<size_t>(start), static_cast<size_t>(len)));
  });
}

int fg_tensor_log_softmax(fg_tensor* t, int64_t axis, fg_tensor** out) {
  return guard([&] {
    FG_CHECK(axis >= 0, "log_softmax: negative axis");
    *out = wrap(t->t.log_softmax(static_cast<size_t>(axis)));
  });
}

int fg_tensor_assign(fg_tensor* t, fg_tensor* v) {
  return guard([&] { t->t.assign(v->t); });
}

int fg_tensor_replace(fg_tensor* t, fg_tensor* v) {
  return guard([&] { t->t.replace(v->t); });
}

int fg_tensor_realize_many(fg_tensor** ts, int n) {
  return guard([&] {
    std::vector<fg::Tensor> v;
    for (int i = 0; i < n; i++) v.push_back(ts[i]->t);
    fg::Tensor::realize_many(v);
  });
}

int fg_tensor_read(fg_tensor* t, void* dst, size_t nbytes) {
  return guard([&] {
    fg::Buffer b = t->t.realized_buffer();
    FG_CHECK(b->nbytes() == nbytes,
             "fg_tensor_read: expected " + std::to_string(b->nbytes()) + " bytes, got " + std::to_string(nbytes));
    FG_CHECK(dst || nbytes == 0, "fg_tensor_read: null destination");
    fg::get_device(b->device).copy_to_host_into(b, dst, nbytes);
  });
}

int fg_tensor_write(fg_tensor* t, const void* src, size_t nbytes) {
  return guard([&] {
    FG_CHECK(src || nbytes == 0, "fg_tensor_write: null source");
    fg::Buffer b = t->t.realized_buffer();
    fg::get_device(b->device).copy_from_host(b, src, nbytes);
  });
}

int fg_tensor_shape(fg_tensor* t, int64_t* shape, int* ndim) {
  return guard([&] {
    auto s = t->t.shape();
    FG_CHECK(static_cast<int>(s.size()) <= *ndim, "fg_tensor_shape: shape buffer too small");
    for (size_t i = 0; i < s.size(); i++) shape[i] = static_cast<int64_t>(s[i]);
    *ndim = static_cast<int>(s.size());
  });
}

int fg_tensor_info(fg_tensor* t, int* dtype, int* device, int* realized, int* rg) {
  return guard([&] {
    if (dtype) *dtype = from_dtype(t->t.dtype());
    if (device) *device = static_cast<int>(t->t.device());
    if (realized) *realized = t->t.is_realized() ? 1 : 0;
    if (rg) *rg = t->t.requires_grad() ? 1 : 0;
  });
}

int fg_tensor_data_ptr(fg_tensor* t, void** ptr, size_t* nbytes) {
  return guard([&] {
    FG_CHECK(t->t.is_realized(), "fg_tensor_data_ptr: tensor is not realized");
    fg::Buffer b = t->t.realized_buffer();
    b->ensure_allocated();
    *ptr = b->storage;
    if (nbytes) *nbytes = b->nbytes();
  });
}

int fg_tensor_set_requires_grad(fg_tensor* t, int rg) {
  return guard([&] { t->t.with_requires_grad(rg != 0); });
}

int fg_tensor_same(fg_tensor* a, fg_tensor* b, int* same) {
  return guard([&] { *same = a->t.ptr_eq(b->t) ? 1 : 0; });
}

int fg_tensor_grad(fg_tensor* t, fg_tensor** out) {
  return guard([&] {
    auto g = t->t.grad();
    *out = g ? wrap(*g) : nullptr;
  });
}

int fg_tensor_backward(fg_tensor* loss) {
  return guard([&] { loss->t.backward(); });
}

int fg_tensor_gradient(fg_tensor* loss, fg_tensor** targets, int n, fg_tensor** outs) {
  return guard([&] {
    std::vector<fg::Tensor> ts;
    for (int i = 0; i < n; i++) ts.push_back(targets[i]->t);
    auto gs = loss->t.gradient(ts);
    for (int i = 0; i < n; i++) outs[i] = wrap(gs[static_cast<size_t>(i)]);
  });
}

int fg_reset_init_seed(uint64_t seed) {
  fg::reset_init_seed(seed);
  return 0;
}

int fg_linear_new(int device, int64_t in, int64_t outf, int bias, fg_linear** out) {
  return guard([&] {
    FG_CHECK(in > 0 && outf > 0, "Linear: features must be positive");
    *out = new fg_linear{fg::Linear::create(static_cast<size_t>(in), static_cast<size_t>(outf), to_dev(device), bias != 0)};
  });
}

int fg_linear_forward(fg_linear* l, fg_tensor* x, fg_tensor** out) {
  return guard([&] { *out = wrap(l->l.forward(x->t)); });
}

int fg_mlp_train_steps(fg_linear* const* layers, int nlayers, fg_sgd* opt, fg_tensor* x, fg_tensor* targets, int steps,
                       float* losses) {
  return guard([&] {
    FG_CHECK(layers && nlayers > 0 && opt && x && targets && (losses || steps == 0),
             "fg_mlp_train_steps: null argument or no layers");
    std::vector<const fg::Linear*> ls;
    for (int i = 0; i < nlayers; i++) {
      FG_CHECK(layers[i], "fg_mlp_train_steps: null layer");
      ls.push_back(&layers[i]->l);
    }
    std::vector<float> v = fg::train_steps(ls, opt->s, x->t, targets->t, steps);
    std::copy(v.begin(), v.end(), losses);
  });
}

int fg_mlp_train_batches(fg_linear* const* layers, int nlayers, fg_sgd* opt, fg_tensor* images, fg_tensor* targets,
                         int64_t batch_size, int64_t first_batch, int steps, float* losses) {
  return guard([&] {
    FG_CHECK(layers && nlayers > 0 && opt && images && targets && (losses || steps == 0),
             "fg_mlp_train_batches: null argument or no layers");
    FG_CHECK(batch_size > 0, "fg_mlp_train_batches: batch size must be positive");
    std::vector<const fg::Linear*> ls;
    for (int i = 0; i < nlayers; i++) {
      FG_CHECK(layers[i], "fg_mlp_train_batches: null layer");
      ls.push_back(&layers[i]->l);
    }
    std::vector<float> v = fg::train_steps(ls, opt->s, images->t, targets->t, steps, batch_size, first_batch);
    std::copy(v.begin(), v.end(), losses);
  });
}

int fg_linear_num_params(fg_linear* l, int* n) {
  return guard([&] { *n = static_cast<int>(l->l.parameters().size()); });
}

int fg_linear_param(fg_linear* l, int i, fg_tensor** out) {
  return guard([&] {
    auto ps = l->l.parameters();
    FG_CHECK(i >= 0 && static_cast<size_t>(i) < ps.size(), "Linear parameter index out of range");
    *out = wrap(ps[static_cast<size_t>(i)]);
  });
}

int fg_linear_free(fg_linear* l) {
  delete l;
  return 0;
}

int fg_sgd_new(fg_tensor** params, int n, float lr, fg_sgd** out) {
  return guard([&] {
    std::vector<fg::Tensor> ps;
    for (int i = 0; i < n; i++) ps.push_back(params[i]->t);
    *out = new fg_sgd{fg::Sgd(ps, lr)};
  });
}

int fg_sgd_zero_grad(fg_sgd* s) {
  return guard([&] { s->s.zero_grad(); });
}

int fg_sgd_step(fg_sgd* s) {
  return guard([&] { s->s.step(); });
}

int fg_sgd_free(fg_sgd* s) {
  delete s;
  return 0;
}

int fg_synchronize(int device) {
  return guard([&] { fg::get_device(to_dev(device)).synchronize(); });
}

int fg_default_device(int* device) {
  return guard([&] { *device = fg::default_device() == fg::DeviceId::Cpu ? FG_DEV_CPU : FG_DEV_HIP; });
}

int fg_gpu_passes(int* symbolic, int* mfma, int* narrow, int* fuse, int* block, int* batch) {
  return guard([&] {
    const fg::GpuPasses& p = fg::gpu_passes();
    const char* e = std::getenv("FG_FUSE");
    *symbolic = p.symbolic;
    *mfma = p.mfma;
    *narrow = p.narrow;
    *fuse = p.fuse && !(e && std::strcmp(e, "0") == 0);
    *block = p.block;
    *batch = p.batch;
  });
}

int fg_device_context(int device, void** ctx) {
  return guard([&] {
    FG_CHECK(device == FG_DEV_HIP, "fg_device_context: only the HIP device has a context");
    *ctx = fg::hip_context_raw();
  });
}

int fg_stats(uint64_t* k, uint64_t* p, uint64_t* h) {
  auto& s = fg::realize_stats();
  if (k) *k = s.kernels_launched;
  if (p) *p = s.programs_compiled;
  if (h) *h = s.lowering_cache_hits;
  return 0;
}

int fg_step_capture_stats(uint64_t* captured, uint64_t* replayed) {
  if (captured) *captured = fg::realize_stats().steps_captured;
  if (replayed) *replayed = fg::realize_stats().steps_replayed;
  return 0;
}

int fg_graph_stats(uint64_t* replays, uint64_t* updated_launches) {
  if (replays) *replays = fg::realize_stats().graph_replays;
  if (updated_launches) *updated_launches = fg::realize_stats().graph_updates;
  return 0;
}

int fg_host_times(uint64_t out[5]) {
  auto& s = fg::realize_stats();
  out[0] = s.ns_schedule;
  out[1] = s.ns_lower;
  out[2] = s.ns_launch;
  out[3] = s.ns_apply_map;
  out[4] = s.ns_backward;
  return 0;
}

int fg_clear_caches(void) {
  return guard([&] { fg::clear_kernel_caches(); });
}

int fg_plan_cache_enable(int on) {
  return guard([&] { fg::set_plan_cache_enabled(on != 0); });
}

int fg_set_graph_min_launches(int n, int* previous) {
  return guard([&] {
    int prev = fg::set_graph_min_launches(n);
    if (previous) *previous = prev;
  });
}

int fg_plan_cache_stats(uint64_t* hits, uint64_t* misses, uint64_t* entries) {
  return guard([&] { fg::plan_cache_stats(hits, misses, entries); });
}

int fg_debug_plan(fg_tensor** roots, int n, int fuse, int render, char* buf, size_t len, size_t* needed) {
  // Scheduling reserves fresh buffer ids, so the plan is computed once (call
  // with buf == NULL) and a second call with a buffer copies that result.
  static thread_local std::string last;
  if (buf) {
    if (needed) *needed = last.size() + 1;
    size_t m = len ? std::min(len - 1, last.size()) : 0;
    if (len) {
      std::memcpy(buf, last.data(), m);
      buf[m] = '\0';
    }
    return 0;
  }
  return guard([&] {
    std::vector<fg::UOp> rs;
    fg::UOpSet seen;
    for (int i = 0; i < n; i++) {
      if (roots[i]->t.is_realized()) continue;
      fg::UOp u = roots[i]->t.uop();
      if (seen.insert(u).second) rs.push_back(u);
    }
    std::ostringstream os;
    os << "{\"items\": [";
    // With `render`: which launches are block kernels, and their argument
    // counts, for the batch runs a replayed sequence would launch.
    std::vector<bool> is_block;
    std::vector<size_t> nargs;
    std::vector<fg::RenderedKernel> rks;
    std::vector<std::vector<fg::BatchArg>> binfo;
    if (!rs.empty()) {
      fg::ScheduleOptions opt;
      opt.fuse = fuse != 0;
      fg::PtrIndexMap held(64);
      if (opt.fuse) {
        fg::collect_held_nodes(&held, nullptr);
        opt.held = &held;
      }
      auto plan = fg::schedule_many(rs, opt);
      for (size_t i = 0; i < plan.items.size(); i++) {
        auto& it = plan.items[i];
        if (i) os << ", ";
        os << "{\"output\": ";
        if (it.output_buffer) os << it.output_buffer->id;
        else os << "null";
        os << ", \"out_shape\": [";
        for (size_t j = 0; j < it.out_shape.size(); j++) os << (j ? ", " : "") << it.out_shape[j];
        os << "], \"inputs\": [";
        for (size_t j = 0; j < it.inputs.size(); j++) {
          auto& a = it.inputs[j];
          if (j) os << ", ";
          switch (a.kind) {
            case fg::KernelArg::Kind::Buffer: os << "{\"buffer\": " << a.buffer->id << "}"; break;
            case fg::KernelArg::Kind::I32: os << "{\"i32\": " << a.i << "}"; break;
            case fg::KernelArg::Kind::F32: os << "{\"f32\": " << a.f << "}"; break;
            case fg::KernelArg::Kind::Bool: os << "{\"bool\": " << (a.b ? "true" : "false") << "}"; break;
          }
        }
        os << "]";
        if (render) {
          fg::UOp rangeified = fg::rangeify(it.sink);
          os << ", \"kernel\": \"" << json_escape(fg::kernel_to_text(rangeified)) << "\"";
          fg::UOp k = fg::with_all_params(fg::gpu_optimize(rangeified), it.sink);
          auto rk = fg::render_hip_stable(k);
          os << ", \"name\": \"" << rk.name << "\", \"class\": \"" << rk.kind << "\", \"base_class\": \""
             << fg::kernel_class_name(fg::base_class(k)) << "\", \"grid\": [" << rk.grid[0] << ", " << rk.grid[1] << ", "
             << rk.grid[2] << "], \"block\": [" << rk.block[0] << ", " << rk.block[1] << ", " << rk.block[2]
             << "], \"source\": \"" << json_escape(rk.source) << "\"";
          is_block.push_back(!rk.stage_fn.empty() && rk.launches.empty());
          nargs.push_back(it.output_buffer ? it.inputs.size() + 1 : it.inputs.size());
          std::vector<fg::BatchArg> bi;
          if (it.output_buffer) bi.push_back({it.output_buffer.get(), it.output_buffer->numel});
          for (auto& a : it.inputs)
            bi.push_back(a.kind == fg::KernelArg::Kind::Buffer ? fg::BatchArg{a.buffer.get(), a.buffer->numel}
                                                              : fg::BatchArg{});
          binfo.push_back(std::move(bi));
          rks.push_back(std::move(rk));
        }
        os << "}";
      }
    }
    os << "]";
    if (render) {
      os << ", \"batches\": [";
      auto runs = fg::block_batch_runs(is_block, nargs);
      for (size_t i = 0; i < runs.size(); i++)
        os << (i ? ", " : "") << "[" << runs[i].first << ", " << runs[i].second << "]";
      // Each run's batch kernel as a replayed sequence would compile it (in
      // plan order), with the stage outputs it keeps in LDS.
      os << "], \"batch_kernels\": [";
      for (size_t i = 0; i < runs.size(); i++) {
        std::vector<const fg::RenderedKernel*> stages;
        std::vector<std::vector<fg::BatchArg>> args;
        for (size_t j = runs[i].first; j < runs[i].first + runs[i].second; j++) {
          stages.push_back(&rks[j]);
          args.push_back(binfo[j]);
        }
        const fg::BatchForwarding fwd = fg::batch_forwarding(stages, args);
        const fg::RenderedKernel bk = fg::render_block_batch(stages, false, &fwd);
        os << (i ? ", " : "") << "{\"name\": \"" << bk.name << "\", \"forwarded\": " << fwd.dtypes.size()
           << ", \"source\": \"" << json_escape(bk.source) << "\"}";
      }
      // Adjacent independent kernels that a replayed sequence would launch
      // together (in plan order, outside the batches).
      os << "], \"pairs\": [";
      std::vector<bool> in_batch(rks.size(), false);
      for (auto [f, c] : runs)
        for (size_t j = f; j < f + c; j++) in_batch[j] = true;
      std::vector<const fg::RenderedKernel*> all;
      for (auto& r : rks) all.push_back(&r);
      auto firsts = fg::pair_runs(all, binfo, in_batch);
      for (size_t i = 0; i < firsts.size(); i++) {
        const fg::RenderedKernel pk = fg::render_hfused(rks[firsts[i]], rks[firsts[i] + 1]);
        os << (i ? ", " : "") << "{\"first\": " << firsts[i] << ", \"name\": \"" << pk.name
           << "\", \"grid\": " << pk.grid[0] << ", \"source\": \"" << json_escape(pk.source) << "\"}";
      }
      // Batches that a replayed sequence would run beside an adjacent
      // independent small GEMM or pair (in plan order), and that launch.
      os << "], \"hbatches\": [";
      auto hruns = fg::hbatch_runs(all, binfo, runs, firsts);
      for (size_t i = 0; i < hruns.size(); i++) {
        const auto [f, c] = runs[hruns[i].group];
        std::vector<const fg::RenderedKernel*> hb, stages;
        std::vector<std::vector<fg::BatchArg>> args;
        for (size_t j : hruns[i].hb) hb.push_back(&rks[j]);
        for (size_t j = f; j < f + c; j++) {
          stages.push_back(&rks[j]);
          args.push_back(binfo[j]);
        }
        const fg::BatchForwarding fwd = fg::batch_forwarding(stages, args);
        const fg::RenderedKernel hk = fg::render_hbatch(hb, stages, false, &fwd);
        os << (i ? ", " : "") << "{\"hb\": [";
        for (size_t j = 0; j < hruns[i].hb.size(); j++) os << (j ? ", " : "") << hruns[i].hb[j];
        os << "], \"batch\": " << hruns[i].group << ", \"name\": \"" << hk.name << "\", \"grid\": " << hk.grid[0]
           << ", \"source\": \"" << json_escape(hk.source) << "\"}";
      }
      os << "]";
    }
    os << "}";
    last = os.str();
    if (needed) *needed = last.size() + 1;
  });
}

}  // extern "C"
