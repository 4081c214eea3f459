// The Renderer half of the HIP device boundary (include/ferrograd_hip.h):
// render a rangeified kernel, given as text (kernel_text.hpp), to gfx950 HIP
// source plus everything its launches need, then load and run it.
//
// The reference's `Renderer::render(uops, name) -> String` (codegen.rs:17-20)
// returns source only and its call site hard-codes ClangRenderer
// (tensor.rs:845-852). A caller binding this device gets, for one kernel:
// the source, the launch passes (function, grid, block, LDS) in order, the
// kernel parameters in slot order with their kinds, and the bytes of scratch
// its passes share (split-K and split column-reduction partials).
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/ferrograd_hip.h"
#include "gpu_lower.hpp"
#include "hip_internal.hpp"
#include "kernel_text.hpp"

// Scratch of fg_hip_kernel_run_noalloc: FG_NOALLOC_SCRATCH_BYTES on every GPU
// the library is initialised on, held until the process ends. Host code never
// uses this name as an address (on the host it is a stand-in for the symbol):
// fg_hip_kernel_device_setup looks up each device's copy once and every later
// use goes through that pointer.
static __device__ __align__(256) unsigned char scratch[FG_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch` per ordinal
}  // namespace

struct fg_rendered {
  fg::RenderedKernel rk;
  std::vector<fg::LaunchSpec> launches;  // every pass, in order
  std::vector<int32_t> param_kinds;      // FG_ARG_* per slot
};

struct fg_kernel {
  std::vector<fg_prog*> passes;
  std::vector<fg::LaunchSpec> launches;
  std::vector<int32_t> param_kinds;
  size_t scratch_bytes = 0;
  fg_ctx* scratch_ctx = nullptr;  // where `scratch` was allocated
  void* scratch = nullptr;        // allocated by the first fg_hip_kernel_run
  ~fg_kernel() {
    for (auto* p : passes) fg_hip_program_free(p);
    if (scratch) fg_hip_free(scratch_ctx, scratch);
  }
};

namespace {

template <class F>
int guard(const char* what, F&& f) {
  try {
    return f();
  } catch (const std::exception& e) {
    return fg_hip_set_error(FG_ERR_INVALID, (std::string(what) + ": " + e.what()).c_str());
  }
}

// The caller's arguments against the kernel's parameter kinds. Builds no
// heap object unless it reports an error.
int check_args(const fg_kernel* k, const fg_arg* args, int nargs) {
  if (nargs != static_cast<int>(k->param_kinds.size()))
    return fg_hip_set_error(FG_ERR_ARGS, ("kernel takes " + std::to_string(k->param_kinds.size()) +
                                          " arguments, got " + std::to_string(nargs)).c_str());
  if (nargs && !args) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_kernel_run: null arguments");
  static const char* names[] = {"pointer", "i32", "f32", "bool"};
  for (int i = 0; i < nargs; i++) {
    if (args[i].kind != k->param_kinds[static_cast<size_t>(i)]) {
      const int want = k->param_kinds[static_cast<size_t>(i)];
      const int got = args[i].kind;
      return fg_hip_set_error(FG_ERR_ARGS, ("argument " + std::to_string(i) + " must be a " + names[want] + ", got " +
                                            (got >= 0 && got < 4 ? names[got] : "unknown kind"))
                                               .c_str());
    }
    if (args[i].kind == FG_ARG_PTR && !args[i].v.p)
      return fg_hip_set_error(FG_ERR_INVALID, ("argument " + std::to_string(i) + " is a null pointer").c_str());
  }
  return FG_OK;
}

// The launch arguments: the caller's, then the scratch pointer when the
// kernel has scratch. `out` holds at least 65 entries (launches take at most
// 64 arguments, fg_hip_launch's limit, which it checks).
int launch_args(const fg_kernel* k, const fg_arg* args, int nargs, void* scratch_ptr, fg_arg* out, int* n) {
  if (int rc = check_args(k, args, nargs)) return rc;
  if (nargs > 64) return fg_hip_set_error(FG_ERR_ARGS, "a kernel takes at most 64 arguments");
  if (nargs) std::memcpy(out, args, sizeof(fg_arg) * static_cast<size_t>(nargs));
  *n = nargs;
  if (k->scratch_bytes) {
    std::memset(&out[nargs], 0, sizeof(fg_arg));
    out[nargs].kind = FG_ARG_PTR;
    out[nargs].v.p = scratch_ptr;
    *n = nargs + 1;
  }
  return FG_OK;
}

// Queues every pass. `direct` launches skip launch profiling, which records
// events.
int launch_all(fg_ctx* ctx, const fg_kernel* k, const fg_arg* a, int n, bool direct) {
  for (size_t i = 0; i < k->passes.size(); i++) {
    const fg::LaunchSpec& l = k->launches[i];
    int rc = direct ? fg_hip_launch_direct(ctx, k->passes[i], a, n, l.grid, l.block, l.lds_bytes)
                    : fg_hip_launch(ctx, k->passes[i], a, n, l.grid, l.block, l.lds_bytes);
    if (rc) return rc;
  }
  return FG_OK;
}

}  // namespace

extern "C" {

int fg_hip_render(const char* kernel_text, fg_rendered** out) {
  if (!kernel_text || !out) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_render: null argument");
  return guard("fg_hip_render", [&] {
    fg::UOp kernel = fg::gpu_optimize(fg::kernel_from_text(kernel_text));
    auto r = std::make_unique<fg_rendered>();
    r->rk = fg::render_hip_stable(kernel);
    if (r->rk.launches.empty()) {
      fg::LaunchSpec l;
      l.func = r->rk.name;
      std::memcpy(l.grid, r->rk.grid, sizeof(l.grid));
      std::memcpy(l.block, r->rk.block, sizeof(l.block));
      l.lds_bytes = r->rk.lds_bytes;
      r->launches.push_back(l);
    } else {
      r->launches = r->rk.launches;
    }
    std::map<int64_t, int32_t> kinds;
    for (auto& n : kernel.toposort()) {
      if (n.op() == fg::Op::ParamBuffer) kinds[n.arg().a] = FG_ARG_PTR;
      if (n.op() == fg::Op::ParamScalar)
        kinds[n.arg().a] = n.dtype().kind == fg::DTypeKind::F32 ? FG_ARG_F32
                           : n.dtype().kind == fg::DTypeKind::I32 ? FG_ARG_I32 : FG_ARG_BOOL;
    }
    int64_t next = 0;
    for (auto& [slot, kind] : kinds) {
      if (slot != next) fg::fail("kernel parameter slots must be 0..n-1; slot " + std::to_string(next) + " is missing");
      r->param_kinds.push_back(kind);
      next++;
    }
    *out = r.release();
    return FG_OK;
  });
}

int fg_hip_rendered_info(const fg_rendered* r, const char** source, const char** kind, int* num_params,
                         int* num_launches, size_t* scratch_bytes) {
  if (!r) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_rendered_info: null rendered kernel");
  if (source) *source = r->rk.source.c_str();
  if (kind) *kind = r->rk.kind.c_str();
  if (num_params) *num_params = static_cast<int>(r->param_kinds.size());
  if (num_launches) *num_launches = static_cast<int>(r->launches.size());
  if (scratch_bytes) *scratch_bytes = r->rk.scratch_bytes;
  return FG_OK;
}

int fg_hip_rendered_param(const fg_rendered* r, int slot, int* kind) {
  if (!r || !kind) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_rendered_param: null argument");
  if (slot < 0 || slot >= static_cast<int>(r->param_kinds.size()))
    return fg_hip_set_error(FG_ERR_INVALID, ("parameter slot " + std::to_string(slot) + " out of range").c_str());
  *kind = r->param_kinds[static_cast<size_t>(slot)];
  return FG_OK;
}

int fg_hip_rendered_launch(const fg_rendered* r, int i, const char** func, unsigned grid[3], unsigned block[3],
                           unsigned* lds_bytes) {
  if (!r) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_rendered_launch: null rendered kernel");
  if (i < 0 || i >= static_cast<int>(r->launches.size()))
    return fg_hip_set_error(FG_ERR_INVALID, ("launch " + std::to_string(i) + " out of range").c_str());
  const fg::LaunchSpec& l = r->launches[static_cast<size_t>(i)];
  if (func) *func = l.func.c_str();
  if (grid) std::memcpy(grid, l.grid, sizeof(l.grid));
  if (block) std::memcpy(block, l.block, sizeof(l.block));
  if (lds_bytes) *lds_bytes = l.lds_bytes;
  return FG_OK;
}

int fg_hip_rendered_free(fg_rendered* r) {
  delete r;
  return FG_OK;
}

int fg_hip_kernel_load(fg_ctx* ctx, const fg_rendered* r, fg_kernel** out) {
  if (!ctx || !r || !out) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_kernel_load: null argument");
  auto k = std::make_unique<fg_kernel>();
  const int nargs = static_cast<int>(r->param_kinds.size()) + (r->rk.scratch_bytes ? 1 : 0);
  fg_prog* first = nullptr;
  if (int rc = fg_hip_compile(ctx, r->rk.source.c_str(), r->launches[0].func.c_str(), nargs, &first)) return rc;
  k->passes.push_back(first);
  for (size_t i = 1; i < r->launches.size(); i++) {
    fg_prog* p = nullptr;
    if (int rc = fg_hip_program_function(first, r->launches[i].func.c_str(), nargs, &p)) return rc;
    k->passes.push_back(p);
  }
  k->launches = r->launches;
  k->param_kinds = r->param_kinds;
  k->scratch_bytes = r->rk.scratch_bytes;
  *out = k.release();
  return FG_OK;
}

int fg_hip_kernel_run(fg_ctx* ctx, fg_kernel* k, const fg_arg* args, int nargs) {
  if (!ctx || !k) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_kernel_run: null argument");
  if (k->scratch_bytes && !k->scratch) {
    if (int rc = fg_hip_alloc(ctx, k->scratch_bytes, 0, &k->scratch)) return rc;
    k->scratch_ctx = ctx;
  }
  if (k->scratch && k->scratch_ctx != ctx)
    return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_kernel_run: the kernel's scratch belongs to another context");
  fg_arg a[65];
  int n = 0;
  if (int rc = launch_args(k, args, nargs, k->scratch, a, &n)) return rc;
  return launch_all(ctx, k, a, n, false);
}

int fg_hip_kernel_device_setup(int ordinal) {
  if (ordinal < 0 || ordinal >= kMaxDevices)
    return fg_hip_set_error(FG_ERR_INVALID, ("device ordinal " + std::to_string(ordinal) + " beyond the " +
                                             std::to_string(kMaxDevices) + " this library supports").c_str());
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[ordinal]) return FG_OK;
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr)
    return fg_hip_set_error(FG_ERR_HIP, (std::string("hipGetSymbolAddress(scratch) on device ") +
                                         std::to_string(ordinal) + ": " + hipGetErrorString(e))
                                            .c_str());
  g_scratch_ptr[ordinal] = ptr;
  return FG_OK;
}

int fg_hip_kernel_run_noalloc(fg_ctx* ctx, fg_kernel* k, const fg_arg* args, int nargs) {
  if (!ctx || !k) return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_kernel_run_noalloc: null argument");
  if (k->scratch_bytes > FG_NOALLOC_SCRATCH_BYTES)
    return fg_hip_set_error(FG_ERR_INVALID, ("fg_hip_kernel_run_noalloc: the kernel needs " +
                                             std::to_string(k->scratch_bytes) + " bytes of scratch, more than the " +
                                             std::to_string(FG_NOALLOC_SCRATCH_BYTES) +
                                             " the library holds per GPU; run it with fg_hip_kernel_run")
                                                .c_str());
  const int dev = fg_hip_context_device(ctx);
  void* ptr = dev >= 0 && dev < kMaxDevices ? g_scratch_ptr[dev] : nullptr;
  if (k->scratch_bytes && !ptr)
    return fg_hip_set_error(FG_ERR_INVALID, "fg_hip_kernel_run_noalloc: no scratch set up for this context's device");
  fg_arg a[65];
  int n = 0;
  if (int rc = launch_args(k, args, nargs, ptr, a, &n)) return rc;
  return launch_all(ctx, k, a, n, true);
}

int fg_hip_kernel_free(fg_kernel* k) {
  delete k;
  return FG_OK;
}

}  // extern "C"
