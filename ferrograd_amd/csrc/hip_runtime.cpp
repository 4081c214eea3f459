// HIP runtime behind the C-ABI in include/ferrograd_hip.h: hiprtc compile with
// an on-disk code-object cache, module load, kernel launch, a size-keyed
// caching allocator and host copies. Replaces src/device/cpu.rs:151-394
// (clang subprocess + dlopen + libffi) for the MI355X.
#include <dlfcn.h>
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>
#include <hsa/hsa.h>
#include <hsa/hsa_ext_amd.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <functional>
#include <thread>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ferrograd_hip.h"
#include "hip_internal.hpp"

namespace {

thread_local std::string g_last_error;

int set_err(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

#define HIP_TRY(expr)                                                                            \
  do {                                                                                           \
    hipError_t _e = (expr);                                                                      \
    if (_e != hipSuccess)                                                                        \
      return set_err(FG_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(_e));             \
  } while (0)

// Options every generated kernel is compiled with. -ffp-contract=off keeps each
// product and sum separately rounded, as the reference's one-statement-per-op C
// is (codegen/clang.rs:203-239). Packed fp32 instructions are disabled.
const char* kRtcOptions[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-Xclang", "-target-feature",
                             "-Xclang", "-packed-fp32-ops", "-std=c++17"};
constexpr int kNumRtcOptions = sizeof(kRtcOptions) / sizeof(kRtcOptions[0]);

uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ULL) {
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ULL;
  }
  return h;
}

void cache_anchor() {}

// Code objects live in `_kcache/` next to this shared library unless
// FG_KERNEL_CACHE names another directory.
std::string cache_dir() {
  if (const char* e = std::getenv("FG_KERNEL_CACHE")) return e;
  static std::string dir = [] {
    Dl_info info;
    std::string d = "/tmp";
    if (dladdr(reinterpret_cast<void*>(&cache_anchor), &info) && info.dli_fname) {
      std::string f = info.dli_fname;
      auto pos = f.rfind('/');
      if (pos != std::string::npos) d = f.substr(0, pos);
    }
    return d + "/_kcache";
  }();
  return dir;
}

bool read_file(const std::string& path, std::vector<char>* out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  f.seekg(0, std::ios::end);
  auto n = f.tellg();
  if (n <= 0) return false;
  out->resize(static_cast<size_t>(n));
  f.seekg(0);
  f.read(out->data(), n);
  return static_cast<bool>(f);
}

// Writes `data` to a temporary file and renames it into place only when every
// byte reached the file, so a reader never sees a partial code object.
void write_file_atomic(const std::string& path, const std::vector<char>& data) {
  std::string tmp = path + ".tmp" + std::to_string(getpid());
  bool ok;
  {
    std::ofstream f(tmp, std::ios::binary);
    f.write(data.data(), static_cast<std::streamsize>(data.size()));
    f.flush();
    ok = static_cast<bool>(f);
    f.close();
    ok = ok && !f.fail();
  }
  if (!ok || std::rename(tmp.c_str(), path.c_str()) != 0) std::remove(tmp.c_str());
}

// The hiprtc version, part of every cache key: a code object cached by one
// toolchain is never loaded under another.
std::string hiprtc_version() {
  int major = 0, minor = 0;
  if (hiprtcVersion(&major, &minor) != HIPRTC_SUCCESS) return "hiprtc ?";
  return "hiprtc " + std::to_string(major) + "." + std::to_string(minor);
}

}  // namespace

struct AqlQueue;
// The context's AQL queue while a replay loop runs on it (one HIP context per
// process in practice); a module loaded into it is destroyed only once the
// queue has drained.
AqlQueue* g_active_aql = nullptr;
void aql_drain_before_unload();

struct ModuleRef {
  hipModule_t module = nullptr;
  // The code object again, loaded by the context's own HSA queue on its
  // first dispatch from the module (fg_hip_aql_launch).
  std::vector<char> code;
  bool hsa_loaded = false;
  hsa_code_object_reader_t reader{};
  hsa_executable_t exe{};
  ~ModuleRef() {
    if (hsa_loaded) {
      aql_drain_before_unload();
      (void)hsa_executable_destroy(exe);
      (void)hsa_code_object_reader_destroy(reader);
    }
    if (module) (void)hipModuleUnload(module);
  }
};

struct fg_prog {
  std::shared_ptr<ModuleRef> module;
  hipFunction_t func = nullptr;
  int num_args = 0;
  std::string name;
  // The kernel as the HSA queue dispatches it: its descriptor and segment
  // sizes (read on the first dispatch).
  bool aql_loaded = false;
  uint64_t kernel_object = 0;
  uint32_t kernarg_size = 0, group_size = 0, private_size = 0;
};

// The context's own HSA queue, written directly by the host: a kernel launch
// is one 64-byte AQL packet and its arguments, about 0.5 us of host time on
// MI355X against 2.5-4 us for hipModuleLaunchKernel, for the same device
// cost per dependent launch (1.7 us) when the arguments sit in device memory
// and the packets fence at agent scope.
struct AqlQueue {
  hsa_agent_t gpu{}, cpu{};
  hsa_queue_t* q = nullptr;
  char* kargs = nullptr;  // a ring of argument slots in fine-grained device memory, one per queue entry
  hsa_signal_t slot_signal[FG_READ_SLOTS] = {};
  uint64_t slot_packet[FG_READ_SLOTS] = {};
  bool slot_pending[FG_READ_SLOTS] = {};
  hsa_signal_t drain{};
  uint64_t done = 0;         // every packet below this index has completed
  bool active = false;
  bool first = true;         // the next packet is the first since the HIP stream ran
};

struct fg_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  // Modules loaded on this context, by code-object cache path (a hash of
  // source, options and compiler version), oldest first in `loaded_order`:
  // compiling a source again reuses its loaded module (and its HSA
  // executable) instead of reading, loading and, for the direct queue,
  // loading the code object again.
  std::unordered_map<std::string, std::shared_ptr<ModuleRef>> loaded;
  std::deque<std::string> loaded_order;
  hipEvent_t events[64] = {};
  // Caching allocator: exact-size free lists. Blocks are only reused by work
  // queued later on the same stream, so reuse needs no synchronisation.
  std::unordered_map<size_t, std::vector<void*>> free_blocks;
  std::unordered_map<void*, size_t> sizes;
  size_t cached_bytes = 0;
  // Pinned staging for small host->device copies, used as a ring: a region is
  // reused only after the stream has passed the copy that read it.
  char* staging = nullptr;
  size_t staging_size = 0;
  size_t staging_head = 0;
  hipEvent_t staging_event = nullptr;
  bool staging_event_pending = false;
  // Pinned landing buffer for small device->host copies. A copy into pageable
  // memory goes through the runtime's own staging and took 25 us for 4 bytes
  // on MI355X, against 16.5 us into pinned memory (the kernel + sync floor is
  // 12.9 us). Reads are synchronous, so one buffer serves them all.
  char* readback = nullptr;
  // Asynchronous read-back slots: pinned landing areas, each with the event
  // recorded behind its copy.
  char* async_read = nullptr;
  hipEvent_t async_events[FG_READ_SLOTS] = {};
  size_t async_bytes[FG_READ_SLOTS] = {};
  bool async_pending[FG_READ_SLOTS] = {};
  // Direct AQL dispatch (fg_hip_aql_begin / fg_hip_aql_end); null until used.
  AqlQueue* aql = nullptr;
  // Large host<->device copies: two pinned chunks, each with the event of
  // its last DMA, so the host copies one chunk while the other is in flight
  // (allocated for each large copy and given back at its end).
  char* chunk[2] = {nullptr, nullptr};
  hipEvent_t chunk_event[2] = {};
  bool chunk_pending[2] = {false, false};
  // Launch profiling.
  bool profiling = false;
  std::vector<hipEvent_t> event_pool;
  struct Rec {
    std::string name;
    hipEvent_t a, b;
  };
  std::vector<Rec> records;
  std::string profile_json;
};

struct fg_graph {
  struct Launch {
    fg_prog* prog = nullptr;
    unsigned grid[3] = {1, 1, 1}, block[3] = {1, 1, 1}, lds = 0;
    std::vector<fg_arg> args;  // as last set on the instantiated graph
    hipGraphNode_t node = nullptr;
    hipKernelNodeParams params = {};
  };
  std::vector<Launch> launches;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  ~fg_graph() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
  }
};

namespace {
constexpr size_t kAllocGranule = 256;
constexpr size_t kSmallCopy = 1 << 16;
constexpr size_t kStagingBytes = 8 << 20;
constexpr size_t kReadbackBytes = 1 << 20;
constexpr size_t kMaxCachedBytes = size_t(96) << 30;

size_t round_up(size_t n) { return (n + kAllocGranule - 1) / kAllocGranule * kAllocGranule; }

// Copies of at least kChunkedCopy bytes go through the pinned chunks: into
// or out of pinned memory a DMA runs at about 57 GB/s each way on MI355X,
// from or to pageable memory at 15-25 GB/s, and several host threads move
// 70-90 GB/s between pageable and pinned memory where one moves 20.
constexpr size_t kChunkedCopy = size_t(4) << 20;
constexpr size_t kChunkBytes = size_t(16) << 20;

// Modules a context keeps loaded for sources compiled again. A native train
// loop's first replay compiled its batch kernels again in every call: 1.9 ms
// per call, against 0.4 ms for three steps run in full.
constexpr size_t kLoadedModules = 1024;

// A few host threads for those memcpys (created on first use; the caller
// takes a share too).
class CopyPool {
 public:
  static CopyPool& get() {
    static CopyPool* p = new CopyPool();
    return *p;
  }
  // dst[0, n) = src[0, n), split over the pool. Calls from several threads
  // (contexts used on different threads) take turns: the pool runs one job.
  void copy(void* dst, const void* src, size_t n) {
    std::lock_guard<std::mutex> one(call_m_);
    const size_t parts = std::max<size_t>(1, std::min<size_t>(workers_.size() + 1, n >> 20));
    if (parts == 1) {
      std::memcpy(dst, src, n);
      return;
    }
    const size_t piece = ((n + parts - 1) / parts + 63) / 64 * 64;  // parts * piece >= n
    auto part = [=](size_t i) {
      const size_t off = std::min(n, i * piece), end = std::min(n, off + piece);
      if (end > off) std::memcpy(static_cast<char*>(dst) + off, static_cast<const char*>(src) + off, end - off);
    };
    {
      std::lock_guard<std::mutex> lk(m_);
      job_ = part;
      next_ = 1;
      total_ = parts;
      left_ = parts - 1;
      gen_++;
    }
    cv_.notify_all();
    part(0);
    for (;;) {  // the caller helps with what the workers have not started
      size_t i;
      {
        std::lock_guard<std::mutex> lk(m_);
        if (next_ >= total_) break;
        i = next_++;
      }
      part(i);
      std::lock_guard<std::mutex> lk(m_);
      left_--;
    }
    std::unique_lock<std::mutex> lk(m_);
    done_.wait(lk, [&] { return left_ == 0; });
  }

 private:
  CopyPool() {
    const unsigned hw = std::thread::hardware_concurrency();
    const unsigned n = std::min(7u, hw > 2 ? hw / 2 - 1 : 0u);
    for (unsigned i = 0; i < n; i++)
      workers_.emplace_back([this] {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(m_);
        for (;;) {
          cv_.wait(lk, [&] { return gen_ != seen && next_ < total_; });
          seen = gen_;
          while (next_ < total_) {
            const size_t i = next_++;
            auto job = job_;
            lk.unlock();
            job(i);
            lk.lock();
            if (--left_ == 0) done_.notify_all();
          }
        }
      });
    for (auto& w : workers_) w.detach();
  }
  std::vector<std::thread> workers_;
  std::mutex call_m_, m_;
  std::condition_variable cv_, done_;
  std::function<void(size_t)> job_;
  size_t next_ = 0, total_ = 0, left_ = 0;
  uint64_t gen_ = 0;
};

int ensure_chunks(fg_ctx* c);
int release_chunks(fg_ctx* c);
// Before a HIP-stream operation while the context's AQL queue is active: the
// queue's packets complete first (defined with the queue below).
int aql_interlude(fg_ctx* c);
int aql_wait(hsa_signal_t sg);
void aql_close(AqlQueue* a);
}  // namespace

extern "C" {

const char* fg_hip_last_error(void) { return g_last_error.c_str(); }

int fg_hip_init(int ordinal, fg_ctx** out) {
  if (!out) return set_err(FG_ERR_INVALID, "fg_hip_init: null out");
  int count = 0;
  HIP_TRY(hipGetDeviceCount(&count));
  if (ordinal < 0 || ordinal >= count)
    return set_err(FG_ERR_INVALID, "fg_hip_init: device ordinal " + std::to_string(ordinal) + " out of range (" +
                                       std::to_string(count) + " devices)");
  HIP_TRY(hipSetDevice(ordinal));
  if (int rc = fg_hip_kernel_device_setup(ordinal)) return rc;
  auto* c = new fg_ctx();
  c->device = ordinal;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return set_err(FG_ERR_HIP, std::string("hipStreamCreate: ") + hipGetErrorString(e));
  }
  for (auto& ev : c->events) HIP_TRY(hipEventCreate(&ev));
  HIP_TRY(hipEventCreateWithFlags(&c->staging_event, hipEventDisableTiming));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->staging), kStagingBytes, hipHostMallocDefault));
  c->staging_size = kStagingBytes;
  HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->readback), kReadbackBytes, hipHostMallocDefault));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->async_read), FG_READ_SLOTS * FG_READ_SLOT_BYTES,
                        hipHostMallocDefault));
  for (auto& ev : c->async_events) HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  *out = c;
  return FG_OK;
}

namespace {
int ensure_chunks(fg_ctx* c) {
  for (int b = 0; b < 2; b++) {
    if (c->chunk[b]) continue;
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->chunk[b]), kChunkBytes, hipHostMallocDefault));
    HIP_TRY(hipEventCreateWithFlags(&c->chunk_event[b], hipEventDisableTiming));
  }
  return FG_OK;
}

// The chunks are given back at the end of each copy that used them. Held in
// the process, they made its host code slower afterwards: C1's realise path
// (graph key, live-tensor rewrite) ran 2-4x longer after C2's copies in most
// runs, 2.9-4.2 against 5.5-5.7 TB/s per realise, and re-allocating them
// costs the host-buffer C2 leg 52.7 -> 49.0 GB/s.
int release_chunks(fg_ctx* c) {
  for (int b = 0; b < 2; b++) {
    if (!c->chunk[b]) continue;
    if (c->chunk_pending[b]) HIP_TRY(hipEventSynchronize(c->chunk_event[b]));
    HIP_TRY(hipHostFree(c->chunk[b]));
    HIP_TRY(hipEventDestroy(c->chunk_event[b]));
    c->chunk[b] = nullptr;
    c->chunk_event[b] = nullptr;
    c->chunk_pending[b] = false;
  }
  return FG_OK;
}
}  // namespace

int fg_hip_destroy(fg_ctx* c) {
  if (!c) return FG_OK;
  // Teardown: errors here have nowhere to go, so they are not checked.
  if (c->aql) {
    (void)fg_hip_aql_end(c);
    aql_close(c->aql);
    c->aql = nullptr;
  }
  (void)hipStreamSynchronize(c->stream);
  c->loaded.clear();  // modules no program holds are unloaded here
  fg_hip_trim(c);
  for (auto& ev : c->events) (void)hipEventDestroy(ev);
  (void)hipEventDestroy(c->staging_event);
  (void)hipHostFree(c->staging);
  (void)hipHostFree(c->readback);
  (void)hipHostFree(c->async_read);
  for (int b = 0; b < 2; b++) {
    if (c->chunk[b]) (void)hipHostFree(c->chunk[b]);
    if (c->chunk_event[b]) (void)hipEventDestroy(c->chunk_event[b]);
  }
  for (auto& ev : c->async_events) (void)hipEventDestroy(ev);
  (void)hipStreamDestroy(c->stream);
  delete c;
  return FG_OK;
}

int fg_hip_alloc(fg_ctx* c, size_t nbytes, int zero, void** dptr) {
  return fg_hip_alloc_hint(c, nbytes, zero, nullptr, dptr);
}

int fg_hip_alloc_hint(fg_ctx* c, size_t nbytes, int zero, void* hint, void** dptr) {
  if (!c || !dptr) return set_err(FG_ERR_INVALID, "fg_hip_alloc: null argument");
  size_t sz = round_up(nbytes == 0 ? 1 : nbytes);
  void* p = nullptr;
  auto it = c->free_blocks.find(sz);
  if (it != c->free_blocks.end() && !it->second.empty()) {
    auto& blocks = it->second;
    size_t pick = blocks.size() - 1;
    if (hint)
      for (size_t i = blocks.size(); i-- > 0;)
        if (blocks[i] == hint) {
          pick = i;
          break;
        }
    p = blocks[pick];
    blocks[pick] = blocks.back();
    blocks.pop_back();
    c->cached_bytes -= sz;
  } else {
    hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) {
      // Give cached blocks back and retry once (the retry reports the error).
      (void)hipStreamSynchronize(c->stream);
      fg_hip_trim(c);
      HIP_TRY(hipMalloc(&p, sz));
    }
    c->sizes[p] = sz;
  }
  if (zero) {
    if (int rc = aql_interlude(c)) return rc;
    HIP_TRY(hipMemsetAsync(p, 0, sz, c->stream));
  }
  *dptr = p;
  return FG_OK;
}

int fg_hip_free(fg_ctx* c, void* p) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_free: null context");
  if (!p) return FG_OK;
  auto it = c->sizes.find(p);
  if (it == c->sizes.end()) return set_err(FG_ERR_INVALID, "fg_hip_free: pointer was not allocated by fg_hip_alloc");
  size_t sz = it->second;
  if (c->cached_bytes + sz > kMaxCachedBytes) {
    if (int rc = aql_interlude(c)) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->sizes.erase(it);
    HIP_TRY(hipFree(p));
    return FG_OK;
  }
  c->free_blocks[sz].push_back(p);
  c->cached_bytes += sz;
  return FG_OK;
}

int fg_hip_trim(fg_ctx* c) {
  if (!c) return FG_OK;
  if (int rc = aql_interlude(c)) return rc;
  HIP_TRY(hipStreamSynchronize(c->stream));
  for (auto& kv : c->free_blocks) {
    for (void* p : kv.second) {
      c->sizes.erase(p);
      HIP_TRY(hipFree(p));
    }
  }
  c->free_blocks.clear();
  c->cached_bytes = 0;
  return FG_OK;
}

int fg_hip_copy_h2d(fg_ctx* c, void* dst, const void* src, size_t n) {
  if (!c || (!dst && n) || (!src && n)) return set_err(FG_ERR_INVALID, "fg_hip_copy_h2d: null argument");
  if (int rc = aql_interlude(c)) return rc;
  if (n == 0) return FG_OK;
  if (n <= kSmallCopy) {
    // Stage through pinned memory so the copy can stay asynchronous.
    if (c->staging_head + n > c->staging_size) {
      if (c->staging_event_pending) HIP_TRY(hipEventSynchronize(c->staging_event));
      c->staging_head = 0;
    }
    char* s = c->staging + c->staging_head;
    std::memcpy(s, src, n);
    c->staging_head = (c->staging_head + n + 255) / 256 * 256;
    HIP_TRY(hipMemcpyAsync(dst, s, n, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipEventRecord(c->staging_event, c->stream));
    c->staging_event_pending = true;
    return FG_OK;
  }
  if (n >= kChunkedCopy) {
    // Pinned chunks in turn: the host fills one while the other's DMA runs.
    if (int rc = ensure_chunks(c)) return rc;
    for (size_t off = 0, i = 0; off < n; off += kChunkBytes, i++) {
      const int b = static_cast<int>(i % 2);
      const size_t len = std::min(kChunkBytes, n - off);
      if (c->chunk_pending[b]) HIP_TRY(hipEventSynchronize(c->chunk_event[b]));
      CopyPool::get().copy(c->chunk[b], static_cast<const char*>(src) + off, len);
      HIP_TRY(hipMemcpyAsync(static_cast<char*>(dst) + off, c->chunk[b], len, hipMemcpyHostToDevice, c->stream));
      HIP_TRY(hipEventRecord(c->chunk_event[b], c->stream));
      c->chunk_pending[b] = true;
    }
    return release_chunks(c);
  }
  HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return FG_OK;
}

int fg_hip_copy_d2h(fg_ctx* c, void* dst, const void* src, size_t n) {
  if (!c || (!dst && n) || (!src && n)) return set_err(FG_ERR_INVALID, "fg_hip_copy_d2h: null argument");
  if (int rc = aql_interlude(c)) return rc;
  if (n == 0) return fg_hip_sync(c);
  if (n <= kReadbackBytes) {
    HIP_TRY(hipMemcpyAsync(c->readback, src, n, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    std::memcpy(dst, c->readback, n);
    return FG_OK;
  }
  if (n >= kChunkedCopy) {
    // The DMA of chunk i+1 runs while the host copies chunk i out.
    if (int rc = ensure_chunks(c)) return rc;
    const size_t nch = (n + kChunkBytes - 1) / kChunkBytes;
    auto drain = [&](size_t i) -> int {
      const int b = static_cast<int>(i % 2);
      HIP_TRY(hipEventSynchronize(c->chunk_event[b]));
      c->chunk_pending[b] = false;
      const size_t off = i * kChunkBytes;
      CopyPool::get().copy(static_cast<char*>(dst) + off, c->chunk[b], std::min(kChunkBytes, n - off));
      return FG_OK;
    };
    for (size_t i = 0; i < nch; i++) {
      const int b = static_cast<int>(i % 2);
      const size_t off = i * kChunkBytes;
      HIP_TRY(hipMemcpyAsync(c->chunk[b], static_cast<const char*>(src) + off, std::min(kChunkBytes, n - off),
                             hipMemcpyDeviceToHost, c->stream));
      HIP_TRY(hipEventRecord(c->chunk_event[b], c->stream));
      c->chunk_pending[b] = true;
      if (i > 0)
        if (int rc = drain(i - 1)) return rc;
    }
    if (int rc = drain(nch - 1)) return rc;
    return release_chunks(c);
  }
  HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipStreamSynchronize(c->stream));
  return FG_OK;
}

int fg_hip_read_async(fg_ctx* c, int slot, const void* src, size_t n) {
  if (!c || (!src && n)) return set_err(FG_ERR_INVALID, "fg_hip_read_async: null argument");
  if (int rc = aql_interlude(c)) return rc;
  if (slot < 0 || slot >= FG_READ_SLOTS)
    return set_err(FG_ERR_INVALID, "fg_hip_read_async: slot " + std::to_string(slot) + " outside 0.." +
                                       std::to_string(FG_READ_SLOTS - 1));
  if (n > FG_READ_SLOT_BYTES)
    return set_err(FG_ERR_INVALID, "fg_hip_read_async: " + std::to_string(n) + " bytes exceed a slot's " +
                                       std::to_string(FG_READ_SLOT_BYTES));
  if (c->async_pending[slot]) HIP_TRY(hipEventSynchronize(c->async_events[slot]));  // the slot's last copy landed
  if (n) HIP_TRY(hipMemcpyAsync(c->async_read + static_cast<size_t>(slot) * FG_READ_SLOT_BYTES, src, n,
                                hipMemcpyDeviceToHost, c->stream));
  HIP_TRY(hipEventRecord(c->async_events[slot], c->stream));
  c->async_bytes[slot] = n;
  c->async_pending[slot] = true;
  return FG_OK;
}

int fg_hip_read_slot(fg_ctx* c, int slot, void** device_ptr) {
  if (!c || !device_ptr) return set_err(FG_ERR_INVALID, "fg_hip_read_slot: null argument");
  if (slot < 0 || slot >= FG_READ_SLOTS)
    return set_err(FG_ERR_INVALID, "fg_hip_read_slot: slot " + std::to_string(slot) + " outside 0.." +
                                       std::to_string(FG_READ_SLOTS - 1));
  if (c->aql && c->aql->slot_pending[slot]) {
    // Its last read-back, written by a packet of the AQL queue, landed.
    if (int rc = aql_wait(c->aql->slot_signal[slot])) return rc;
    c->aql->slot_pending[slot] = false;
    c->aql->done = std::max(c->aql->done, c->aql->slot_packet[slot] + 1);
  } else if (c->async_pending[slot]) {
    HIP_TRY(hipEventSynchronize(c->async_events[slot]));  // its last read landed
  }
  c->async_pending[slot] = false;
  HIP_TRY(hipHostGetDevicePointer(device_ptr, c->async_read + static_cast<size_t>(slot) * FG_READ_SLOT_BYTES, 0));
  return FG_OK;
}

int fg_hip_read_queued(fg_ctx* c, int slot, size_t n) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_read_queued: null context");
  if (slot < 0 || slot >= FG_READ_SLOTS)
    return set_err(FG_ERR_INVALID, "fg_hip_read_queued: slot " + std::to_string(slot) + " outside 0.." +
                                       std::to_string(FG_READ_SLOTS - 1));
  if (n > FG_READ_SLOT_BYTES)
    return set_err(FG_ERR_INVALID, "fg_hip_read_queued: " + std::to_string(n) + " bytes exceed a slot's " +
                                       std::to_string(FG_READ_SLOT_BYTES));
  // A read-back stored by a packet of the AQL queue is signalled by that
  // packet; otherwise the stream's event marks it.
  if (!(c->aql && c->aql->slot_pending[slot])) {
    if (int rc = aql_interlude(c)) return rc;
    HIP_TRY(hipEventRecord(c->async_events[slot], c->stream));
  }
  c->async_bytes[slot] = n;
  c->async_pending[slot] = true;
  return FG_OK;
}

int fg_hip_read_wait(fg_ctx* c, int slot, void* dst, size_t n) {
  if (!c || (!dst && n)) return set_err(FG_ERR_INVALID, "fg_hip_read_wait: null argument");
  if (slot < 0 || slot >= FG_READ_SLOTS || !c->async_pending[slot])
    return set_err(FG_ERR_INVALID, "fg_hip_read_wait: no read queued in slot " + std::to_string(slot));
  if (n != c->async_bytes[slot])
    return set_err(FG_ERR_INVALID, "fg_hip_read_wait: slot " + std::to_string(slot) + " holds " +
                                       std::to_string(c->async_bytes[slot]) + " bytes, " + std::to_string(n) +
                                       " asked for");
  if (c->aql && c->aql->slot_pending[slot]) {
    if (int rc = aql_wait(c->aql->slot_signal[slot])) return rc;
    c->aql->slot_pending[slot] = false;
    c->aql->done = std::max(c->aql->done, c->aql->slot_packet[slot] + 1);
  } else {
    HIP_TRY(hipEventSynchronize(c->async_events[slot]));
  }
  c->async_pending[slot] = false;
  if (n) std::memcpy(dst, c->async_read + static_cast<size_t>(slot) * FG_READ_SLOT_BYTES, n);
  return FG_OK;
}

int fg_hip_copy_d2d(fg_ctx* c, void* dst, const void* src, size_t n) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_copy_d2d: null context");
  if (int rc = aql_interlude(c)) return rc;
  if (n == 0) return FG_OK;
  HIP_TRY(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, c->stream));
  return FG_OK;
}

extern "C++" {
namespace {
// hiprtc compile of `source` into `code`.
int rtc_compile(const char* source, const char* func, std::vector<char>* code) {
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, (std::string(func) + ".hip").c_str(), 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return set_err(FG_ERR_COMPILE, std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
  r = hiprtcCompileProgram(prog, kNumRtcOptions, kRtcOptions);
  if (r != HIPRTC_SUCCESS) {
    size_t ls = 0;
    hiprtcGetProgramLogSize(prog, &ls);
    std::string log(ls, '\0');
    if (ls) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    return set_err(FG_ERR_COMPILE, "hiprtc compilation failed:\n" + log);
  }
  size_t cs = 0;
  hiprtcGetCodeSize(prog, &cs);
  code->resize(cs);
  hiprtcGetCode(prog, code->data());
  hiprtcDestroyProgram(&prog);
  return FG_OK;
}

// Where the code object of `source` is cached: a file named by the FNV-1a
// hash of the source, every compile option (the gfx950 target included) and
// the hiprtc version.
std::string cache_path(const char* source) {
  std::string key_material = std::string(source) + "\n" + hiprtc_version();
  for (int i = 0; i < kNumRtcOptions; i++) key_material += std::string("\n") + kRtcOptions[i];
  char hex[32];
  std::snprintf(hex, sizeof(hex), "%016llx", static_cast<unsigned long long>(fnv1a(key_material)));
  return cache_dir() + "/" + hex + ".co";
}
}  // namespace
}  // extern "C++"

int fg_hip_compile(fg_ctx* c, const char* source, const char* func, int num_args, fg_prog** out) {
  if (!source || !func || !out) return set_err(FG_ERR_INVALID, "fg_hip_compile: null argument");
  std::string dir = cache_dir();
  std::string path = cache_path(source);
  if (c) {
    auto hit = c->loaded.find(path);
    if (hit != c->loaded.end()) {
      auto* p = new fg_prog();
      p->num_args = num_args;
      p->name = func;
      p->module = hit->second;
      hipError_t e = hipModuleGetFunction(&p->func, p->module->module, func);
      if (e != hipSuccess) {
        delete p;
        return set_err(FG_ERR_SYMBOL, std::string("symbol '") + func + "' not found: " + hipGetErrorString(e));
      }
      *out = p;
      return FG_OK;
    }
  }
  std::vector<char> code;
  bool cached = read_file(path, &code);
  if (!cached) {
    if (int rc = rtc_compile(source, func, &code)) return rc;
    mkdir(dir.c_str(), 0755);
    write_file_atomic(path, code);
  }
  if (!c) {
    // Compile-only use (no device): the code object is now cached.
    *out = nullptr;
    return FG_OK;
  }
  auto* p = new fg_prog();
  p->num_args = num_args;
  p->name = func;
  p->module = std::make_shared<ModuleRef>();
  hipError_t e = hipModuleLoadData(&p->module->module, code.data());
  if (e != hipSuccess && cached) {
    // A cached file the runtime rejects (damaged, or written by something
    // else) is replaced by a fresh compile, once.
    std::remove(path.c_str());
    if (int rc = rtc_compile(source, func, &code)) {
      delete p;
      return rc;
    }
    write_file_atomic(path, code);
    e = hipModuleLoadData(&p->module->module, code.data());
  }
  if (e != hipSuccess) {
    delete p;
    return set_err(FG_ERR_HIP, std::string("hipModuleLoadData: ") + hipGetErrorString(e));
  }
  e = hipModuleGetFunction(&p->func, p->module->module, func);
  if (e != hipSuccess) {
    delete p;
    return set_err(FG_ERR_SYMBOL, std::string("symbol '") + func + "' not found: " + hipGetErrorString(e));
  }
  p->module->code = std::move(code);
  c->loaded[path] = p->module;
  c->loaded_order.push_back(path);
  if (c->loaded_order.size() > kLoadedModules) {
    // The oldest leaves the table; programs still using it keep it loaded.
    c->loaded.erase(c->loaded_order.front());
    c->loaded_order.pop_front();
  }
  *out = p;
  return FG_OK;
}

const char* fg_hip_code_object_path(const char* source) {
  static thread_local std::string path;
  path = cache_path(source ? source : "");
  return path.c_str();
}

int fg_hip_set_error(int code, const char* msg) { return set_err(code, msg ? msg : ""); }

int fg_hip_program_function(fg_prog* prog, const char* func, int num_args, fg_prog** out) {
  if (!prog || !func || !out) return set_err(FG_ERR_INVALID, "fg_hip_program_function: null argument");
  auto* p = new fg_prog();
  p->module = prog->module;
  p->num_args = num_args;
  p->name = func;
  hipError_t e = hipModuleGetFunction(&p->func, p->module->module, func);
  if (e != hipSuccess) {
    delete p;
    return set_err(FG_ERR_SYMBOL, std::string("symbol '") + func + "' not found: " + hipGetErrorString(e));
  }
  *out = p;
  return FG_OK;
}

int fg_hip_program_free(fg_prog* p) {
  delete p;
  return FG_OK;
}

int fg_hip_program_num_args(const fg_prog* p) { return p ? p->num_args : -1; }

namespace {
// Points params[i] at the value of args[i] (kernelParams for a HIP launch).
int marshal_args(const fg_arg* args, int nargs, void** params) {
  if (nargs > FG_MAX_LAUNCH_ARGS) return set_err(FG_ERR_ARGS, "fg_hip_launch: at most 64 arguments");
  for (int i = 0; i < nargs; i++) {
    switch (args[i].kind) {
      case FG_ARG_PTR: params[i] = const_cast<void**>(&args[i].v.p); break;
      case FG_ARG_I32: params[i] = const_cast<int32_t*>(&args[i].v.i); break;
      case FG_ARG_F32: params[i] = const_cast<float*>(&args[i].v.f); break;
      case FG_ARG_BOOL: params[i] = const_cast<uint8_t*>(&args[i].v.b); break;
      default: return set_err(FG_ERR_ARGS, "fg_hip_launch: unknown argument kind " + std::to_string(args[i].kind));
    }
  }
  return FG_OK;
}

bool same_args(const fg_arg* a, const fg_arg* b, int n) {
  for (int i = 0; i < n; i++) {
    if (a[i].kind != b[i].kind) return false;
    switch (a[i].kind) {
      case FG_ARG_PTR: if (a[i].v.p != b[i].v.p) return false; break;
      case FG_ARG_I32: if (a[i].v.i != b[i].v.i) return false; break;
      case FG_ARG_F32: if (std::memcmp(&a[i].v.f, &b[i].v.f, sizeof(float)) != 0) return false; break;
      default: if (a[i].v.b != b[i].v.b) return false; break;
    }
  }
  return true;
}
}  // namespace

namespace {
// The checks every launch makes before anything is queued.
int check_launch(const fg_ctx* c, const fg_prog* p, int nargs, const unsigned grid[3], const unsigned block[3]) {
  if (!c || !p || !grid || !block) return set_err(FG_ERR_INVALID, "fg_hip_launch: null argument");
  if (nargs != p->num_args)
    return set_err(FG_ERR_ARGS, "expected " + std::to_string(p->num_args) + " kernel args, got " + std::to_string(nargs));
  if (block[0] * block[1] * block[2] == 0 || block[0] * block[1] * block[2] > 1024)
    return set_err(FG_ERR_INVALID, "fg_hip_launch: block size must be in [1, 1024]");
  if (grid[0] == 0 || grid[1] == 0 || grid[2] == 0) return set_err(FG_ERR_INVALID, "fg_hip_launch: empty grid");
  return FG_OK;
}
}  // namespace

int fg_hip_launch_direct(fg_ctx* c, fg_prog* p, const fg_arg* args, int nargs, const unsigned grid[3],
                         const unsigned block[3], unsigned lds) {
  if (int rc = check_launch(c, p, nargs, grid, block)) return rc;
  if (int rc = aql_interlude(c)) return rc;
  void* params[FG_MAX_LAUNCH_ARGS];
  if (int rc = marshal_args(args, nargs, params)) return rc;
  HIP_TRY(hipModuleLaunchKernel(p->func, grid[0], grid[1], grid[2], block[0], block[1], block[2], lds, c->stream,
                                params, nullptr));
  return FG_OK;
}

int fg_hip_context_device(const fg_ctx* c) { return c ? c->device : -1; }

// ── Direct AQL dispatch ─────────────────────────────────────────────────────
namespace {
constexpr uint32_t kAqlQueueSize = 4096;  // packets (a power of two)
constexpr size_t kAqlArgBytes = 1024;     // argument bytes per packet
constexpr double kAqlWaitSeconds = 120.0;

int hsa_err(hsa_status_t st, const char* what) {
  const char* m = nullptr;
  hsa_status_string(st, &m);
  return set_err(FG_ERR_HIP, std::string(what) + ": " + (m ? m : "HSA error"));
}
#define HSA_TRY(expr, what)                          \
  do {                                               \
    hsa_status_t _st = (expr);                       \
    if (_st != HSA_STATUS_SUCCESS) return hsa_err(_st, what); \
  } while (0)

struct AgentSearch {
  uint32_t bdf = 0, domain = 0;
  hsa_agent_t gpu{}, cpu{};
  bool have_gpu = false, have_cpu = false;
};

hsa_status_t find_agents(hsa_agent_t a, void* data) {
  auto* s = static_cast<AgentSearch*>(data);
  hsa_device_type_t t;
  if (hsa_agent_get_info(a, HSA_AGENT_INFO_DEVICE, &t) != HSA_STATUS_SUCCESS) return HSA_STATUS_SUCCESS;
  if (t == HSA_DEVICE_TYPE_CPU && !s->have_cpu) {
    s->cpu = a;
    s->have_cpu = true;
  }
  if (t == HSA_DEVICE_TYPE_GPU && !s->have_gpu) {
    uint32_t bdf = 0, domain = 0;
    hsa_agent_get_info(a, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_BDFID), &bdf);
    hsa_agent_get_info(a, static_cast<hsa_agent_info_t>(HSA_AMD_AGENT_INFO_DOMAIN), &domain);
    if (bdf == s->bdf && domain == s->domain) {
      s->gpu = a;
      s->have_gpu = true;
    }
  }
  return HSA_STATUS_SUCCESS;
}

hsa_status_t find_fine_pool(hsa_amd_memory_pool_t p, void* data) {
  hsa_amd_segment_t seg;
  if (hsa_amd_memory_pool_get_info(p, HSA_AMD_MEMORY_POOL_INFO_SEGMENT, &seg) != HSA_STATUS_SUCCESS ||
      seg != HSA_AMD_SEGMENT_GLOBAL)
    return HSA_STATUS_SUCCESS;
  uint32_t flags = 0;
  hsa_amd_memory_pool_get_info(p, HSA_AMD_MEMORY_POOL_INFO_GLOBAL_FLAGS, &flags);
  auto* out = static_cast<std::pair<bool, hsa_amd_memory_pool_t>*>(data);
  if ((flags & HSA_AMD_MEMORY_POOL_GLOBAL_FLAG_FINE_GRAINED) && !out->first) *out = {true, p};
  return HSA_STATUS_SUCCESS;
}

void aql_close(AqlQueue* a) {
  if (!a) return;
  if (a->kargs) (void)hsa_amd_memory_pool_free(a->kargs);
  for (auto& sg : a->slot_signal)
    if (sg.handle) (void)hsa_signal_destroy(sg);
  if (a->drain.handle) (void)hsa_signal_destroy(a->drain);
  if (a->q) (void)hsa_queue_destroy(a->q);
  delete a;
  (void)hsa_shut_down();
}

int aql_open(fg_ctx* c) {
  if (c->aql) return FG_OK;
  HSA_TRY(hsa_init(), "hsa_init");  // reference-counted: the HIP runtime holds its own
  auto* a = new AqlQueue();
  auto fail = [&](int rc) {
    aql_close(a);
    return rc;
  };
  hipDeviceProp_t prop;
  hipError_t he = hipGetDeviceProperties(&prop, c->device);
  if (he != hipSuccess) return fail(set_err(FG_ERR_HIP, std::string("hipGetDeviceProperties: ") + hipGetErrorString(he)));
  AgentSearch s;
  s.bdf = (static_cast<uint32_t>(prop.pciBusID) << 8) | (static_cast<uint32_t>(prop.pciDeviceID) << 3);
  s.domain = static_cast<uint32_t>(prop.pciDomainID);
  if (hsa_status_t st = hsa_iterate_agents(find_agents, &s); st != HSA_STATUS_SUCCESS)
    return fail(hsa_err(st, "hsa_iterate_agents"));
  if (!s.have_gpu || !s.have_cpu)
    return fail(set_err(FG_ERR_HIP, "fg_hip_aql_begin: no HSA agent matches HIP device " + std::to_string(c->device)));
  a->gpu = s.gpu;
  a->cpu = s.cpu;
  std::pair<bool, hsa_amd_memory_pool_t> pool{false, {}};
  if (hsa_status_t st = hsa_amd_agent_iterate_memory_pools(a->gpu, find_fine_pool, &pool); st != HSA_STATUS_SUCCESS)
    return fail(hsa_err(st, "hsa_amd_agent_iterate_memory_pools"));
  if (!pool.first) return fail(set_err(FG_ERR_HIP, "fg_hip_aql_begin: the device has no fine-grained memory pool"));
  if (hsa_status_t st = hsa_queue_create(a->gpu, kAqlQueueSize, HSA_QUEUE_TYPE_SINGLE, nullptr, nullptr, UINT32_MAX,
                                         UINT32_MAX, &a->q);
      st != HSA_STATUS_SUCCESS)
    return fail(hsa_err(st, "hsa_queue_create"));
  if (hsa_status_t st = hsa_amd_memory_pool_allocate(pool.second, kAqlQueueSize * kAqlArgBytes, 0,
                                                     reinterpret_cast<void**>(&a->kargs));
      st != HSA_STATUS_SUCCESS)
    return fail(hsa_err(st, "hsa_amd_memory_pool_allocate"));
  if (hsa_status_t st = hsa_amd_agents_allow_access(1, &a->cpu, nullptr, a->kargs); st != HSA_STATUS_SUCCESS)
    return fail(hsa_err(st, "hsa_amd_agents_allow_access"));
  std::memset(a->kargs, 0, kAqlQueueSize * kAqlArgBytes);
  for (auto& sg : a->slot_signal)
    if (hsa_status_t st = hsa_signal_create(0, 0, nullptr, &sg); st != HSA_STATUS_SUCCESS)
      return fail(hsa_err(st, "hsa_signal_create"));
  if (hsa_status_t st = hsa_signal_create(0, 0, nullptr, &a->drain); st != HSA_STATUS_SUCCESS)
    return fail(hsa_err(st, "hsa_signal_create"));
  c->aql = a;
  return FG_OK;
}

// Waits (spinning) until `sg` drops below 1, for at most kAqlWaitSeconds.
int aql_wait(hsa_signal_t sg) {
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::duration<double>(kAqlWaitSeconds);
  while (hsa_signal_wait_scacquire(sg, HSA_SIGNAL_CONDITION_LT, 1, 1000000, HSA_WAIT_STATE_ACTIVE) >= 1)
    if (std::chrono::steady_clock::now() > deadline)
      return set_err(FG_ERR_HIP, "fg_hip_aql: a dispatched kernel did not complete within " +
                                     std::to_string(static_cast<int>(kAqlWaitSeconds)) + " s");
  return FG_OK;
}

// The next queue entry, once the packet processor has a free one and, with
// `arg_slot`, the argument slot it shares an index with is no longer read
// (the packet a whole queue earlier has completed).
int aql_reserve(AqlQueue& a, uint64_t* idx, bool arg_slot);

// Everything queued so far completes, its writes made visible to the host
// and to other queues (a barrier-AND packet with system-scope fences).
int aql_drain(AqlQueue& a) {
  uint64_t idx = 0;
  if (int rc = aql_reserve(a, &idx, false)) return rc;
  auto* p = reinterpret_cast<hsa_barrier_and_packet_t*>(a.q->base_address) + (idx & (kAqlQueueSize - 1));
  std::memset(reinterpret_cast<char*>(p) + 4, 0, sizeof(*p) - 4);
  hsa_signal_store_relaxed(a.drain, 1);
  p->completion_signal = a.drain;
  const uint16_t header = (HSA_PACKET_TYPE_BARRIER_AND << HSA_PACKET_HEADER_TYPE) | (1 << HSA_PACKET_HEADER_BARRIER) |
                          (HSA_FENCE_SCOPE_SYSTEM << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
                          (HSA_FENCE_SCOPE_SYSTEM << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE);
  __atomic_store_n(reinterpret_cast<uint32_t*>(p), static_cast<uint32_t>(header), __ATOMIC_RELEASE);
  hsa_signal_store_screlease(a.q->doorbell_signal, static_cast<hsa_signal_value_t>(idx));
  if (int rc = aql_wait(a.drain)) return rc;
  a.done = idx + 1;
  return FG_OK;
}

int aql_reserve(AqlQueue& a, uint64_t* idx, bool arg_slot) {
  uint64_t w = hsa_queue_load_write_index_relaxed(a.q);
  if (arg_slot && w >= a.done + kAqlQueueSize) {
    // A whole queue of packets since the last one known complete: wait for
    // all of them (only reached without read-backs to observe completions).
    if (int rc = aql_drain(a)) return rc;
    w = hsa_queue_load_write_index_relaxed(a.q);
  }
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::duration<double>(kAqlWaitSeconds);
  while (w - hsa_queue_load_read_index_scacquire(a.q) >= kAqlQueueSize)
    if (std::chrono::steady_clock::now() > deadline)
      return set_err(FG_ERR_HIP, "fg_hip_aql: the device read no packet for " +
                                     std::to_string(static_cast<int>(kAqlWaitSeconds)) + " s");
  *idx = hsa_queue_add_write_index_relaxed(a.q, 1);
  return FG_OK;
}

// Loads the program's module into the HSA queue's agent (once per module)
// and reads the kernel's descriptor and segment sizes.
int aql_load(AqlQueue& a, fg_prog* p) {
  if (p->aql_loaded) return FG_OK;
  ModuleRef& m = *p->module;
  if (!m.hsa_loaded) {
    if (m.code.empty()) return set_err(FG_ERR_INVALID, "fg_hip_aql_launch: no code object for " + p->name);
    HSA_TRY(hsa_code_object_reader_create_from_memory(m.code.data(), m.code.size(), &m.reader),
            "hsa_code_object_reader_create_from_memory");
    if (hsa_status_t st = hsa_executable_create_alt(HSA_PROFILE_FULL, HSA_DEFAULT_FLOAT_ROUNDING_MODE_DEFAULT, nullptr,
                                                    &m.exe);
        st != HSA_STATUS_SUCCESS) {
      (void)hsa_code_object_reader_destroy(m.reader);
      return hsa_err(st, "hsa_executable_create_alt");
    }
    hsa_status_t st = hsa_executable_load_agent_code_object(m.exe, a.gpu, m.reader, nullptr, nullptr);
    if (st == HSA_STATUS_SUCCESS) st = hsa_executable_freeze(m.exe, nullptr);
    if (st != HSA_STATUS_SUCCESS) {
      (void)hsa_executable_destroy(m.exe);
      (void)hsa_code_object_reader_destroy(m.reader);
      return hsa_err(st, "hsa_executable_load_agent_code_object");
    }
    m.hsa_loaded = true;
  }
  hsa_executable_symbol_t sym;
  HSA_TRY(hsa_executable_get_symbol_by_name(m.exe, (p->name + ".kd").c_str(), &a.gpu, &sym),
          "hsa_executable_get_symbol_by_name");
  HSA_TRY(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_OBJECT, &p->kernel_object),
          "kernel object");
  HSA_TRY(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_KERNARG_SEGMENT_SIZE, &p->kernarg_size),
          "kernarg segment size");
  HSA_TRY(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_GROUP_SEGMENT_SIZE, &p->group_size),
          "group segment size");
  HSA_TRY(hsa_executable_symbol_get_info(sym, HSA_EXECUTABLE_SYMBOL_INFO_KERNEL_PRIVATE_SEGMENT_SIZE, &p->private_size),
          "private segment size");
  p->aql_loaded = true;
  return FG_OK;
}

// The explicit arguments at their natural alignment (the AMDGPU kernel ABI:
// pointers at multiples of 8, i32/f32 of 4, bool of 1); returns the end
// offset, or 0 with `ok` false when they do not fit in `cap` bytes.
size_t aql_pack(const fg_arg* args, int nargs, char* out, size_t cap, bool* ok) {
  size_t off = 0;
  *ok = true;
  for (int i = 0; i < nargs; i++) {
    size_t sz = 0;
    const void* v = nullptr;
    switch (args[i].kind) {
      case FG_ARG_PTR: sz = 8; v = &args[i].v.p; break;
      case FG_ARG_I32: sz = 4; v = &args[i].v.i; break;
      case FG_ARG_F32: sz = 4; v = &args[i].v.f; break;
      default: sz = 1; v = &args[i].v.b; break;
    }
    off = (off + sz - 1) / sz * sz;
    if (off + sz > cap) {
      *ok = false;
      return 0;
    }
    if (out) std::memcpy(out + off, v, sz);
    off += sz;
  }
  return off;
}

// Before a HIP-stream operation while the queue is active: everything the
// queue holds completes first, and the queue's next packet waits for the
// stream (fg_hip_aql_launch synchronises it).
int aql_interlude(fg_ctx* c) {
  if (!c || !c->aql || !c->aql->active) return FG_OK;
  if (c->aql->first) return FG_OK;  // nothing queued since the stream last ran
  if (int rc = aql_drain(*c->aql)) return rc;
  c->aql->first = true;
  return FG_OK;
}
}  // namespace

}  // extern "C"

void aql_drain_before_unload() {
  if (g_active_aql && !g_active_aql->first) (void)aql_drain(*g_active_aql);
}

extern "C" {

int fg_hip_aql_begin(fg_ctx* c) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_aql_begin: null context");
  if (int rc = aql_open(c)) return rc;
  c->aql->active = true;
  c->aql->first = true;
  g_active_aql = c->aql;
  return FG_OK;
}

int fg_hip_aql_end(fg_ctx* c) {
  if (!c || !c->aql || !c->aql->active) return FG_OK;
  int rc = c->aql->first ? FG_OK : aql_drain(*c->aql);
  c->aql->active = false;
  c->aql->first = true;
  if (g_active_aql == c->aql) g_active_aql = nullptr;
  return rc;
}

int fg_hip_aql_active(const fg_ctx* c) { return c && c->aql && c->aql->active ? 1 : 0; }

int fg_hip_aql_launch(fg_ctx* c, fg_prog* p, const fg_arg* args, int nargs, const unsigned grid[3],
                      const unsigned block[3], unsigned lds, int signal_slot) {
  if (int rc = check_launch(c, p, nargs, grid, block)) return rc;
  if (!c->aql || !c->aql->active) return set_err(FG_ERR_INVALID, "fg_hip_aql_launch: no active queue");
  if (c->profiling) return FG_AQL_UNSUPPORTED;  // profiled launches keep their dispatch-attached events
  if (signal_slot >= FG_READ_SLOTS) return set_err(FG_ERR_INVALID, "fg_hip_aql_launch: read-back slot out of range");
  AqlQueue& a = *c->aql;
  if (int rc = aql_load(a, p)) return rc;
  bool fits = false;
  const size_t end = aql_pack(args, nargs, nullptr, kAqlArgBytes, &fits);
  // Kernels reading hidden arguments (a kernarg segment beyond the explicit
  // ones) and oversized argument lists take the HIP path.
  if (!fits || p->kernarg_size > kAqlArgBytes || p->kernarg_size > (end + 15) / 16 * 16) return FG_AQL_UNSUPPORTED;
  if (a.first) {
    // The stream's work (copies, zero fills, launches) precedes this packet.
    HIP_TRY(hipStreamSynchronize(c->stream));
  }
  uint64_t idx = 0;
  if (int rc = aql_reserve(a, &idx, true)) return rc;
  char* karg = a.kargs + (idx & (kAqlQueueSize - 1)) * kAqlArgBytes;
  bool ok = false;
  aql_pack(args, nargs, karg, kAqlArgBytes, &ok);
  if (p->kernarg_size > end) std::memset(karg + end, 0, p->kernarg_size - end);
  auto* pk = reinterpret_cast<hsa_kernel_dispatch_packet_t*>(a.q->base_address) + (idx & (kAqlQueueSize - 1));
  pk->workgroup_size_x = static_cast<uint16_t>(block[0]);
  pk->workgroup_size_y = static_cast<uint16_t>(block[1]);
  pk->workgroup_size_z = static_cast<uint16_t>(block[2]);
  pk->reserved0 = 0;
  pk->grid_size_x = grid[0] * block[0];
  pk->grid_size_y = grid[1] * block[1];
  pk->grid_size_z = grid[2] * block[2];
  pk->private_segment_size = p->private_size;
  pk->group_segment_size = p->group_size + lds;
  pk->kernel_object = p->kernel_object;
  pk->kernarg_address = karg;
  pk->reserved2 = 0;
  hsa_fence_scope_t release = HSA_FENCE_SCOPE_AGENT;
  pk->completion_signal = hsa_signal_t{0};
  if (signal_slot >= 0) {
    // The sequence's read-back: its store into pinned host memory is made
    // visible to the host before the slot's signal drops.
    hsa_signal_store_relaxed(a.slot_signal[signal_slot], 1);
    pk->completion_signal = a.slot_signal[signal_slot];
    a.slot_packet[signal_slot] = idx;
    a.slot_pending[signal_slot] = true;
    release = HSA_FENCE_SCOPE_SYSTEM;
  }
  const hsa_fence_scope_t acquire = a.first ? HSA_FENCE_SCOPE_SYSTEM : HSA_FENCE_SCOPE_AGENT;
  a.first = false;
  // The arguments sit in write-combined device memory: flush them before the
  // packet becomes valid.
  __builtin_ia32_sfence();
  const uint16_t dims = grid[2] * block[2] > 1 ? 3 : grid[1] * block[1] > 1 ? 2 : 1;
  const uint16_t setup = static_cast<uint16_t>(dims << HSA_KERNEL_DISPATCH_PACKET_SETUP_DIMENSIONS);
  const uint16_t header = (HSA_PACKET_TYPE_KERNEL_DISPATCH << HSA_PACKET_HEADER_TYPE) |
                          (1 << HSA_PACKET_HEADER_BARRIER) | (acquire << HSA_PACKET_HEADER_SCACQUIRE_FENCE_SCOPE) |
                          (release << HSA_PACKET_HEADER_SCRELEASE_FENCE_SCOPE);
  __atomic_store_n(reinterpret_cast<uint32_t*>(pk), header | (static_cast<uint32_t>(setup) << 16), __ATOMIC_RELEASE);
  hsa_signal_store_screlease(a.q->doorbell_signal, static_cast<hsa_signal_value_t>(idx));
  return FG_OK;
}

int fg_hip_program_resident(fg_ctx* c, fg_prog* p, unsigned block, unsigned lds, long* out) {
  if (!c || !p || !out || block == 0) return set_err(FG_ERR_INVALID, "fg_hip_program_resident: null argument");
  int per_cu = 0, cus = 0;
  HIP_TRY(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, p->func, static_cast<int>(block), lds));
  HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, c->device));
  *out = static_cast<long>(per_cu) * cus;
  return FG_OK;
}

int fg_hip_launch(fg_ctx* c, fg_prog* p, const fg_arg* args, int nargs, const unsigned grid[3],
                  const unsigned block[3], unsigned lds) {
  if (int rc = check_launch(c, p, nargs, grid, block)) return rc;
  if (int rc = aql_interlude(c)) return rc;
  void* params[FG_MAX_LAUNCH_ARGS];
  if (int rc = marshal_args(args, nargs, params)) return rc;
  if (c->profiling) {
    // Start/stop events attached to the dispatch itself, so the duration
    // excludes any host gap before the launch reaches the queue.
    hipEvent_t ea = nullptr, eb = nullptr;
    for (hipEvent_t* e : {&ea, &eb}) {
      if (!c->event_pool.empty()) {
        *e = c->event_pool.back();
        c->event_pool.pop_back();
      } else {
        HIP_TRY(hipEventCreate(e));
      }
    }
    HIP_TRY(hipExtModuleLaunchKernel(p->func, grid[0] * block[0], grid[1] * block[1], grid[2] * block[2], block[0],
                                     block[1], block[2], lds, c->stream, params, nullptr, ea, eb, 0));
    c->records.push_back({p->name, ea, eb});
    return FG_OK;
  }
  HIP_TRY(hipModuleLaunchKernel(p->func, grid[0], grid[1], grid[2], block[0], block[1], block[2], lds, c->stream,
                                params, nullptr));
  return FG_OK;
}

int fg_hip_graph_create(fg_ctx* c, int n, fg_prog* const* progs, const unsigned* grids, const unsigned* blocks,
                        const unsigned* lds, const int* nargs, const fg_arg* args, fg_graph** out) {
  if (!c || !progs || !grids || !blocks || !lds || !nargs || !args || !out || n <= 0)
    return set_err(FG_ERR_INVALID, "fg_hip_graph_create: null argument or empty sequence");
  auto g = std::make_unique<fg_graph>();
  size_t off = 0;
  for (int i = 0; i < n; i++) {
    if (!progs[i] || nargs[i] != progs[i]->num_args)
      return set_err(FG_ERR_ARGS, "fg_hip_graph_create: launch " + std::to_string(i) + " has the wrong argument count");
    fg_graph::Launch l;
    l.prog = progs[i];
    for (int d = 0; d < 3; d++) {
      l.grid[d] = grids[3 * i + d];
      l.block[d] = blocks[3 * i + d];
    }
    l.lds = lds[i];
    l.args.assign(args + off, args + off + nargs[i]);
    off += static_cast<size_t>(nargs[i]);
    g->launches.push_back(std::move(l));
  }
  // Record the sequence by capturing its launches on the context's stream
  // (nothing executes during capture), then walk the resulting chain from its
  // root so node k is launch k.
  HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
  int rc = FG_OK;
  for (auto& l : g->launches) {
    void* params[FG_MAX_LAUNCH_ARGS];
    rc = marshal_args(l.args.data(), static_cast<int>(l.args.size()), params);
    if (rc) break;
    hipError_t e = hipModuleLaunchKernel(l.prog->func, l.grid[0], l.grid[1], l.grid[2], l.block[0], l.block[1],
                                         l.block[2], l.lds, c->stream, params, nullptr);
    if (e != hipSuccess) {
      rc = set_err(FG_ERR_HIP, std::string("hipModuleLaunchKernel (capture): ") + hipGetErrorString(e));
      break;
    }
  }
  hipError_t ee = hipStreamEndCapture(c->stream, &g->graph);
  if (rc) return rc;
  if (ee != hipSuccess) return set_err(FG_ERR_HIP, std::string("hipStreamEndCapture: ") + hipGetErrorString(ee));
  size_t nroots = 0;
  HIP_TRY(hipGraphGetRootNodes(g->graph, nullptr, &nroots));
  if (nroots != 1) return set_err(FG_ERR_HIP, "fg_hip_graph_create: captured graph is not a single chain");
  hipGraphNode_t node = nullptr;
  HIP_TRY(hipGraphGetRootNodes(g->graph, &node, &nroots));
  for (size_t i = 0; i < g->launches.size(); i++) {
    g->launches[i].node = node;
    HIP_TRY(hipGraphKernelNodeGetParams(node, &g->launches[i].params));
    size_t ndep = 0;
    HIP_TRY(hipGraphNodeGetDependentNodes(node, nullptr, &ndep));
    if (i + 1 < g->launches.size()) {
      if (ndep != 1) return set_err(FG_ERR_HIP, "fg_hip_graph_create: captured graph is not a single chain");
      HIP_TRY(hipGraphNodeGetDependentNodes(node, &node, &ndep));
    } else if (ndep != 0) {
      return set_err(FG_ERR_HIP, "fg_hip_graph_create: captured graph has extra nodes");
    }
  }
  HIP_TRY(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0));
  *out = g.release();
  return FG_OK;
}

int fg_hip_graph_launch(fg_ctx* c, fg_graph* g, const fg_arg* args, int* updated) {
  if (!c || !g || !args) return set_err(FG_ERR_INVALID, "fg_hip_graph_launch: null argument");
  if (int rc = aql_interlude(c)) return rc;
  size_t off = 0;
  if (updated) *updated = 0;
  if (c->profiling) {
    for (auto& l : g->launches) {
      if (int rc = fg_hip_launch(c, l.prog, args + off, static_cast<int>(l.args.size()), l.grid, l.block, l.lds))
        return rc;
      off += l.args.size();
    }
    return FG_OK;
  }
  for (auto& l : g->launches) {
    const int n = static_cast<int>(l.args.size());
    if (!same_args(l.args.data(), args + off, n)) {
      std::copy(args + off, args + off + n, l.args.begin());
      void* params[FG_MAX_LAUNCH_ARGS];
      if (int rc = marshal_args(l.args.data(), n, params)) return rc;
      hipKernelNodeParams p = l.params;
      p.kernelParams = params;
      p.extra = nullptr;
      HIP_TRY(hipGraphExecKernelNodeSetParams(g->exec, l.node, &p));
      if (updated) ++*updated;
    }
    off += static_cast<size_t>(n);
  }
  HIP_TRY(hipGraphLaunch(g->exec, c->stream));
  return FG_OK;
}

int fg_hip_graph_free(fg_graph* g) {
  delete g;
  return FG_OK;
}

int fg_hip_profile_enable(fg_ctx* c, int on) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_profile_enable: null context");
  c->profiling = on != 0;
  return FG_OK;
}

int fg_hip_profile_read(fg_ctx* c, char* buf, size_t len, size_t* needed) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_profile_read: null context");
  if (!buf) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    std::ostringstream os;
    os << "[";
    for (size_t i = 0; i < c->records.size(); i++) {
      float ms = 0.f;
      HIP_TRY(hipEventElapsedTime(&ms, c->records[i].a, c->records[i].b));
      os << (i ? ", " : "") << "{\"kernel\": \"" << c->records[i].name << "\", \"ms\": " << ms << "}";
      c->event_pool.push_back(c->records[i].a);
      c->event_pool.push_back(c->records[i].b);
    }
    os << "]";
    c->records.clear();
    c->profile_json = os.str();
  }
  if (needed) *needed = c->profile_json.size() + 1;
  if (buf && len) {
    size_t m = std::min(len - 1, c->profile_json.size());
    std::memcpy(buf, c->profile_json.data(), m);
    buf[m] = '\0';
  }
  return FG_OK;
}

int fg_hip_sync(fg_ctx* c) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_sync: null context");
  if (int rc = aql_interlude(c)) return rc;
  HIP_TRY(hipStreamSynchronize(c->stream));
  return FG_OK;
}

int fg_hip_event_record(fg_ctx* c, int slot) {
  if (!c || slot < 0 || slot >= 64) return set_err(FG_ERR_INVALID, "fg_hip_event_record: bad slot");
  HIP_TRY(hipEventRecord(c->events[slot], c->stream));
  return FG_OK;
}

int fg_hip_event_elapsed_ms(fg_ctx* c, int a, int b, float* ms) {
  if (!c || a < 0 || a >= 64 || b < 0 || b >= 64 || !ms) return set_err(FG_ERR_INVALID, "fg_hip_event_elapsed_ms: bad slot");
  HIP_TRY(hipEventSynchronize(c->events[b]));
  HIP_TRY(hipEventElapsedTime(ms, c->events[a], c->events[b]));
  return FG_OK;
}

int fg_hip_device_info(fg_ctx* c, int* cu, int* clk, size_t* lds, char* arch, size_t arch_len) {
  if (!c) return set_err(FG_ERR_INVALID, "fg_hip_device_info: null context");
  hipDeviceProp_t p;
  HIP_TRY(hipGetDeviceProperties(&p, c->device));
  if (cu) *cu = p.multiProcessorCount;
  if (clk) *clk = p.clockRate;
  if (lds) *lds = p.sharedMemPerBlock;
  if (arch && arch_len) std::snprintf(arch, arch_len, "%s", p.gcnArchName);
  return FG_OK;
}

}  // extern "C"
