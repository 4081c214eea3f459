// The HIP device: implements the Device interface (src/device.rs:275-332) on
// top of the C-ABI in include/ferrograd_hip.h, with the gfx950 lowering in
// gpu_lower.cpp as its optimize/render stages.
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>

#include "../../include/ferrograd_hip.h"
#include "device.hpp"
#include "hip_internal.hpp"
#include "gpu_lower.hpp"
#include "tensor.hpp"

namespace fg {

namespace {

// Replayed sequences of at least this many launches are recorded as HIP
// graphs; 0 launches every sequence directly (the default, FG_HIP_GRAPHS=1
// sets 2). See graphs_enabled().
int g_graph_min_launches = [] {
  const char* e = std::getenv("FG_HIP_GRAPHS");
  return e && std::strcmp(e, "1") == 0 ? 2 : 0;
}();

void check(int rc, const char* what) {
  if (rc != FG_OK) fail(std::string(what) + ": " + fg_hip_last_error());
}

struct HipProgram : Program {
  fg_prog* prog = nullptr;             // single-launch programs
  std::vector<fg_prog*> passes;        // multi-launch programs, in launch order
  fg_ctx* ctx = nullptr;
  void* scratch = nullptr;
  ~HipProgram() override {
    fg_hip_program_free(prog);
    for (auto* p : passes) fg_hip_program_free(p);
    if (scratch && ctx) fg_hip_free(ctx, scratch);
  }
};

class HipDevice : public Device {
 public:
  DeviceId id() const override { return DeviceId::Hip; }

  fg_ctx* ctx() {
    if (!ctx_) {
      int ord = 0;
      if (const char* e = std::getenv("FG_HIP_DEVICE")) ord = std::atoi(e);
      check(fg_hip_init(ord, &ctx_), "fg_hip_init");
    }
    return ctx_;
  }

  // cpu.rs:277-280 (zero-filled). Storage is created lazily: a buffer that is
  // only ever folded to a literal 0 (relu's zeros) never touches HBM. Any read
  // (kernel input, copy_to_host) or write materialises it first.
  Buffer allocate(DType dtype, size_t numel) override {
    Buffer b = reserve_buffer(dtype, numel);
    b->known_zero = true;
    b->zero_init = true;
    return b;
  }

  void realize_storage(BufferInner& b, bool zero) override { realize_storage_at(b, zero, nullptr); }

  void realize_storage_at(BufferInner& b, bool zero, void* hint) override {
    if (b.realized) return;
    void* p = nullptr;
    check(fg_hip_alloc_hint(ctx(), b.nbytes(), zero ? 1 : 0, hint, &p), "fg_hip_alloc");
    b.storage = p;
    b.realized = true;
    b.zero_init = false;
  }

  void release(BufferInner& b) override {
    if (!b.realized || !ctx_) return;
    fg_hip_free(ctx_, b.storage);
    b.storage = nullptr;
    b.realized = false;
  }

  void copy_from_host(const Buffer& b, const void* src, size_t nbytes) override {  // cpu.rs:282-302
    FG_CHECK(b->device == DeviceId::Hip, "HIP backend received non-HIP buffer " + std::to_string(b->id));
    FG_CHECK(nbytes == b->nbytes(), "copy_from_host: expected " + std::to_string(b->nbytes()) + " bytes, got " +
                                        std::to_string(nbytes));
    realize_storage(*b, false);  // fully overwritten below
    check(fg_hip_copy_h2d(ctx(), b->storage, src, nbytes), "fg_hip_copy_h2d");
    b->known_zero = false;
  }

  std::vector<uint8_t> copy_to_host(const Buffer& b) override {  // cpu.rs:304-316
    FG_CHECK(b->device == DeviceId::Hip, "HIP backend received non-HIP buffer " + std::to_string(b->id));
    std::vector<uint8_t> out(b->nbytes());
    if (!b->realized && b->zero_init) return out;  // allocated zeros, never materialised
    FG_CHECK(b->realized, "copy_to_host called on unrealized or non-HIP buffer");
    check(fg_hip_copy_d2h(ctx(), out.data(), b->storage, out.size()), "fg_hip_copy_d2h");
    return out;
  }

  void copy_to_host_into(const Buffer& b, void* dst, size_t nbytes) override {
    FG_CHECK(b->device == DeviceId::Hip, "HIP backend received non-HIP buffer " + std::to_string(b->id));
    FG_CHECK(nbytes == b->nbytes(), "copy_to_host: expected " + std::to_string(b->nbytes()) + " bytes, got " +
                                        std::to_string(nbytes));
    if (!b->realized && b->zero_init) {  // allocated zeros, never materialised
      if (nbytes) std::memset(dst, 0, nbytes);
      return;
    }
    FG_CHECK(b->realized, "copy_to_host called on unrealized or non-HIP buffer");
    check(fg_hip_copy_d2h(ctx(), dst, b->storage, nbytes), "fg_hip_copy_d2h");
  }

  void read_async(const Buffer& b, int slot) override {
    FG_CHECK(b->device == DeviceId::Hip, "HIP backend received non-HIP buffer " + std::to_string(b->id));
    FG_CHECK(slot >= 0 && slot < FG_READ_SLOTS, "read_async: slot " + std::to_string(slot) + " out of range");
    if (!b->realized && b->zero_init) realize_storage(*b, true);  // allocated zeros, never materialised
    FG_CHECK(b->realized, "copy_to_host called on unrealized or non-HIP buffer");
    check(fg_hip_read_async(ctx(), slot, b->storage, b->nbytes()), "fg_hip_read_async");
    read_bytes_[slot] = b->nbytes();
  }

  std::vector<uint8_t> read_wait(int slot) override {
    FG_CHECK(slot >= 0 && slot < FG_READ_SLOTS, "read_wait: slot " + std::to_string(slot) + " out of range");
    std::vector<uint8_t> out(read_bytes_[slot]);
    check(fg_hip_read_wait(ctx(), slot, out.data(), out.size()), "fg_hip_read_wait");
    return out;
  }

  UOp optimize(const UOp& rangeified) override { return gpu_optimize(rangeified); }
  UOp bind_params(const UOp& optimized, const UOp& scheduled) override {
    return with_all_params(optimized, scheduled);
  }

  RenderedKernel render(const UOp& optimized, const std::string& name) override {
    (void)name;  // symbols are content-named so code objects cache across runs
    return render_hip_stable(optimized);
  }

  std::shared_ptr<Program> compile(const RenderedKernel& rk, size_t num_args) override {
    auto p = std::make_shared<HipProgram>();
    FG_CHECK(rk.params.size() == num_args || rk.params.empty(),
             "kernel declares " + std::to_string(rk.params.size()) + " parameters but is launched with " +
                 std::to_string(num_args));
    int extra = rk.scratch_bytes ? 1 : 0;
    if (rk.launches.empty()) {
      check(fg_hip_compile(ctx(), rk.source.c_str(), rk.name.c_str(), static_cast<int>(num_args) + extra, &p->prog),
            "compile failed");
    } else {
      fg_prog* first = nullptr;
      check(fg_hip_compile(ctx(), rk.source.c_str(), rk.launches[0].func.c_str(), static_cast<int>(num_args) + extra,
                           &first),
            "compile failed");
      p->passes.push_back(first);
      for (size_t i = 1; i < rk.launches.size(); i++) {
        fg_prog* q = nullptr;
        check(fg_hip_program_function(first, rk.launches[i].func.c_str(), static_cast<int>(num_args) + extra, &q),
              "compile failed");
        p->passes.push_back(q);
      }
    }
    if (rk.scratch_bytes) {
      p->ctx = ctx();
      check(fg_hip_alloc(p->ctx, rk.scratch_bytes, 0, &p->scratch), "fg_hip_alloc (scratch)");
    }
    p->num_args = num_args;
    p->meta = rk;
    return p;
  }

  // The launch arguments of one program execution: the kernel arguments in
  // slot order, then the program's scratch buffer if it has one.
  std::vector<fg_arg> marshal(HipProgram& p, std::vector<KernelArg>& args) {
    FG_CHECK(args.size() == p.num_args,
             "expected " + std::to_string(p.num_args) + " kernel args, got " + std::to_string(args.size()));
    std::vector<fg_arg> a(args.size());
    for (size_t i = 0; i < args.size(); i++) {
      std::memset(&a[i], 0, sizeof(fg_arg));
      switch (args[i].kind) {
        case KernelArg::Kind::Buffer:
          FG_CHECK(args[i].buffer->device == DeviceId::Hip && args[i].buffer->realized,
                   "HIP backend received unrealized or non-HIP buffer");
          a[i].kind = FG_ARG_PTR;
          a[i].v.p = args[i].buffer->storage;
          break;
        case KernelArg::Kind::I32: a[i].kind = FG_ARG_I32; a[i].v.i = args[i].i; break;
        case KernelArg::Kind::F32: a[i].kind = FG_ARG_F32; a[i].v.f = args[i].f; break;
        case KernelArg::Kind::Bool: a[i].kind = FG_ARG_BOOL; a[i].v.b = args[i].b ? 1 : 0; break;
      }
    }
    if (p.scratch) {
      fg_arg s;
      std::memset(&s, 0, sizeof(s));
      s.kind = FG_ARG_PTR;
      s.v.p = p.scratch;
      a.push_back(s);
    }
    return a;
  }

  void execute(Program& prog, std::vector<KernelArg>& args) override {  // cpu.rs:328-380
    auto& p = static_cast<HipProgram&>(prog);
    std::vector<fg_arg> a = marshal(p, args);
    if (p.passes.empty()) {
      check(fg_hip_launch(ctx(), p.prog, a.data(), static_cast<int>(a.size()), p.meta.grid, p.meta.block,
                          p.meta.lds_bytes),
            "execution failed");
      return;
    }
    for (size_t i = 0; i < p.passes.size(); i++) {
      const LaunchSpec& l = p.meta.launches[i];
      check(fg_hip_launch(ctx(), p.passes[i], a.data(), static_cast<int>(a.size()), l.grid, l.block, l.lds_bytes),
            "execution failed");
    }
  }

  // A replayed plan: its runs of block kernels batched, independent small
  // GEMMs paired or run beside a batch, then launched kernel by kernel (in
  // the native loop's replay brackets, as packets of the context's own AQL
  // queue); with graphs on, recorded once as a HIP graph from its second use
  // and replayed through it (one graph launch, with only the changed launch
  // arguments updated; a sequence whose graph cannot be built keeps
  // launching one by one).
  void execute_sequence(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                        std::shared_ptr<void>& state) override {
    run_sequence(progs, args, state, nullptr);
  }

  // The read-back of `result` as part of the sequence, storing straight into
  // the pinned slot: the captured train step then reads its loss with no
  // separate copy behind its graph (that copy and the gap before it were
  // about 12 us of a 55 us C4 step under the profiler). When the sequence
  // ends in a block kernel or a batch of them, the copy is that launch's last
  // stage; otherwise it is one more kernel.
  void execute_sequence_read(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                             std::shared_ptr<void>& state, const Buffer& result, int slot) override {
    const size_t nb = result->nbytes();
    if (nb % 4 != 0 || nb > FG_READ_SLOT_BYTES || !result->realized) {
      Device::execute_sequence_read(progs, args, state, result, slot);
      return;
    }
    void* dst = nullptr;
    check(fg_hip_read_slot(ctx(), slot, &dst), "fg_hip_read_slot");
    Readback rb{dst, result->storage, static_cast<int>(nb / 4), slot};
    run_sequence(progs, args, state, &rb);
    check(fg_hip_read_queued(ctx(), slot, nb), "fg_hip_read_queued");
    read_bytes_[slot] = nb;
  }

 private:
  // A launch running small GEMMs beside a batch (render_hbatch): the GEMM
  // programs (launch order), the batch's programs, the programs the launch
  // covers, and its launch.
  struct HBatch {
    std::vector<size_t> hb;
    size_t stage_first = 0, stage_count = 0;
    size_t span_first = 0, span_count = 0;
    std::shared_ptr<Program> prog;
  };

  struct Readback {
    void* dst;        // device address of a pinned read-back slot
    const void* src;  // the result's device buffer
    int words;        // 32-bit words to copy
    int slot;         // the read-back slot
  };

  // The kernel that copies a read-back into its slot: lane-indexed 32-bit
  // vector stores into pinned host memory.
  HipProgram& readback_program() {
    if (!readback_) {
      RenderedKernel rk;
      rk.name = "fg_readback";
      rk.kind = "readback";
      rk.source =
          "extern \"C\" __global__ void __launch_bounds__(64) fg_readback(unsigned int* dst, const unsigned int* src, "
          "int words) {\n  for (int i = threadIdx.x; i < words; i += 64) dst[i] = src[i];\n}\n";
      rk.block[0] = 64;
      readback_ = compile(rk, 3);
    }
    return static_cast<HipProgram&>(*readback_);
  }

  void run_sequence(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                    std::shared_ptr<void>& state, const Readback* rb) {
    struct Replay {
      int uses = 0;
      bool failed = false;
      bool readback = false;  // whether the recorded graph ends with a read-back
      fg_graph* graph = nullptr;
      // Runs of consecutive block kernels that launch as one batch: (first
      // program, count) and the batch program of each.
      std::vector<std::pair<size_t, size_t>> groups;
      std::vector<std::shared_ptr<Program>> batches;
      // Pairs of adjacent independent kernels launched together
      // (render_hfused): the first program of each pair, and its launch.
      std::vector<size_t> pair_first;
      std::vector<std::shared_ptr<Program>> pairs;
      std::vector<size_t> order;  // launch order of the programs (empty: as given)
      // The sequence's last launch with the read-back as its last stage, when
      // that launch is a block kernel or a batch of them: from program
      // rb_first (in launch order) to the end.
      std::shared_ptr<Program> rb_batch;
      size_t rb_first = 0;
      // With the read-back launch running a small GEMM (or a pair) beside
      // its batch (render_hbatch): those programs, and the batch's first.
      std::vector<size_t> rb_hb;
      size_t rb_stage_first = 0;
      // Launches that run a small GEMM or a pair of them beside an
      // independent batch (render_hbatch).
      std::vector<HBatch> hbatches;
      ~Replay() { fg_hip_graph_free(graph); }
    };
    if (!state) state = std::make_shared<Replay>();
    auto* r = static_cast<Replay*>(state.get());
    r->uses++;
    if (r->graph && r->readback != (rb != nullptr)) {
      // Called with and without a read-back: record the graph again.
      fg_hip_graph_free(r->graph);
      r->graph = nullptr;
      r->uses = 2;
    }
    if (r->uses == 1 && gpu_passes().batch) {
      r->order = sink_blocks(progs, args);
      std::vector<Program*> ordered;
      std::vector<std::vector<KernelArg>> ordered_args;
      for (size_t i = 0; i < progs.size(); i++) {
        const size_t k = r->order.empty() ? i : r->order[i];
        ordered.push_back(progs[k]);
        ordered_args.push_back(args[k]);
      }
      group_blocks(ordered, ordered_args, r->groups, r->batches);
      if (pairs_on()) pair_kernels(ordered, ordered_args, r->groups, r->pair_first, r->pairs);
      if (hbatch_on()) hbatch_kernels(ordered, ordered_args, r->groups, r->pair_first, r->hbatches);
    }
    auto prog_at = [&](size_t i) -> Program* { return r->order.empty() ? progs[i] : progs[r->order[i]]; };
    auto args_at = [&](size_t i) -> std::vector<KernelArg>& { return r->order.empty() ? args[i] : args[r->order[i]]; };
    if (rb && gpu_passes().batch && !r->rb_batch && !progs.empty()) {
      size_t first = progs.size(), count = 0;
      if (!r->groups.empty() && r->groups.back().first + r->groups.back().second == progs.size()) {
        first = r->groups.back().first;
        count = r->groups.back().second;
      } else if (is_block_program(*prog_at(progs.size() - 1))) {
        first = progs.size() - 1;
        count = 1;
      }
      std::vector<const RenderedKernel*> stages;
      size_t total = 3;  // the read-back stage's destination, source and word count
      for (size_t j = first; j < first + count; j++) {
        stages.push_back(&prog_at(j)->meta);
        total += args_at(j).size();
      }
      // With no room left for the read-back's arguments, the read-back stays
      // a kernel of its own after the batch.
      if (count && total <= FG_MAX_LAUNCH_ARGS) {
        std::vector<Program*> ordered;
        std::vector<std::vector<KernelArg>> ordered_args;
        for (size_t j = 0; j < progs.size(); j++) {
          ordered.push_back(prog_at(j));
          ordered_args.push_back(args_at(j));
        }
        const BatchForwarding fwd = forwarding_of(ordered, ordered_args, first, count);
        // The batch's planned hbatch, when its small GEMM part comes first:
        // the read-back launch runs that part too.
        for (const HBatch& h : r->hbatches) {
          if (h.stage_first != first || h.stage_count != count || h.hb.back() >= first) continue;
          std::vector<const RenderedKernel*> hbm;
          size_t hb_args = 0;
          for (size_t j : h.hb) {
            hbm.push_back(&ordered[j]->meta);
            hb_args += ordered_args[j].size();
          }
          if (total + hb_args > FG_MAX_LAUNCH_ARGS) break;
          auto prog = compile(render_hbatch(hbm, stages, true, forwarding_on() ? &fwd : nullptr), total + hb_args);
          if (!fits_resident(static_cast<HipProgram&>(*prog))) break;
          r->rb_batch = prog;
          r->rb_first = h.hb.front();
          r->rb_hb = h.hb;
          r->rb_stage_first = first;
          break;
        }
        if (!r->rb_batch) {
          r->rb_batch = compile(render_block_batch(stages, true, forwarding_on() ? &fwd : nullptr), total);
          r->rb_first = first;
          r->rb_stage_first = first;
          r->rb_hb.clear();
        }
      }
    }
    const bool fold_rb = rb && r->rb_batch;
    auto rb_args = [&]() {
      std::vector<fg_arg> a(3);
      std::memset(a.data(), 0, a.size() * sizeof(fg_arg));
      a[0].kind = FG_ARG_PTR;
      a[0].v.p = rb->dst;
      a[1].kind = FG_ARG_PTR;
      a[1].v.p = const_cast<void*>(rb->src);
      a[2].kind = FG_ARG_I32;
      a[2].v.i = rb->words;
      return a;
    };
    std::vector<fg_prog*> lp;
    std::vector<unsigned> grids, blocks, lds;
    std::vector<int> nargs;
    std::vector<fg_arg> all;
    auto add = [&](fg_prog* fp, const unsigned* g, const unsigned* b, unsigned l, const std::vector<fg_arg>& a) {
      lp.push_back(fp);
      grids.insert(grids.end(), g, g + 3);
      blocks.insert(blocks.end(), b, b + 3);
      lds.push_back(l);
      nargs.push_back(static_cast<int>(a.size()));
      all.insert(all.end(), a.begin(), a.end());
    };
    size_t next_group = 0, next_pair = 0, next_hbatch = 0;
    auto append = [&](std::vector<fg_arg>& a, size_t j) {
      std::vector<fg_arg> aj = marshal(static_cast<HipProgram&>(*prog_at(j)), args_at(j));
      a.insert(a.end(), aj.begin(), aj.end());
    };
    for (size_t i = 0; i < progs.size(); i++) {
      if (fold_rb && i == r->rb_first) {
        std::vector<fg_arg> a;
        for (size_t j : r->rb_hb) append(a, j);
        for (size_t j = r->rb_stage_first; j < progs.size(); j++) append(a, j);
        std::vector<fg_arg> ra = rb_args();
        a.insert(a.end(), ra.begin(), ra.end());
        auto& bp = static_cast<HipProgram&>(*r->rb_batch);
        add(bp.prog, bp.meta.grid, bp.meta.block, bp.meta.lds_bytes, a);
        break;
      }
      while (next_hbatch < r->hbatches.size() && r->hbatches[next_hbatch].span_first < i) next_hbatch++;
      if (next_hbatch < r->hbatches.size() && r->hbatches[next_hbatch].span_first == i) {
        const HBatch& h = r->hbatches[next_hbatch++];
        const size_t end = h.span_first + h.span_count;
        // The sequence's last batch carries the read-back instead.
        if (!(fold_rb && end == progs.size())) {
          std::vector<fg_arg> a;
          for (size_t j : h.hb) append(a, j);
          for (size_t j = h.stage_first; j < h.stage_first + h.stage_count; j++) append(a, j);
          auto& hp = static_cast<HipProgram&>(*h.prog);
          add(hp.prog, hp.meta.grid, hp.meta.block, hp.meta.lds_bytes, a);
          while (next_group < r->groups.size() && r->groups[next_group].first < end) next_group++;
          while (next_pair < r->pair_first.size() && r->pair_first[next_pair] < end) next_pair++;
          i = end - 1;
          continue;
        }
      }
      if (next_group < r->groups.size() && r->groups[next_group].first == i) {
        const size_t n = r->groups[next_group].second;
        std::vector<fg_arg> a;
        for (size_t j = i; j < i + n; j++) {
          std::vector<fg_arg> aj = marshal(static_cast<HipProgram&>(*prog_at(j)), args_at(j));
          a.insert(a.end(), aj.begin(), aj.end());
        }
        auto& bp = static_cast<HipProgram&>(*r->batches[next_group]);
        add(bp.prog, bp.meta.grid, bp.meta.block, bp.meta.lds_bytes, a);
        next_group++;
        i += n - 1;
        continue;
      }
      if (next_pair < r->pair_first.size() && r->pair_first[next_pair] == i) {
        std::vector<fg_arg> a = marshal(static_cast<HipProgram&>(*prog_at(i)), args_at(i));
        std::vector<fg_arg> b = marshal(static_cast<HipProgram&>(*prog_at(i + 1)), args_at(i + 1));
        a.insert(a.end(), b.begin(), b.end());
        auto& pp = static_cast<HipProgram&>(*r->pairs[next_pair]);
        add(pp.prog, pp.meta.grid, pp.meta.block, pp.meta.lds_bytes, a);
        next_pair++;
        i++;
        continue;
      }
      auto& p = static_cast<HipProgram&>(*prog_at(i));
      std::vector<fg_arg> a = marshal(p, args_at(i));
      if (p.passes.empty()) add(p.prog, p.meta.grid, p.meta.block, p.meta.lds_bytes, a);
      for (size_t k = 0; k < p.passes.size(); k++)
        add(p.passes[k], p.meta.launches[k].grid, p.meta.launches[k].block, p.meta.launches[k].lds_bytes, a);
    }
    if (rb && !fold_rb) {
      HipProgram& p = readback_program();
      add(p.prog, p.meta.grid, p.meta.block, 0, rb_args());
    }
    if (aql_on_) {
      // The replay loop's direct queue: one AQL packet per launch, the last
      // one completing the read-back slot when the sequence stores into it.
      size_t off = 0;
      for (size_t i = 0; i < lp.size(); i++) {
        const int sig = rb && i + 1 == lp.size() ? rb->slot : -1;
        int rc = fg_hip_aql_launch(ctx(), lp[i], all.data() + off, nargs[i], &grids[3 * i], &blocks[3 * i], lds[i], sig);
        if (rc == FG_AQL_UNSUPPORTED)
          rc = fg_hip_launch(ctx(), lp[i], all.data() + off, nargs[i], &grids[3 * i], &blocks[3 * i], lds[i]);
        check(rc, "execution failed");
        off += static_cast<size_t>(nargs[i]);
      }
      return;
    }
    if (graphs_enabled() && !r->failed && !r->graph && r->uses >= 2 &&
        lp.size() >= static_cast<size_t>(graph_min_launches())) {
      if (fg_hip_graph_create(ctx(), static_cast<int>(lp.size()), lp.data(), grids.data(), blocks.data(), lds.data(),
                              nargs.data(), all.data(), &r->graph) != FG_OK) {
        r->failed = true;
        r->graph = nullptr;
      }
      r->readback = rb != nullptr;
    }
    if (r->graph) {
      int updated = 0;
      check(fg_hip_graph_launch(ctx(), r->graph, all.data(), &updated), "execution failed");
      realize_stats().graph_replays++;
      realize_stats().graph_updates += static_cast<size_t>(updated);
      return;
    }
    size_t off = 0;
    for (size_t i = 0; i < lp.size(); i++) {
      check(fg_hip_launch(ctx(), lp[i], all.data() + off, nargs[i], &grids[3 * i], &blocks[3 * i], lds[i]),
            "execution failed");
      off += static_cast<size_t>(nargs[i]);
    }
  }

  // FG_PAIRS=0 launches every kernel of a sequence on its own (read once);
  // pairs also need the batch pass (OPT).
  static bool pairs_on() {
    static const bool on = [] {
      const char* e = std::getenv("FG_PAIRS");
      return !(e && std::strcmp(e, "0") == 0);
    }();
    return on && gpu_passes().batch;
  }

  // Adjacent kernels of the sequence that share one launch (pair_runs,
  // render_hfused); kernels in a batch stay out of pairs. Buffers are told
  // apart by identity, as in forwarding_of.
  void pair_kernels(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                    const std::vector<std::pair<size_t, size_t>>& groups, std::vector<size_t>& pair_first,
                    std::vector<std::shared_ptr<Program>>& pairs) {
    const size_t n = progs.size();
    std::vector<bool> grouped(n, false);
    for (auto [f, c] : groups)
      for (size_t j = f; j < f + c; j++) grouped[j] = true;
    std::vector<const RenderedKernel*> metas;
    std::vector<std::vector<BatchArg>> info;
    for (size_t i = 0; i < n; i++) {
      metas.push_back(&progs[i]->meta);
      info.emplace_back();
      for (auto& a : args[i])
        info.back().push_back(a.kind == KernelArg::Kind::Buffer ? BatchArg{a.buffer.get(), a.buffer->numel}
                                                                 : BatchArg{});
      if (static_cast<HipProgram&>(*progs[i]).scratch) grouped[i] = true;
    }
    for (size_t i : pair_runs(metas, info, grouped)) {
      pairs.push_back(compile(render_hfused(progs[i]->meta, progs[i + 1]->meta), args[i].size() + args[i + 1].size()));
      pair_first.push_back(i);
    }
  }

  // FG_HBATCH=0 launches small GEMMs apart from the batches (read once);
  // hbatches also need the batch pass (OPT).
  static bool hbatch_on() {
    static const bool on = [] {
      const char* e = std::getenv("FG_HBATCH");
      return !(e && std::strcmp(e, "0") == 0);
    }();
    return on && gpu_passes().batch;
  }

  // Whether every workgroup of a launch is resident at once, so the batch's
  // workgroup and the small GEMM's run side by side in one round.
  bool fits_resident(HipProgram& p) {
    long cap = 0;
    check(fg_hip_program_resident(ctx(), p.prog, p.meta.block[0], p.meta.lds_bytes, &cap), "fg_hip_program_resident");
    return cap >= static_cast<long>(p.meta.grid[0]);
  }

  // Batches that run beside an adjacent independent small GEMM or pair in one
  // launch (hbatch_runs, render_hbatch), each kept only when all of its
  // workgroups fit on the device at once.
  void hbatch_kernels(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                      const std::vector<std::pair<size_t, size_t>>& groups, const std::vector<size_t>& pair_first,
                      std::vector<HBatch>& out) {
    std::vector<const RenderedKernel*> metas;
    std::vector<std::vector<BatchArg>> info;
    for (size_t i = 0; i < progs.size(); i++) {
      metas.push_back(&progs[i]->meta);
      info.emplace_back();
      for (auto& a : args[i])
        info.back().push_back(a.kind == KernelArg::Kind::Buffer ? BatchArg{a.buffer.get(), a.buffer->numel}
                                                                 : BatchArg{});
    }
    for (const HBatchRun& run : hbatch_runs(metas, info, groups, pair_first)) {
      const auto [first, count] = groups[run.group];
      std::vector<const RenderedKernel*> hbm, stages;
      size_t total = 0;
      for (size_t j : run.hb) {
        hbm.push_back(metas[j]);
        total += args[j].size();
      }
      for (size_t j = first; j < first + count; j++) {
        stages.push_back(metas[j]);
        total += args[j].size();
      }
      const BatchForwarding fwd = forwarding_of(progs, args, first, count);
      auto prog = compile(render_hbatch(hbm, stages, false, forwarding_on() ? &fwd : nullptr), total);
      if (!fits_resident(static_cast<HipProgram&>(*prog))) continue;
      HBatch h;
      h.hb = run.hb;
      h.stage_first = first;
      h.stage_count = count;
      h.span_first = std::min(run.hb.front(), first);
      h.span_count = run.hb.size() + count;
      h.prog = prog;
      out.push_back(std::move(h));
    }
  }

  // FG_BATCH_LDS=0 keeps every batch stage's output in its buffer (read once).
  static bool forwarding_on() {
    static const bool on = [] {
      const char* e = std::getenv("FG_BATCH_LDS");
      return !(e && std::strcmp(e, "0") == 0);
    }();
    return on;
  }

  // A block kernel: one workgroup, a single launch, no scratch; its body can
  // run as a stage of a batch.
  static bool is_block_program(Program& prog) {
    auto& p = static_cast<HipProgram&>(prog);
    return !p.meta.stage_fn.empty() && p.passes.empty() && !p.scratch;
  }

  // A launch order in which block kernels sit next to each other where the
  // data allow: a block kernel moves later, past kernels it shares no buffer
  // with (neither reads what the other writes, nor both write one buffer),
  // when that brings it up to the next block kernel. Buffers are told apart by
  // their device addresses in this first call: within one sequence every
  // output is a fresh allocation and every input is live, so equal addresses
  // are the same buffer in every later call too. Empty when nothing moves.
  std::vector<size_t> sink_blocks(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args) {
    const size_t n = progs.size();
    auto is_block = [&](size_t i) { return is_block_program(*progs[i]); };
    std::vector<std::set<void*>> reads(n), writes(n);
    for (size_t i = 0; i < n; i++) {
      const RenderedKernel& m = progs[i]->meta;
      for (size_t j = 0; j < args[i].size(); j++) {
        if (args[i][j].kind != KernelArg::Kind::Buffer || !args[i][j].buffer->realized) continue;
        void* ptr = args[i][j].buffer->storage;
        const bool out = j < m.params.size() && m.params[j].first == m.out_slot;
        (out ? writes : reads)[i].insert(ptr);
        if (out) reads[i].insert(ptr);  // an in-place update also reads its destination
      }
    }
    auto independent = [&](size_t a, size_t b) {
      for (void* w : writes[a])
        if (reads[b].count(w) || writes[b].count(w)) return false;
      for (void* w : writes[b])
        if (reads[a].count(w)) return false;
      return true;
    };
    std::vector<size_t> order(n);
    for (size_t i = 0; i < n; i++) order[i] = i;
    bool moved = false;
    for (size_t pos = 0; pos < n; pos++) {
      const size_t k = order[pos];
      if (!is_block(k) || (pos + 1 < n && is_block(order[pos + 1]))) continue;
      size_t q = pos + 1;
      while (q < n && !is_block(order[q]) && independent(k, order[q])) q++;
      if (q == pos + 1 || q == n || !is_block(order[q])) continue;
      // Move k from pos to just before q (after the kernels it passed).
      order.erase(order.begin() + static_cast<long>(pos));
      order.insert(order.begin() + static_cast<long>(q - 1), k);
      moved = true;
      pos--;  // re-examine the kernel that slid into pos
    }
    if (!moved) order.clear();
    return order;
  }

  // The LDS forwarding of the batch of progs[first, first + n): buffers are
  // told apart by identity (within one sequence every output is a buffer of
  // its own and every input a live one).
  static BatchForwarding forwarding_of(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                                       size_t first, size_t n) {
    std::vector<const RenderedKernel*> stages;
    std::vector<std::vector<BatchArg>> info;
    for (size_t j = first; j < first + n; j++) {
      stages.push_back(&progs[j]->meta);
      info.emplace_back();
      for (auto& a : args[j])
        info.back().push_back(a.kind == KernelArg::Kind::Buffer ? BatchArg{a.buffer.get(), a.buffer->numel}
                                                                 : BatchArg{});
    }
    return batch_forwarding(stages, info);
  }

  // Runs of two or more consecutive block kernels (one workgroup each, no
  // scratch) in a sequence (block_batch_runs): each becomes one launch of a
  // batch program that runs the kernels' bodies in order behind workgroup
  // barriers, its stages' outputs handed on through LDS (batch_forwarding).
  // The batch's code object is cached by its source like any other.
  void group_blocks(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                    std::vector<std::pair<size_t, size_t>>& groups, std::vector<std::shared_ptr<Program>>& batches) {
    std::vector<bool> is_block;
    std::vector<size_t> nargs;
    for (size_t i = 0; i < progs.size(); i++) {
      is_block.push_back(is_block_program(*progs[i]));
      nargs.push_back(args[i].size());
    }
    for (auto [first, n] : block_batch_runs(is_block, nargs)) {
      std::vector<const RenderedKernel*> stages;
      size_t total = 0;
      for (size_t j = first; j < first + n; j++) {
        stages.push_back(&progs[j]->meta);
        total += args[j].size();
      }
      const BatchForwarding fwd = forwarding_of(progs, args, first, n);
      batches.push_back(compile(render_block_batch(stages, false, forwarding_on() ? &fwd : nullptr), total));
      groups.emplace_back(first, n);
    }
  }

  // Replayed sequences launch kernel by kernel unless graphs are on
  // (graph_min_launches() >= 2: FG_HIP_GRAPHS=1, or fg_set_graph_min_launches).
  // Measured on MI355X, queued behind a spinning kernel so the host does not
  // matter: a dependent direct launch costs the device 1.5-1.75 us, a kernel
  // node of a replayed graph 2.8-3.0 us. On the host a direct launch costs
  // about 2.5 us, a graph launch about 20 us plus under 1 us per node. C4
  // (five launches per step) on one box: 24.2-28.3K steps/s direct against
  // 21.8-22.7K as graphs, 8.6-8.8K against 6.3-6.5K driven from Python; C5
  // (24 launches, 6.9 ms) 144.6-144.8 against 143.8-144.5.
  static bool graphs_enabled() { return graph_min_launches() >= 2; }

 public:
  void synchronize() override {
    if (ctx_) check(fg_hip_sync(ctx_), "fg_hip_sync");
  }

  // FG_AQL=0 keeps the replay loop on hipModuleLaunchKernel (read once). On
  // a context whose HSA queue cannot be opened the loop keeps it too.
  void begin_replay_loop() override {
    static const bool on = [] {
      const char* e = std::getenv("FG_AQL");
      return !(e && std::strcmp(e, "0") == 0);
    }();
    if (!on || aql_failed_ || aql_on_) return;
    if (fg_hip_aql_begin(ctx()) != FG_OK) {
      aql_failed_ = true;
      if (debug_level() >= 1) std::fprintf(stderr, "*** HIP direct queue unavailable: %s\n", fg_hip_last_error());
      return;
    }
    aql_on_ = true;
  }

  void end_replay_loop() override {
    if (!aql_on_) return;
    aql_on_ = false;
    check(fg_hip_aql_end(ctx()), "fg_hip_aql_end");
  }

  bool shares_relu_zeros() const override { return true; }

  // FG_FUSE=0, or an OPT list without "fuse", keeps the reference's kernel
  // partition (read once per process).
  bool fuse_elementwise() const override {
    static const bool on = [] {
      const char* e = std::getenv("FG_FUSE");
      return !(e && std::strcmp(e, "0") == 0) && gpu_passes().fuse;
    }();
    return on;
  }

 private:
  fg_ctx* ctx_ = nullptr;
  bool aql_on_ = false, aql_failed_ = false;
  size_t read_bytes_[FG_READ_SLOTS] = {};
  std::shared_ptr<Program> readback_;
};

}  // namespace

Device* make_hip_device() { return new HipDevice(); }

int graph_min_launches() { return g_graph_min_launches; }

int set_graph_min_launches(int n) {
  FG_CHECK(n == 0 || n >= 2,
           "graph_min_launches: 0 (no graphs) or a recorded graph of at least 2 launches, got " + std::to_string(n));
  int prev = g_graph_min_launches;
  g_graph_min_launches = n;
  return prev;
}

void* hip_context_raw() {
  auto& d = static_cast<HipDevice&>(get_device(DeviceId::Hip));
  return d.ctx();
}

}  // namespace fg
