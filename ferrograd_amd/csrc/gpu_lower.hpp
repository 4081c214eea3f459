// gfx950 lowering of rangeified kernels: kernel classification (the GPU
// optimize passes) and HIP source generation (the HIP codegen target).
#pragma once

#include <map>
#include <string>
#include <vector>

#include "device.hpp"
#include "ir.hpp"

namespace fg {

// An int32 index expression as c0 + sum(coef * term), where each term is a
// Range or a ParamScalar. Rangeify only builds Add/Mul/Const over those
// (schedule/indexing.rs:42-62, 102-175), so every index is affine.
struct Affine {
  bool ok = true;
  int64_t c0 = 0;
  std::vector<std::pair<UOp, int64_t>> terms;
  int64_t coef(const UOp& t) const;
  bool has_scalar_terms() const;
};
Affine affine_of(const UOp& e);

// The shape of one rangeified kernel: Sink(End(r0, ... End(rn, Store(idx, v)))).
struct KernelInfo {
  UOp store, out_index, value, out_param;
  std::vector<UOp> out_ranges;  // outermost first
  std::vector<int64_t> out_ext;
  std::vector<UOp> reduces;     // Reduce nodes in the stored value
  std::vector<std::pair<int, UOp>> params;  // slot -> ParamBuffer / ParamScalar
};
KernelInfo analyze_kernel(const UOp& sink);
int64_t range_extent(const UOp& r);

// Lowering classes, in the order they are tried.
// Sequential: an in-place update that reads its destination at another
// index, run by one thread in the reference's loop order.
enum class KernelClass { Gemm, Elementwise, RowReduce, ColumnReduce, Serial, NarrowGemm, Block, Sequential };
const char* kernel_class_name(KernelClass k);

// The HIP path's optional passes, selected by the OPT environment variable
// with the reference's grammar (src/optimize/mod.rs:85-112): unset, empty,
// "1", "on" or "all" enable every pass; "0", "off" or "none" disable them
// all; otherwise a comma-separated list enables the passes it names. Names
// the HIP path does not know (the CPU backend's "upcast", "unroll") are
// ignored here, as the reference ignores unknown names. With a pass off, the
// kernels it would have produced are lowered by the generic classes instead
// (row/column reductions, serial loops; the reference's kernel partition).
struct GpuPasses {
  bool symbolic = true;  // constant and identity folding before lowering
  bool mfma = true;      // MUL-over-broadcast + REDUCE as fp32 MFMA tiles
  bool narrow = true;    // products with a side of 16 or fewer as VALU row/column kernels
  bool fuse = true;      // schedule-time value-preserving fusion (also off with FG_FUSE=0)
  bool block = true;     // small kernels as one 1024-thread workgroup ("_blk")
  bool batch = true;     // consecutive block kernels of a replayed sequence in one launch
};
GpuPasses parse_gpu_passes(const char* raw);
// OPT as read once per process.
const GpuPasses& gpu_passes();

// `kernel` (lowered from the scheduled kernel `scheduled`) with every kernel
// parameter `scheduled` has: one that index simplification or a fold took out
// of the body (a Shrink start times the zero stride of an extent-0 axis, a
// load multiplied by 0) rides along as an extra source of the Sink, so the
// rendered kernel still declares it and its launch arguments keep their
// slots. (The reference renders only the parameters left in the body and
// passes every argument, cpu.rs:338-357.)
UOp with_all_params(const UOp& kernel, const UOp& scheduled);
// Symbolic cleanup (when enabled) plus the GPU range retagging (size-1 reduce
// ranges become the constant 0; output ranges become GLOBAL).
UOp gpu_optimize(const UOp& rangeified);

// Render a gfx950 HIP kernel (source + launch geometry) for an optimized
// kernel. `force` selects a class for tests (Serial is always valid).
RenderedKernel render_hip(const UOp& kernel, const std::string& name, int force_class = -1);
// render_hip with the symbol named by a hash of the source ("k<hash>_<class>").
RenderedKernel render_hip_stable(const UOp& kernel);
KernelClass classify_kernel(const UOp& kernel);
// The class a kernel has before a small one is promoted to KernelClass::Block.
KernelClass base_class(const UOp& kernel);

// One launch for a run of block kernels (KernelClass::Block) that a replayed
// sequence launches back to back: their bodies, in order, separated by
// workgroup barriers, taking every stage's arguments concatenated in stage
// order. Each stage computes exactly what its own kernel computes. With
// `read_back` (one stage or more), three more arguments follow (rb_dst,
// rb_src, rb_words) and a last stage, after a barrier, copies rb_words 32-bit
// words from rb_src to rb_dst: the sequence's result read back by the launch
// that computed it.
//
// With `fwd`, stage outputs that later stages of the batch read stay in LDS:
// the producing stage writes an LDS array instead of its buffer, the later
// stages read that array, and once every stage has run the arrays are copied
// to their buffers. A stage-to-stage hand-off then waits for LDS, not for
// global stores to reach L2 and loads to come back.
struct BatchForwarding {
  std::vector<int> arg_buffer;  // per argument of the batch: the LDS array it reads or writes, or -1
  std::vector<DType> dtypes;    // per LDS array
  std::vector<size_t> numels;
  std::vector<int> out_arg;     // the producing stage's output argument (the copy's destination)
  // Per stage: whether a workgroup barrier precedes it. A stage needs one
  // when it reads a buffer a stage since the last barrier writes, writes one
  // such a stage reads or writes, or shares a body (and so its LDS) with one;
  // empty means a barrier before every stage but the first.
  std::vector<uint8_t> barrier;
};
// The LDS a batch may spend on forwarded outputs (the stage bodies keep their
// own few kilobytes).
constexpr size_t kBatchForwardBytes = 64 * 1024;
// One argument of a stage, for choosing what to forward: the buffer's
// identity (null for a scalar) and its element count.
struct BatchArg {
  const void* id = nullptr;
  size_t numel = 0;
};
// Which stage outputs stay in LDS. An output is kept when one stage alone
// writes its buffer, writes every element of it and does not read it, its
// dtype is f32, i32 or bool, and it fits in what is left of
// kBatchForwardBytes; stages after the writer read the LDS array, stages
// before it the buffer (its contents before the batch, as in the sequence).
BatchForwarding batch_forwarding(const std::vector<const RenderedKernel*>& stages,
                                 const std::vector<std::vector<BatchArg>>& args);
RenderedKernel render_block_batch(const std::vector<const RenderedKernel*>& stages, bool read_back = false,
                                  const BatchForwarding* fwd = nullptr);

// One launch that runs two independent kernels side by side: workgroups
// [0, a.grid) run a's body, the rest b's (the small GEMM's block-index
// bodies, hbody_fn). Both must have the same 1-D workgroup size; the launch
// takes a's arguments, then b's.
RenderedKernel render_hfused(const RenderedKernel& a, const RenderedKernel& b);
// One launch that runs one or two kernels with block-index bodies (hbody_fn:
// the one-pass small GEMMs, alone or as a pair) beside a batch of block
// kernels they share no written buffer with: workgroup 0 runs the batch (its
// stages, LDS hand-off and read-back exactly as render_block_batch renders
// them), the next hb[0].grid workgroups hb[0]'s body, then hb[1]'s. The
// launch has the block kernels' workgroup size (1024); in the other
// workgroups the waves past a body's own workgroup size end at once. The
// launch takes each hb kernel's arguments, then the batch's.
RenderedKernel render_hbatch(const std::vector<const RenderedKernel*>& hb,
                             const std::vector<const RenderedKernel*>& stages, bool read_back = false,
                             const BatchForwarding* fwd = nullptr);
// Whether the kernels at positions `a` and those at positions `b` are
// independent: no buffer one side writes is read or written by the other
// (buffers by identity; a kernel's output counts as read too, for in-place
// updates).
bool kernels_independent(const std::vector<const RenderedKernel*>& kernels,
                         const std::vector<std::vector<BatchArg>>& args, const std::vector<size_t>& a,
                         const std::vector<size_t>& b);
// Whether kernel i can run beside a batch in one launch (render_hbatch): a
// one-launch kernel with a block-index body, no scratch, and a 1-D workgroup
// of whole waves no larger than a block kernel's.
bool hbatch_member(const RenderedKernel& k);
// A launch of render_hbatch in a sequence: the kernels with block-index
// bodies (one, or the two of a pair, in sequence order) and the batch (an
// index into the sequence's batch runs) they run beside.
struct HBatchRun {
  std::vector<size_t> hb;
  size_t group = 0;
};
// The hbatch launches of a sequence whose batches are `groups` (first,
// count) and whose pairs start at `pair_firsts`: each batch joins the launch
// unit right before it, or else the one right after it, when that unit is a
// pair or a single kernel of hbatch_member kernels, not already joined,
// independent of every stage of the batch, and the launch's arguments (plus
// `extra` for a read-back) fit in FG_MAX_LAUNCH_ARGS. In sequence order.
std::vector<HBatchRun> hbatch_runs(const std::vector<const RenderedKernel*>& kernels,
                                   const std::vector<std::vector<BatchArg>>& args,
                                   const std::vector<std::pair<size_t, size_t>>& groups,
                                   const std::vector<size_t>& pair_firsts, size_t extra = 3);
// Adjacent kernels of a sequence that can share one launch: both one-launch
// kernels with a block-index body (hbody_fn) and no scratch, the same
// workgroup size, neither marked in `excluded` (kernels in a batch), at most
// FG_MAX_LAUNCH_ARGS arguments together, and independent: neither writes a
// buffer the other reads or writes (buffers by identity, as in
// batch_forwarding). Taken greedily in sequence order; returns the first
// kernel of each pair.
std::vector<size_t> pair_runs(const std::vector<const RenderedKernel*>& kernels,
                              const std::vector<std::vector<BatchArg>>& args, const std::vector<bool>& excluded);

// The runs of consecutive block kernels a sequence launches as batches, as
// (first, count) pairs: every run of two or more, split after kMaxBatchStages
// kernels and before the kernel that would take the run's arguments past
// FG_MAX_LAUNCH_ARGS (a batch launch passes every stage's arguments).
// `is_block[i]` tells whether launch i is a block kernel; `nargs[i]` is its
// argument count.
constexpr size_t kMaxBatchStages = 16;
std::vector<std::pair<size_t, size_t>> block_batch_runs(const std::vector<bool>& is_block,
                                                        const std::vector<size_t>& nargs);

}  // namespace fg
