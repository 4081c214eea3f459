/* ferrograd_hip.h — C-ABI of the MI355X device backend.
 *
 * These entry points replace the reference's CPU backend primitives behind its
 * `Device` trait (src/device.rs:275-332) and its clang JIT
 * (src/device/cpu.rs:151-394). A Rust `HipDevice` implementing that trait binds
 * them one-to-one:
 *
 *   Device::allocate        (device.rs:283, cpu.rs:277-280)  -> fg_hip_alloc(zero=1)
 *   Buffer::ensure_allocated(device.rs:191-213)              -> fg_hip_alloc
 *   Storage drop            (device.rs:66-70)                -> fg_hip_free
 *   Device::copy_from_host  (device.rs:294, cpu.rs:282-302)  -> fg_hip_copy_h2d
 *   Device::copy_to_host    (device.rs:302, cpu.rs:304-316)  -> fg_hip_copy_d2h
 *   Device::compile         (device.rs:309-314, cpu.rs:151-208, 318-326) -> fg_hip_compile
 *   Device::execute         (device.rs:321, cpu.rs:328-380)  -> fg_hip_launch
 *   Program drop            (cpu.rs:95-106)                  -> fg_hip_program_free
 *
 * Every function returns 0 on success and a nonzero status otherwise; the
 * message is available from fg_hip_last_error(). No exception crosses the ABI.
 * Calls on one context are not thread-safe (the reference backend is !Send).
 * All work is queued on the context's single stream in call order;
 * fg_hip_copy_d2h returns after the data is on the host.
 */
#ifndef FERROGRAD_HIP_H
#define FERROGRAD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fg_ctx fg_ctx;
typedef struct fg_prog fg_prog;

/* Kernel argument kinds, matching KernelArg (src/device.rs:242-251). */
enum { FG_ARG_PTR = 0, FG_ARG_I32 = 1, FG_ARG_F32 = 2, FG_ARG_BOOL = 3 };

typedef struct fg_arg {
  int32_t kind; /* FG_ARG_* */
  int32_t reserved;
  union {
    void* p;
    int32_t i;
    float f;
    uint8_t b;
  } v;
} fg_arg;

/* Status codes. */
enum {
  FG_OK = 0,
  FG_ERR_HIP = 1,        /* a HIP runtime call failed */
  FG_ERR_COMPILE = 2,    /* hiprtc rejected the source (log in last_error) */
  FG_ERR_SYMBOL = 3,     /* the named kernel is not in the compiled module */
  FG_ERR_ARGS = 4,       /* argument count or kind does not match */
  FG_ERR_INVALID = 5     /* null handle, bad size, bad launch geometry */
};

/* Select device `ordinal`, create the context's stream. */
int fg_hip_init(int device_ordinal, fg_ctx** out);
int fg_hip_destroy(fg_ctx* ctx);

/* Device memory. `zero` != 0 asks for zero-filled memory (the allocate
 * contract, device.rs:282). Freed blocks are kept for reuse by later
 * allocations of the same size; reuse is ordered on the context's stream. */
int fg_hip_alloc(fg_ctx* ctx, size_t nbytes, int zero, void** dptr);
int fg_hip_free(fg_ctx* ctx, void* dptr);
/* fg_hip_alloc that returns the cached free block `hint` when it is free and
 * of this size, else any block. No counterpart in the reference: a replayed
 * launch sequence asks for the blocks it used last time, so the addresses its
 * recorded HIP graph holds stay valid and need no update. */
int fg_hip_alloc_hint(fg_ctx* ctx, size_t nbytes, int zero, void* hint, void** dptr);
/* Return cached free blocks to the driver. */
int fg_hip_trim(fg_ctx* ctx);

/* Host<->device copies. h2d returns once `src` may be reused; d2h returns once
 * `dst` holds the data (all earlier work on the stream has completed). */
int fg_hip_copy_h2d(fg_ctx* ctx, void* dst, const void* src, size_t nbytes);
int fg_hip_copy_d2h(fg_ctx* ctx, void* dst, const void* src, size_t nbytes);
int fg_hip_copy_d2d(fg_ctx* ctx, void* dst, const void* src, size_t nbytes);

/* Asynchronous read-back of a small result. No counterpart in the reference,
 * whose copy_to_host returns with the data (device.rs:302): a training loop
 * that reads one loss per step can queue the next step before it waits for
 * this one's. fg_hip_read_async queues a copy of `nbytes` (at most
 * FG_READ_SLOT_BYTES) from device memory into pinned slot `slot` (0 ..
 * FG_READ_SLOTS-1) behind the work already on the stream, and returns.
 * fg_hip_read_wait waits for that copy only, not for work queued after it,
 * and copies the bytes to `dst`; `nbytes` must match. Reusing a slot first
 * waits for its previous copy. */
#define FG_READ_SLOTS 8
#define FG_READ_SLOT_BYTES ((size_t)65536)
int fg_hip_read_async(fg_ctx* ctx, int slot, const void* src, size_t nbytes);
int fg_hip_read_wait(fg_ctx* ctx, int slot, void* dst, size_t nbytes);
/* The same read-back done by a kernel of the caller's own launches (the last
 * node of a replayed sequence's graph), so no separate copy is queued.
 * fg_hip_read_slot waits until `slot` is free (its previous read landed) and
 * gives the device address of its pinned landing area, which a kernel may
 * store up to FG_READ_SLOT_BYTES into. After queuing that kernel,
 * fg_hip_read_queued marks the slot as holding `nbytes` that land behind the
 * work on the stream; fg_hip_read_wait then waits for them as above. */
int fg_hip_read_slot(fg_ctx* ctx, int slot, void** device_ptr);
int fg_hip_read_queued(fg_ctx* ctx, int slot, size_t nbytes);

/* Compile HIP source for gfx950 with hiprtc and load kernel `func`. The code
 * object is cached on disk keyed by a hash of source, options and target, and
 * a context keeps the modules it loaded (the 1024 most recent): the same
 * source compiled again on it reuses its loaded module. */
int fg_hip_compile(fg_ctx* ctx, const char* source, const char* func, int num_args, fg_prog** out);
int fg_hip_program_free(fg_prog* prog);
int fg_hip_program_num_args(const fg_prog* prog);
/* Another kernel `func` of the module `prog` was loaded from (multi-kernel
 * programs, e.g. a partial-sums pass and its finishing pass). The module
 * stays loaded until every program sharing it is freed. */
int fg_hip_program_function(fg_prog* prog, const char* func, int num_args, fg_prog** out);

/* Most arguments one launch takes (fg_hip_launch and graph nodes refuse more). */
#define FG_MAX_LAUNCH_ARGS 64

/* Launch on the context's stream. `nargs` must equal the program's num_args,
 * at most FG_MAX_LAUNCH_ARGS. */
int fg_hip_launch(fg_ctx* ctx, fg_prog* prog, const fg_arg* args, int nargs, const unsigned grid[3],
                  const unsigned block[3], unsigned lds_bytes);

/* Wait for all queued work. */
int fg_hip_sync(fg_ctx* ctx);

/* Launch sequences replayed as one HIP graph. No counterpart in the reference:
 * its CPU backend calls each kernel on the host thread (cpu.rs:373-377). A
 * realisation plan that is replayed every training step launches the same
 * programs with the same geometry each time; only buffer addresses and scalars
 * change. fg_hip_graph_create records `n` launches once (progs[i] with
 * grids[3i..3i+2], blocks[3i..3i+2], lds[i] and nargs[i] arguments taken in
 * order from `args`) by stream capture of the context's stream; nothing runs.
 * fg_hip_graph_launch takes the arguments of every launch, concatenated in
 * launch order, updates the launches whose arguments differ from the previous
 * replay (their number goes to *updated when it is not NULL), and launches the
 * graph on the context's stream. While launch
 * profiling is enabled the launches run one by one instead, so each is timed.
 * The graph holds no memset or copy nodes. */
typedef struct fg_graph fg_graph;
int fg_hip_graph_create(fg_ctx* ctx, int n, fg_prog* const* progs, const unsigned* grids, const unsigned* blocks,
                        const unsigned* lds, const int* nargs, const fg_arg* args, fg_graph** out);
int fg_hip_graph_launch(fg_ctx* ctx, fg_graph* graph, const fg_arg* args, int* updated);
int fg_hip_graph_free(fg_graph* graph);

/* The Renderer half of the boundary. The reference renders a kernel with
 * `Renderer::render(uops, name) -> String` (src/codegen.rs:17-20), called with
 * a hard-coded ClangRenderer in execute_item (src/tensor.rs:845-852), and
 * compiles the string with no launch geometry (device.rs:309-314). For this
 * device a caller hands over the kernel as rangeify leaves it
 * (rangeify.rs:42-206, parameterised by schedule.rs:131-170), in the text
 * form below, and gets back everything a launch needs: the gfx950 HIP source,
 * the launch passes in order (function, grid, block, LDS bytes), the kinds of
 * the kernel parameters in slot order (FG_ARG_*), and the bytes of scratch
 * the passes share (split-K and split column-reduction partials; written
 * before read, so never zeroed). The gfx950 passes of `optimize`
 * (optimize/mod.rs:116-141 on the CPU) run inside: launch mapping, DPP/LDS
 * reductions, MFMA GEMM recognition.
 *
 * Kernel text: a header line "fg-kernel 1", then one node per line in
 * topological order, line i defining node i:
 *   <Op> <dtype> <arg> [#<tag>] [<source node numbers>...]
 * Op is the uop.rs:26-339 variant name; dtype f32|i32|bool|void (xN for
 * vectors); arg "-", device:hip, int:<n>, bool:<0|1>, float:<16 hex digits of
 * the f64 bits>, range:<axis>:<LOOP|GLOBAL|REDUCE|...>, param:<slot>:<numel>,
 * scalar:<slot>, index:<n>, reduce:<Op>:<axes,...>, axes:/shape:/bounds:/
 * lanes:<list>, var:<name>:<min>:<max>. The last node is the kernel's Sink.
 * Malformed text fails with FG_ERR_INVALID and a message naming the line. */
typedef struct fg_rendered fg_rendered;
int fg_hip_render(const char* kernel_text, fg_rendered** out);
/* Any output pointer may be NULL. Strings live as long as the fg_rendered. */
int fg_hip_rendered_info(const fg_rendered* r, const char** source, const char** kind, int* num_params,
                         int* num_launches, size_t* scratch_bytes);
int fg_hip_rendered_param(const fg_rendered* r, int slot, int* kind);
int fg_hip_rendered_launch(const fg_rendered* r, int i, const char** func, unsigned grid[3], unsigned block[3],
                           unsigned* lds_bytes);
int fg_hip_rendered_free(fg_rendered* r);

/* A rendered kernel compiled (fg_hip_compile's cache applies) and loaded:
 * Device::compile (device.rs:309-314) with the geometry attached.
 * fg_hip_kernel_run is Device::execute (device.rs:321, cpu.rs:328-380) for it:
 * the arguments in slot order, as the kernel's parameter kinds require (a
 * wrong count or kind fails with FG_ERR_ARGS before anything is queued); every
 * pass is queued on the context's stream. A kernel with scratch gets it from
 * the library: allocated with fg_hip_alloc by the first run, kept with the
 * kernel, reused by later runs on the same context, freed with the kernel. */
typedef struct fg_kernel fg_kernel;
int fg_hip_kernel_load(fg_ctx* ctx, const fg_rendered* r, fg_kernel** out);
int fg_hip_kernel_run(fg_ctx* ctx, fg_kernel* k, const fg_arg* args, int nargs);
int fg_hip_kernel_free(fg_kernel* k);

/* fg_hip_kernel_run that allocates nothing. No counterpart in the reference
 * (its CPU backend allocates on the host as it likes): it is for callers that
 * cannot allocate device memory, such as code under HIP graph capture and
 * tight serving loops. Its scratch is a static device array of
 * FG_NOALLOC_SCRATCH_BYTES that the library holds on every GPU fg_hip_init
 * was called for, until the process ends; a kernel needing more is rejected
 * with FG_ERR_INVALID before anything is queued. It calls no hipMalloc or
 * hipFree and records no profiling events. The scratch of one GPU is shared
 * by every call on it and keeps the last call's contents (the kernels write
 * every partial before reading it, so nothing needs clearing); calls that
 * overlap on one GPU, from contexts whose streams run concurrently, race on
 * it. Calls on one context are ordered by its stream and do not. */
#define FG_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int fg_hip_kernel_run_noalloc(fg_ctx* ctx, fg_kernel* k, const fg_arg* args, int nargs);

/* The file fg_hip_compile caches the code object of `source` in: named by a
 * hash of the source, every hiprtc option (the gfx950 target among them) and
 * the hiprtc version. A cached file the runtime rejects is compiled again.
 * No reference counterpart (the reference compiles into a temporary
 * directory, cpu.rs:151-208). */
const char* fg_hip_code_object_path(const char* source);

/* Timing events on the context's stream (slots 0..63). */
int fg_hip_event_record(fg_ctx* ctx, int slot);
int fg_hip_event_elapsed_ms(fg_ctx* ctx, int start_slot, int end_slot, float* ms);

/* Launch profiling: while enabled, every fg_hip_launch on the context is
 * bracketed by two events on its stream. fg_hip_profile_read waits for the
 * stream and returns, as JSON, [{"kernel": name, "ms": duration}, ...] for the
 * launches since the last read (two calls: buf == NULL reports the size). */
int fg_hip_profile_enable(fg_ctx* ctx, int on);
int fg_hip_profile_read(fg_ctx* ctx, char* buf, size_t len, size_t* needed);

/* Device properties: CU count, clock (kHz), LDS per block, arch name. */
int fg_hip_device_info(fg_ctx* ctx, int* cu_count, int* clock_khz, size_t* lds_per_block, char* arch,
                       size_t arch_len);

/* Message of the last failed call on this thread ("" if none). */
const char* fg_hip_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* FERROGRAD_HIP_H */
