/* ferrograd.h — C-ABI of the tensor front end that drives the MI355X path.
 *
 * Mirrors the reference's public Rust API (src/tensor.rs, src/nn.rs,
 * src/optim.rs) so a host program (the Python package ferrograd_amd, a Rust
 * shim, the benchmark) can build lazy graphs, realise them on a device and
 * read results. Devices: 0 = cpu (only when the test oracle is loaded),
 * 1 = hip (MI355X). Dtypes: 0 = f32, 1 = i32, 2 = bool.
 *
 * Every function returns 0 on success, nonzero on error; the message is in
 * fg_last_error(). Handles are owned by the caller and released with the
 * matching *_free. A tensor handle aliases shared tensor state, like a cloned
 * reference Tensor (tensor.rs:30-38).
 */
#ifndef FERROGRAD_H
#define FERROGRAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fg_tensor fg_tensor;
typedef struct fg_linear fg_linear;
typedef struct fg_sgd fg_sgd;

enum { FG_DEV_CPU = 0, FG_DEV_HIP = 1 };
enum { FG_F32 = 0, FG_I32 = 1, FG_BOOL = 2 };
enum {
  FG_UNARY_NEG = 0, FG_UNARY_RECIPROCAL, FG_UNARY_EXP2, FG_UNARY_LOG2, FG_UNARY_SQRT, FG_UNARY_RELU,
  FG_UNARY_EXP, FG_UNARY_LOG, FG_UNARY_CONTIGUOUS, FG_UNARY_DETACH, FG_UNARY_ALIAS
};
enum { FG_BINARY_ADD = 0, FG_BINARY_MUL, FG_BINARY_SUB, FG_BINARY_MATMUL, FG_BINARY_CROSS_ENTROPY };
enum { FG_REDUCE_SUM = 0, FG_REDUCE_MAX };
enum { FG_MOVE_RESHAPE = 0, FG_MOVE_PERMUTE, FG_MOVE_EXPAND };

const char* fg_last_error(void);

/* Construction: Tensor::new / zeros / ones (tensor.rs:260-312). */
int fg_tensor_from_data(int device, int dtype, const void* data, size_t nbytes, const int64_t* shape, int ndim,
                        fg_tensor** out);
int fg_tensor_zeros(int device, int dtype, const int64_t* shape, int ndim, fg_tensor** out);
int fg_tensor_ones(int device, int dtype, const int64_t* shape, int ndim, fg_tensor** out);
int fg_tensor_free(fg_tensor* t);

/* Offline MNIST IDX files (dataset.rs:116-161; no download). Images: magic
 * 2051, big-endian u32 count/rows/cols (28x28 required), u8 pixels -> f32
 * [count, 784] scaled by 1/255 on `device`. Labels: magic 2049, u32 count, u8
 * labels; call with out == NULL to get the count, then with a buffer of at
 * least that many bytes. Errors carry the reference's messages ("bad IDX
 * format: expected IDX image magic 2051, got N", "io: ..."). */
int fg_idx_images(const char* path, int device, fg_tensor** out);
int fg_idx_labels(const char* path, uint8_t* out, size_t capacity, size_t* count);

/* Lazy ops (tensor.rs:442-778). */
int fg_tensor_unary(fg_tensor* t, int op, fg_tensor** out);
int fg_tensor_binary(fg_tensor* a, fg_tensor* b, int op, fg_tensor** out);
int fg_tensor_reduce(fg_tensor* t, int op, const int64_t* axes, int naxes, fg_tensor** out);
int fg_tensor_movement(fg_tensor* t, int op, const int64_t* arg, int narg, fg_tensor** out);
int fg_tensor_narrow(fg_tensor* t, int64_t dim, int64_t start, int64_t len, fg_tensor** out);
int fg_tensor_log_softmax(fg_tensor* t, int64_t axis, fg_tensor** out);

/* In-place graph updates (tensor.rs:399-440). */
int fg_tensor_assign(fg_tensor* t, fg_tensor* value);
int fg_tensor_replace(fg_tensor* t, fg_tensor* value);

/* Realisation and readback (tensor.rs:781-930). `nbytes` must equal the
 * tensor's byte size. */
int fg_tensor_realize_many(fg_tensor** ts, int n);
int fg_tensor_read(fg_tensor* t, void* dst, size_t nbytes);
/* Device::copy_from_host (device.rs:294, cpu.rs:282-302) into the realised
 * tensor's buffer (realised first): `nbytes` must equal the buffer's size, or
 * the call fails with the reference's "copy_from_host: expected N bytes, got
 * M". Every alias of the tensor sees the new contents. */
int fg_tensor_write(fg_tensor* t, const void* src, size_t nbytes);

/* Metadata. `ndim` is in/out: capacity of `shape` in, rank out. */
int fg_tensor_shape(fg_tensor* t, int64_t* shape, int* ndim);
int fg_tensor_info(fg_tensor* t, int* dtype, int* device, int* realized, int* requires_grad);
int fg_tensor_set_requires_grad(fg_tensor* t, int requires_grad);
/* Storage of a realised tensor: the device pointer (HIP) or host pointer
 * (cpu) and its byte size, for zero-copy interop. The pointer stays valid while
 * the tensor's buffer is alive and may change when the tensor is realised
 * again; lazily zero-filled storage is materialised first. No reference
 * counterpart (the reference keeps Storage opaque, device.rs:60-70). */
int fg_tensor_data_ptr(fg_tensor* t, void** ptr, size_t* nbytes);
int fg_tensor_same(fg_tensor* a, fg_tensor* b, int* same);

/* Autograd (tensor.rs:938-998). fg_tensor_grad sets *out to NULL if none. */
int fg_tensor_grad(fg_tensor* t, fg_tensor** out);
int fg_tensor_backward(fg_tensor* loss);
int fg_tensor_gradient(fg_tensor* loss, fg_tensor** targets, int n, fg_tensor** outs);

/* nn::Linear (nn.rs:67-104) with the reference's seeded Kaiming init. */
int fg_reset_init_seed(uint64_t seed);
int fg_linear_new(int device, int64_t in_features, int64_t out_features, int bias, fg_linear** out);
int fg_linear_forward(fg_linear* l, fg_tensor* x, fg_tensor** out);
int fg_linear_num_params(fg_linear* l, int* n);
int fg_linear_param(fg_linear* l, int i, fg_tensor** out);
int fg_linear_free(fg_linear* l);

/* The training loop body of examples/mnist.rs:84-101, `steps` times, from native
 * code: logits = layers[0..n) with ReLU between them (mnist.rs:30-54 for any
 * depth), loss = cross_entropy(logits, targets), opt's zero_grad, backward,
 * step, then the loss read back into losses[i]. Replaces the Rust caller's
 * loop; it calls the same Tensor/Linear/Sgd code as the entry points above,
 * and runs the same kernels in the same order. Each step's loss is read once
 * the next step is queued, and once two consecutive steps have replayed the
 * same recorded plans over the same buffers, further steps (all but the last)
 * launch that kernel sequence as one device sequence without rebuilding the
 * lazy graphs. Losses, parameters and gradients come out as from the loop
 * driven call by call. */
int fg_mlp_train_steps(fg_linear* const* layers, int nlayers, fg_sgd* opt, fg_tensor* x, fg_tensor* targets, int steps,
                       float* losses);
/* The same loop over a resident dataset, batched as examples/mnist.rs:84-87:
 * step i trains on rows [s, s + batch_size) of `images` and `targets`
 * (narrow(0, s, batch_size)), s = ((first_batch + i) mod (rows / batch_size))
 * * batch_size, so consecutive calls continue through the epochs. Captured
 * steps take each batch's start as a kernel argument of the replay. */
int fg_mlp_train_batches(fg_linear* const* layers, int nlayers, fg_sgd* opt, fg_tensor* images, fg_tensor* targets,
                         int64_t batch_size, int64_t first_batch, int steps, float* losses);

/* optim::Sgd (optim.rs:16-71). */
int fg_sgd_new(fg_tensor** params, int n, float lr, fg_sgd** out);
int fg_sgd_zero_grad(fg_sgd* s);
int fg_sgd_step(fg_sgd* s);
int fg_sgd_free(fg_sgd* s);

/* Device control and statistics. fg_device_context returns the HIP device's
 * fg_ctx (include/ferrograd_hip.h) — the stream every realised kernel runs
 * on — for event timing and launch profiling. */
int fg_synchronize(int device);
/* The device a program uses when it names none: the reference's
 * tensor::cpu() (tensor.rs:1122-1127), chosen here by the DEVICE environment
 * variable, "hip" (default) or "cpu" (only with the test oracle loaded). */
int fg_default_device(int* device);
/* The HIP path's optional passes as OPT selects them, read once per process
 * with the reference's grammar (src/optimize/mod.rs:85-112): symbolic
 * folding, MFMA GEMM tiles, narrow VALU products, schedule-time fusion (also
 * off with FG_FUSE=0), small kernels as one workgroup, and consecutive such
 * kernels of a replayed sequence batched into one launch. 1 = enabled. */
int fg_gpu_passes(int* symbolic, int* mfma, int* narrow, int* fuse, int* block, int* batch);
int fg_device_context(int device, void** ctx);
int fg_stats(uint64_t* kernels_launched, uint64_t* programs_compiled, uint64_t* lowering_hits);
/* Replayed realisation plans that ran as one HIP graph launch, and the
 * launches in them whose arguments had to be updated (no counterpart in the
 * reference, which has no graphs). */
int fg_graph_stats(uint64_t* replays, uint64_t* updated_launches);
/* fg_mlp_train_steps' step capture: how many times a step was captured, and
 * how many steps were then launched from a capture without rebuilding their
 * lazy graphs (FG_STEP_CAPTURE=0 turns capture off). No reference
 * counterpart. */
int fg_step_capture_stats(uint64_t* captured, uint64_t* replayed);
/* Cumulative host nanoseconds in: schedule, lowering-cache/compile, launch,
 * live-tensor rewrite after realisation, backward graph construction. */
int fg_host_times(uint64_t out[5]);
int fg_clear_caches(void);
/* Realisation plans: realize_many records each distinct lazy-graph structure
 * (with its buffer sharing and which leaves still hold zeros) together with
 * its kernel launches, and replays that record when the structure recurs, as
 * in a training loop. Replays produce the same kernels, arguments and results;
 * disabling the cache (on = 0) also drops it. No reference counterpart (the
 * reference reschedules every realize, tensor.rs:781-821). */
int fg_plan_cache_enable(int on);
int fg_plan_cache_stats(uint64_t* hits, uint64_t* misses, uint64_t* entries);

/* HIP-graph replay threshold: with n >= 2 a replayed plan of at least n
 * kernel launches is recorded once as a HIP graph and relaunched as one, and
 * shorter plans are launched one by one; n = 0 launches every plan one by one
 * (the default, unless FG_HIP_GRAPHS=1 sets 2). Other values fail. *previous
 * (may be NULL) receives the old value. No reference counterpart. */
int fg_set_graph_min_launches(int n, int* previous);

/* Inspection for tests and tooling: schedule the roots (without running
 * anything) and describe the plan as JSON; optionally render each kernel with
 * the HIP code generator (no device needed), adding each kernel's rangeified
 * form as fg_hip_render's kernel text ("kernel"). Two calls: with buf == NULL it
 * plans and reports the JSON size in *needed; with a buffer it copies the
 * JSON of the last plan on this thread. */
int fg_debug_plan(fg_tensor** roots, int n, int fuse, int render_hip, char* buf, size_t len, size_t* needed);

#ifdef __cplusplus
}
#endif

#endif /* FERROGRAD_H */
