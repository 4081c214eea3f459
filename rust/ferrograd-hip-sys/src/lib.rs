//! FFI bindings of `libferrograd_amd.so`, the MI355X (gfx950) realize path.
//!
//! NOT BUILT IN THIS REPOSITORY: the build image has no Rust toolchain. The
//! declarations below follow `include/ferrograd_hip.h` (the device and
//! renderer boundary, binding B) and `include/ferrograd.h` (the tensor front
//! end, binding A) line for line; `reference/src/device/hip.rs` is the module
//! the ferrograd crate adds on top of them.
//!
//! Every function returns 0 on success. On failure the message is in
//! `fg_hip_last_error()` (device calls) or `fg_last_error()` (front end), per
//! thread; [`hip_result`] and [`fg_result`] turn a status into a `Result`.

#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_void, CStr, CString};

// ── include/ferrograd_hip.h ─────────────────────────────────────────────────

/// A device context: one GPU and the stream every launch runs on.
#[repr(C)]
pub struct fg_ctx {
    _p: [u8; 0],
}
/// A compiled and loaded kernel function.
#[repr(C)]
pub struct fg_prog {
    _p: [u8; 0],
}
/// A recorded launch sequence (HIP graph).
#[repr(C)]
pub struct fg_graph {
    _p: [u8; 0],
}
/// A kernel rendered for gfx950: source, launch passes, parameter kinds.
#[repr(C)]
pub struct fg_rendered {
    _p: [u8; 0],
}
/// A rendered kernel compiled and loaded, ready to run.
#[repr(C)]
pub struct fg_kernel {
    _p: [u8; 0],
}

/// Argument kinds, matching `KernelArg` (src/device.rs:242-251).
pub const FG_ARG_PTR: i32 = 0;
pub const FG_ARG_I32: i32 = 1;
pub const FG_ARG_F32: i32 = 2;
pub const FG_ARG_BOOL: i32 = 3;

/// Status codes.
pub const FG_OK: i32 = 0;
pub const FG_ERR_HIP: i32 = 1;
pub const FG_ERR_COMPILE: i32 = 2;
pub const FG_ERR_SYMBOL: i32 = 3;
pub const FG_ERR_ARGS: i32 = 4;
pub const FG_ERR_INVALID: i32 = 5;

pub const FG_READ_SLOTS: i32 = 8;
pub const FG_READ_SLOT_BYTES: usize = 65536;
pub const FG_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

#[repr(C)]
#[derive(Clone, Copy)]
pub union fg_arg_v {
    pub p: *mut c_void,
    pub i: i32,
    pub f: f32,
    pub b: u8,
}

/// One kernel argument (`struct fg_arg`).
#[repr(C)]
#[derive(Clone, Copy)]
pub struct fg_arg {
    pub kind: i32,
    pub reserved: i32,
    pub v: fg_arg_v,
}

impl fg_arg {
    #[must_use]
    pub fn ptr(p: *mut c_void) -> Self {
        Self { kind: FG_ARG_PTR, reserved: 0, v: fg_arg_v { p } }
    }
    #[must_use]
    pub fn i32(i: i32) -> Self {
        Self { kind: FG_ARG_I32, reserved: 0, v: fg_arg_v { i } }
    }
    #[must_use]
    pub fn f32(f: f32) -> Self {
        Self { kind: FG_ARG_F32, reserved: 0, v: fg_arg_v { f } }
    }
    #[must_use]
    pub fn boolean(b: bool) -> Self {
        Self { kind: FG_ARG_BOOL, reserved: 0, v: fg_arg_v { b: u8::from(b) } }
    }
}

extern "C" {
    pub fn fg_hip_init(device_ordinal: i32, out: *mut *mut fg_ctx) -> i32;
    pub fn fg_hip_destroy(ctx: *mut fg_ctx) -> i32;
    pub fn fg_hip_alloc(ctx: *mut fg_ctx, nbytes: usize, zero: i32, dptr: *mut *mut c_void) -> i32;
    pub fn fg_hip_free(ctx: *mut fg_ctx, dptr: *mut c_void) -> i32;
    pub fn fg_hip_alloc_hint(ctx: *mut fg_ctx, nbytes: usize, zero: i32, hint: *mut c_void,
                             dptr: *mut *mut c_void) -> i32;
    pub fn fg_hip_trim(ctx: *mut fg_ctx) -> i32;
    pub fn fg_hip_copy_h2d(ctx: *mut fg_ctx, dst: *mut c_void, src: *const c_void, nbytes: usize) -> i32;
    pub fn fg_hip_copy_d2h(ctx: *mut fg_ctx, dst: *mut c_void, src: *const c_void, nbytes: usize) -> i32;
    pub fn fg_hip_copy_d2d(ctx: *mut fg_ctx, dst: *mut c_void, src: *const c_void, nbytes: usize) -> i32;
    pub fn fg_hip_read_async(ctx: *mut fg_ctx, slot: i32, src: *const c_void, nbytes: usize) -> i32;
    pub fn fg_hip_read_wait(ctx: *mut fg_ctx, slot: i32, dst: *mut c_void, nbytes: usize) -> i32;
    pub fn fg_hip_read_slot(ctx: *mut fg_ctx, slot: i32, device_ptr: *mut *mut c_void) -> i32;
    pub fn fg_hip_read_queued(ctx: *mut fg_ctx, slot: i32, nbytes: usize) -> i32;
    pub fn fg_hip_compile(ctx: *mut fg_ctx, source: *const c_char, func: *const c_char, num_args: i32,
                          out: *mut *mut fg_prog) -> i32;
    pub fn fg_hip_program_free(prog: *mut fg_prog) -> i32;
    pub fn fg_hip_program_num_args(prog: *const fg_prog) -> i32;
    pub fn fg_hip_program_function(prog: *mut fg_prog, func: *const c_char, num_args: i32,
                                   out: *mut *mut fg_prog) -> i32;
    pub fn fg_hip_launch(ctx: *mut fg_ctx, prog: *mut fg_prog, args: *const fg_arg, nargs: i32,
                         grid: *const u32, block: *const u32, lds_bytes: u32) -> i32;
    pub fn fg_hip_sync(ctx: *mut fg_ctx) -> i32;
    pub fn fg_hip_graph_create(ctx: *mut fg_ctx, n: i32, progs: *const *mut fg_prog, grids: *const u32,
                               blocks: *const u32, lds: *const u32, nargs: *const i32, args: *const fg_arg,
                               out: *mut *mut fg_graph) -> i32;
    pub fn fg_hip_graph_launch(ctx: *mut fg_ctx, graph: *mut fg_graph, args: *const fg_arg,
                               updated: *mut i32) -> i32;
    pub fn fg_hip_graph_free(graph: *mut fg_graph) -> i32;
    pub fn fg_hip_render(kernel_text: *const c_char, out: *mut *mut fg_rendered) -> i32;
    pub fn fg_hip_rendered_info(r: *const fg_rendered, source: *mut *const c_char, kind: *mut *const c_char,
                                num_params: *mut i32, num_launches: *mut i32, scratch_bytes: *mut usize) -> i32;
    pub fn fg_hip_rendered_param(r: *const fg_rendered, slot: i32, kind: *mut i32) -> i32;
    pub fn fg_hip_rendered_launch(r: *const fg_rendered, i: i32, func: *mut *const c_char, grid: *mut u32,
                                  block: *mut u32, lds_bytes: *mut u32) -> i32;
    pub fn fg_hip_rendered_free(r: *mut fg_rendered) -> i32;
    pub fn fg_hip_kernel_load(ctx: *mut fg_ctx, r: *const fg_rendered, out: *mut *mut fg_kernel) -> i32;
    pub fn fg_hip_kernel_run(ctx: *mut fg_ctx, k: *mut fg_kernel, args: *const fg_arg, nargs: i32) -> i32;
    pub fn fg_hip_kernel_free(k: *mut fg_kernel) -> i32;
    pub fn fg_hip_kernel_run_noalloc(ctx: *mut fg_ctx, k: *mut fg_kernel, args: *const fg_arg, nargs: i32) -> i32;
    pub fn fg_hip_code_object_path(source: *const c_char) -> *const c_char;
    pub fn fg_hip_event_record(ctx: *mut fg_ctx, slot: i32) -> i32;
    pub fn fg_hip_event_elapsed_ms(ctx: *mut fg_ctx, start_slot: i32, end_slot: i32, ms: *mut f32) -> i32;
    pub fn fg_hip_profile_enable(ctx: *mut fg_ctx, on: i32) -> i32;
    pub fn fg_hip_profile_read(ctx: *mut fg_ctx, buf: *mut c_char, len: usize, needed: *mut usize) -> i32;
    pub fn fg_hip_device_info(ctx: *mut fg_ctx, cu_count: *mut i32, clock_khz: *mut i32,
                              lds_per_block: *mut usize, arch: *mut c_char, arch_len: usize) -> i32;
    pub fn fg_hip_last_error() -> *const c_char;
}

// ── include/ferrograd.h ─────────────────────────────────────────────────────

#[repr(C)]
pub struct fg_tensor {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_linear {
    _p: [u8; 0],
}
#[repr(C)]
pub struct fg_sgd {
    _p: [u8; 0],
}

pub const FG_DEV_CPU: i32 = 0;
pub const FG_DEV_HIP: i32 = 1;
pub const FG_F32: i32 = 0;
pub const FG_I32: i32 = 1;
pub const FG_BOOL: i32 = 2;
pub const FG_UNARY_NEG: i32 = 0;
pub const FG_UNARY_RECIPROCAL: i32 = 1;
pub const FG_UNARY_EXP2: i32 = 2;
pub const FG_UNARY_LOG2: i32 = 3;
pub const FG_UNARY_SQRT: i32 = 4;
pub const FG_UNARY_RELU: i32 = 5;
pub const FG_UNARY_EXP: i32 = 6;
pub const FG_UNARY_LOG: i32 = 7;
pub const FG_UNARY_CONTIGUOUS: i32 = 8;
pub const FG_UNARY_DETACH: i32 = 9;
pub const FG_UNARY_ALIAS: i32 = 10;
pub const FG_BINARY_ADD: i32 = 0;
pub const FG_BINARY_MUL: i32 = 1;
pub const FG_BINARY_SUB: i32 = 2;
pub const FG_BINARY_MATMUL: i32 = 3;
pub const FG_BINARY_CROSS_ENTROPY: i32 = 4;
pub const FG_REDUCE_SUM: i32 = 0;
pub const FG_REDUCE_MAX: i32 = 1;
pub const FG_MOVE_RESHAPE: i32 = 0;
pub const FG_MOVE_PERMUTE: i32 = 1;
pub const FG_MOVE_EXPAND: i32 = 2;

extern "C" {
    pub fn fg_last_error() -> *const c_char;
    pub fn fg_tensor_from_data(device: i32, dtype: i32, data: *const c_void, nbytes: usize, shape: *const i64,
                               ndim: i32, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_zeros(device: i32, dtype: i32, shape: *const i64, ndim: i32, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_ones(device: i32, dtype: i32, shape: *const i64, ndim: i32, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_free(t: *mut fg_tensor) -> i32;
    pub fn fg_idx_images(path: *const c_char, device: i32, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_idx_labels(path: *const c_char, out: *mut u8, capacity: usize, count: *mut usize) -> i32;
    pub fn fg_tensor_unary(t: *mut fg_tensor, op: i32, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_binary(a: *mut fg_tensor, b: *mut fg_tensor, op: i32, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_reduce(t: *mut fg_tensor, op: i32, axes: *const i64, naxes: i32,
                            out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_movement(t: *mut fg_tensor, op: i32, arg: *const i64, narg: i32,
                              out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_narrow(t: *mut fg_tensor, dim: i64, start: i64, len: i64, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_log_softmax(t: *mut fg_tensor, axis: i64, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_assign(t: *mut fg_tensor, value: *mut fg_tensor) -> i32;
    pub fn fg_tensor_replace(t: *mut fg_tensor, value: *mut fg_tensor) -> i32;
    pub fn fg_tensor_realize_many(ts: *mut *mut fg_tensor, n: i32) -> i32;
    pub fn fg_tensor_read(t: *mut fg_tensor, dst: *mut c_void, nbytes: usize) -> i32;
    pub fn fg_tensor_write(t: *mut fg_tensor, src: *const c_void, nbytes: usize) -> i32;
    pub fn fg_tensor_shape(t: *mut fg_tensor, shape: *mut i64, ndim: *mut i32) -> i32;
    pub fn fg_tensor_info(t: *mut fg_tensor, dtype: *mut i32, device: *mut i32, realized: *mut i32,
                          requires_grad: *mut i32) -> i32;
    pub fn fg_tensor_set_requires_grad(t: *mut fg_tensor, requires_grad: i32) -> i32;
    pub fn fg_tensor_data_ptr(t: *mut fg_tensor, ptr: *mut *mut c_void, nbytes: *mut usize) -> i32;
    pub fn fg_tensor_same(a: *mut fg_tensor, b: *mut fg_tensor, same: *mut i32) -> i32;
    pub fn fg_tensor_grad(t: *mut fg_tensor, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_tensor_backward(loss: *mut fg_tensor) -> i32;
    pub fn fg_tensor_gradient(loss: *mut fg_tensor, targets: *mut *mut fg_tensor, n: i32,
                              outs: *mut *mut fg_tensor) -> i32;
    pub fn fg_reset_init_seed(seed: u64) -> i32;
    pub fn fg_linear_new(device: i32, in_features: i64, out_features: i64, bias: i32,
                         out: *mut *mut fg_linear) -> i32;
    pub fn fg_linear_forward(l: *mut fg_linear, x: *mut fg_tensor, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_linear_num_params(l: *mut fg_linear, n: *mut i32) -> i32;
    pub fn fg_linear_param(l: *mut fg_linear, i: i32, out: *mut *mut fg_tensor) -> i32;
    pub fn fg_linear_free(l: *mut fg_linear) -> i32;
    pub fn fg_mlp_train_steps(layers: *const *mut fg_linear, nlayers: i32, opt: *mut fg_sgd, x: *mut fg_tensor,
                              targets: *mut fg_tensor, steps: i32, losses: *mut f32) -> i32;
    pub fn fg_mlp_train_batches(layers: *const *mut fg_linear, nlayers: i32, opt: *mut fg_sgd,
                                images: *mut fg_tensor, targets: *mut fg_tensor, batch_size: i64,
                                first_batch: i64, steps: i32, losses: *mut f32) -> i32;
    pub fn fg_sgd_new(params: *mut *mut fg_tensor, n: i32, lr: f32, out: *mut *mut fg_sgd) -> i32;
    pub fn fg_sgd_zero_grad(s: *mut fg_sgd) -> i32;
    pub fn fg_sgd_step(s: *mut fg_sgd) -> i32;
    pub fn fg_sgd_free(s: *mut fg_sgd) -> i32;
    pub fn fg_synchronize(device: i32) -> i32;
    pub fn fg_default_device(device: *mut i32) -> i32;
    pub fn fg_gpu_passes(symbolic: *mut i32, mfma: *mut i32, narrow: *mut i32, fuse: *mut i32, block: *mut i32,
                         batch: *mut i32) -> i32;
    pub fn fg_device_context(device: i32, ctx: *mut *mut c_void) -> i32;
    pub fn fg_stats(kernels_launched: *mut u64, programs_compiled: *mut u64, lowering_hits: *mut u64) -> i32;
    pub fn fg_graph_stats(replays: *mut u64, updated_launches: *mut u64) -> i32;
    pub fn fg_step_capture_stats(captured: *mut u64, replayed: *mut u64) -> i32;
    pub fn fg_host_times(out: *mut u64) -> i32;
    pub fn fg_clear_caches() -> i32;
    pub fn fg_plan_cache_enable(on: i32) -> i32;
    pub fn fg_plan_cache_stats(hits: *mut u64, misses: *mut u64, entries: *mut u64) -> i32;
    pub fn fg_set_graph_min_launches(n: i32, previous: *mut i32) -> i32;
    pub fn fg_debug_plan(roots: *mut *mut fg_tensor, n: i32, fuse: i32, render_hip: i32, buf: *mut c_char,
                         len: usize, needed: *mut usize) -> i32;
}

// ── status handling and owning wrappers ─────────────────────────────────────

/// A failed call: its status code and the library's message.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct Error {
    pub code: i32,
    pub message: String,
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "ferrograd_amd error {}: {}", self.code, self.message)
    }
}

impl std::error::Error for Error {}

fn message(p: *const c_char) -> String {
    if p.is_null() {
        return String::new();
    }
    // SAFETY: the library returns a NUL-terminated, thread-local string that
    // stays valid until the next failing call on this thread.
    unsafe { CStr::from_ptr(p) }.to_string_lossy().into_owned()
}

/// A device-call status as a `Result` (message from `fg_hip_last_error`).
pub fn hip_result(code: i32) -> Result<(), Error> {
    if code == FG_OK {
        Ok(())
    } else {
        // SAFETY: plain C call with no arguments.
        Err(Error { code, message: message(unsafe { fg_hip_last_error() }) })
    }
}

/// A front-end status as a `Result` (message from `fg_last_error`).
pub fn fg_result(code: i32) -> Result<(), Error> {
    if code == 0 {
        Ok(())
    } else {
        // SAFETY: plain C call with no arguments.
        Err(Error { code, message: message(unsafe { fg_last_error() }) })
    }
}

/// An owned `fg_ctx` (destroyed on drop).
pub struct Context(pub *mut fg_ctx);

impl Context {
    /// `fg_hip_init(ordinal)`: select the GPU and create the context's stream.
    pub fn new(ordinal: i32) -> Result<Self, Error> {
        let mut c = std::ptr::null_mut();
        // SAFETY: `c` is a valid out-pointer.
        hip_result(unsafe { fg_hip_init(ordinal, &mut c) })?;
        Ok(Self(c))
    }

    pub fn sync(&self) -> Result<(), Error> {
        // SAFETY: `self.0` is a live context.
        hip_result(unsafe { fg_hip_sync(self.0) })
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        // SAFETY: `self.0` came from fg_hip_init and is destroyed once.
        unsafe { fg_hip_destroy(self.0) };
    }
}

/// One launch pass of a rendered kernel.
#[derive(Debug, Clone)]
pub struct Launch {
    pub func: String,
    pub grid: [u32; 3],
    pub block: [u32; 3],
    pub lds_bytes: u32,
}

/// An owned `fg_rendered`: the Renderer half of the boundary.
pub struct Rendered(pub *mut fg_rendered);

impl Rendered {
    /// `fg_hip_render`: a rangeified kernel in fg-kernel text form to gfx950
    /// HIP source, launch passes and parameter kinds.
    pub fn new(kernel_text: &str) -> Result<Self, Error> {
        let t = CString::new(kernel_text).map_err(|_| Error { code: FG_ERR_INVALID, message: "NUL in kernel text".into() })?;
        let mut r = std::ptr::null_mut();
        // SAFETY: `t` outlives the call; `r` is a valid out-pointer.
        hip_result(unsafe { fg_hip_render(t.as_ptr(), &mut r) })?;
        Ok(Self(r))
    }

    /// (source, lowering class, parameter count, launch count, scratch bytes).
    pub fn info(&self) -> Result<(String, String, usize, usize, usize), Error> {
        let (mut src, mut kind) = (std::ptr::null(), std::ptr::null());
        let (mut np, mut nl, mut scratch) = (0i32, 0i32, 0usize);
        // SAFETY: `self.0` is live; every out-pointer is valid.
        hip_result(unsafe { fg_hip_rendered_info(self.0, &mut src, &mut kind, &mut np, &mut nl, &mut scratch) })?;
        Ok((message(src), message(kind), np as usize, nl as usize, scratch))
    }

    /// The FG_ARG_* kind the kernel expects in parameter `slot`.
    pub fn param_kind(&self, slot: usize) -> Result<i32, Error> {
        let mut k = 0;
        // SAFETY: `self.0` is live; `k` is a valid out-pointer.
        hip_result(unsafe { fg_hip_rendered_param(self.0, slot as i32, &mut k) })?;
        Ok(k)
    }

    pub fn launch(&self, i: usize) -> Result<Launch, Error> {
        let mut func = std::ptr::null();
        let (mut grid, mut block, mut lds) = ([0u32; 3], [0u32; 3], 0u32);
        // SAFETY: `self.0` is live; the arrays hold three elements each.
        hip_result(unsafe {
            fg_hip_rendered_launch(self.0, i as i32, &mut func, grid.as_mut_ptr(), block.as_mut_ptr(), &mut lds)
        })?;
        Ok(Launch { func: message(func), grid, block, lds_bytes: lds })
    }
}

impl Drop for Rendered {
    fn drop(&mut self) {
        // SAFETY: `self.0` came from fg_hip_render and is freed once.
        unsafe { fg_hip_rendered_free(self.0) };
    }
}

/// An owned `fg_kernel`: `Device::compile` with the geometry attached.
pub struct Kernel(pub *mut fg_kernel);

impl Kernel {
    pub fn load(ctx: &Context, r: &Rendered) -> Result<Self, Error> {
        let mut k = std::ptr::null_mut();
        // SAFETY: both handles are live; `k` is a valid out-pointer.
        hip_result(unsafe { fg_hip_kernel_load(ctx.0, r.0, &mut k) })?;
        Ok(Self(k))
    }

    /// `Device::execute`: every pass queued on the context's stream.
    pub fn run(&self, ctx: &Context, args: &[fg_arg]) -> Result<(), Error> {
        // SAFETY: handles are live; `args` holds `args.len()` arguments.
        hip_result(unsafe { fg_hip_kernel_run(ctx.0, self.0, args.as_ptr(), args.len() as i32) })
    }

    /// `run` with no device allocation (static per-GPU scratch; see the header).
    pub fn run_noalloc(&self, ctx: &Context, args: &[fg_arg]) -> Result<(), Error> {
        // SAFETY: as for `run`.
        hip_result(unsafe { fg_hip_kernel_run_noalloc(ctx.0, self.0, args.as_ptr(), args.len() as i32) })
    }
}

impl Drop for Kernel {
    fn drop(&mut self) {
        // SAFETY: `self.0` came from fg_hip_kernel_load and is freed once.
        unsafe { fg_hip_kernel_free(self.0) };
    }
}

/// Binding A: a tensor handle of the front end. Cloning aliases the shared
/// tensor state, like cloning a reference `Tensor` (tensor.rs:30-38).
pub struct Tensor(pub *mut fg_tensor);

impl Tensor {
    pub fn from_f32(data: &[f32], shape: &[i64], device: i32) -> Result<Self, Error> {
        let mut t = std::ptr::null_mut();
        // SAFETY: `data` and `shape` outlive the call; `t` is a valid out-pointer.
        fg_result(unsafe {
            fg_tensor_from_data(device, FG_F32, data.as_ptr().cast(), std::mem::size_of_val(data), shape.as_ptr(),
                                shape.len() as i32, &mut t)
        })?;
        Ok(Self(t))
    }

    fn unary(&self, op: i32) -> Result<Self, Error> {
        let mut t = std::ptr::null_mut();
        // SAFETY: `self.0` is live; `t` is a valid out-pointer.
        fg_result(unsafe { fg_tensor_unary(self.0, op, &mut t) })?;
        Ok(Self(t))
    }

    fn binary(&self, other: &Self, op: i32) -> Result<Self, Error> {
        let mut t = std::ptr::null_mut();
        // SAFETY: both handles are live; `t` is a valid out-pointer.
        fg_result(unsafe { fg_tensor_binary(self.0, other.0, op, &mut t) })?;
        Ok(Self(t))
    }

    pub fn add(&self, o: &Self) -> Result<Self, Error> { self.binary(o, FG_BINARY_ADD) }
    pub fn mul(&self, o: &Self) -> Result<Self, Error> { self.binary(o, FG_BINARY_MUL) }
    pub fn sub(&self, o: &Self) -> Result<Self, Error> { self.binary(o, FG_BINARY_SUB) }
    pub fn matmul(&self, o: &Self) -> Result<Self, Error> { self.binary(o, FG_BINARY_MATMUL) }
    pub fn cross_entropy(&self, targets: &Self) -> Result<Self, Error> { self.binary(targets, FG_BINARY_CROSS_ENTROPY) }
    pub fn relu(&self) -> Result<Self, Error> { self.unary(FG_UNARY_RELU) }
    pub fn exp(&self) -> Result<Self, Error> { self.unary(FG_UNARY_EXP) }
    pub fn log(&self) -> Result<Self, Error> { self.unary(FG_UNARY_LOG) }

    pub fn sum(&self, axes: &[i64]) -> Result<Self, Error> {
        let mut t = std::ptr::null_mut();
        // SAFETY: `self.0` is live; `axes` outlives the call.
        fg_result(unsafe { fg_tensor_reduce(self.0, FG_REDUCE_SUM, axes.as_ptr(), axes.len() as i32, &mut t) })?;
        Ok(Self(t))
    }

    pub fn permute(&self, axes: &[i64]) -> Result<Self, Error> {
        let mut t = std::ptr::null_mut();
        // SAFETY: `self.0` is live; `axes` outlives the call.
        fg_result(unsafe { fg_tensor_movement(self.0, FG_MOVE_PERMUTE, axes.as_ptr(), axes.len() as i32, &mut t) })?;
        Ok(Self(t))
    }

    /// `Tensor::realize_many` (tensor.rs:780-821) over `ts`.
    pub fn realize_many(ts: &[&Self]) -> Result<(), Error> {
        let mut hs: Vec<*mut fg_tensor> = ts.iter().map(|t| t.0).collect();
        // SAFETY: every handle is live for the call.
        fg_result(unsafe { fg_tensor_realize_many(hs.as_mut_ptr(), hs.len() as i32) })
    }

    /// `Tensor::to_vec` (tensor.rs:907-930): realise and read back f32 data.
    pub fn to_vec(&self, numel: usize) -> Result<Vec<f32>, Error> {
        Self::realize_many(&[self])?;
        let mut out = vec![0f32; numel];
        // SAFETY: `out` holds `numel` f32; the call checks the size.
        fg_result(unsafe { fg_tensor_read(self.0, out.as_mut_ptr().cast(), numel * 4) })?;
        Ok(out)
    }
}

impl Clone for Tensor {
    fn clone(&self) -> Self {
        self.unary(FG_UNARY_ALIAS).expect("fg_tensor_unary(ALIAS) does not fail on a live handle")
    }
}

impl Drop for Tensor {
    fn drop(&mut self) {
        // SAFETY: `self.0` is owned by this handle and freed once.
        unsafe { fg_tensor_free(self.0) };
    }
}
