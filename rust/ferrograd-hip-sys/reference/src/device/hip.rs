//! `src/device/hip.rs` — the module the ferrograd crate adds to run its
//! realize path on one MI355X through `ferrograd-hip-sys` (binding B).
//!
//! NOT BUILT IN THIS REPOSITORY: the build image has no Rust toolchain. It is
//! written against the reference's Device trait (src/device.rs:275-332), its
//! Renderer trait (src/codegen.rs:17-20), Buffer/Storage (device.rs:60-228)
//! and UOp (uop.rs:390-427, 561-1079), and needs these edits elsewhere in the
//! crate (each one line or one match arm):
//!
//! 1. `DeviceId::Hip` (device.rs:38-41) and its Display name "hip".
//! 2. `Storage::Hip(Rc<HipAlloc>)` (device.rs:66-70), with `HipAlloc` below.
//! 3. `Program::Hip { kernel: HipKernel, num_args: usize }` (device.rs:260-270).
//! 4. `DeviceError::Hip(String)` (device.rs:53-58).
//! 5. `new_device`: `DeviceId::Hip => Rc::new(HipDevice::new())` (device.rs:338-342).
//! 6. `realize_many` (tensor.rs:800-818): for a HIP sink, skip optimize /
//!    late_expand / devectorize (the gfx950 lowering runs inside
//!    `fg_hip_render` on the rangeified kernel) and render with `HipRenderer`:
//!
//!    ```ignore
//!    let rangeified = rangeify(&item.sink);
//!    if rangeified.device() == DeviceId::Hip {
//!        Self::execute_item_with(&HipRenderer, &rangeified, &item.inputs, item.output_buffer.as_ref());
//!        continue;
//!    }
//!    ```
//!
//!    where `execute_item_with` is `execute_item` (tensor.rs:832-893) with the
//!    renderer passed in instead of the hard-coded `ClangRenderer`
//!    (tensor.rs:850) and `linearize` applied only for the clang renderer.
//!
//! The program cache key stays the kernel sink (device.rs:323-327), and
//! kernel arguments stay `KernelArg` in parameter-slot order.

use std::cell::RefCell;
use std::collections::HashMap;
use std::ffi::c_void;
use std::fmt::Write as _;
use std::rc::Rc;

use ferrograd_hip_sys as sys;

use super::{Buffer, Device, DeviceError, DeviceId, KernelArg, Program, Storage};
use crate::codegen::Renderer;
use crate::dtype::{DType, DTypeKind};
use crate::uop::{Arg, AxisKind, UOp};

// ── Renderer half: the kernel as fg-kernel text ────────────────────────────

/// Renders a rangeified kernel for the HIP device. The "source" it returns is
/// the kernel in the fg-kernel text form of include/ferrograd_hip.h (one
/// node per line, in toposort order); `HipDevice::compile` hands that text
/// to `fg_hip_render`, which runs the gfx950 passes and produces the HIP
/// source and launch passes.
pub struct HipRenderer;

impl Renderer for HipRenderer {
    fn render(&self, uops: &[UOp], _name: &str) -> String {
        // Called with the rangeified sink as the only (last) element.
        kernel_text(uops.last().expect("HipRenderer renders one kernel sink"))
    }
}

fn dtype_text(d: DType) -> String {
    let base = match d.kind() {
        DTypeKind::F32 => "f32",
        DTypeKind::I32 => "i32",
        DTypeKind::Bool => "bool",
        DTypeKind::Void => "void",
    };
    if d.vcount() == 1 { base.to_string() } else { format!("{base}x{}", d.vcount()) }
}

fn axis_text(k: AxisKind) -> &'static str {
    match k {
        AxisKind::Loop => "LOOP",
        AxisKind::Global => "GLOBAL",
        AxisKind::Local => "LOCAL",
        AxisKind::Reduce => "REDUCE",
        AxisKind::GroupReduce => "GROUP_REDUCE",
        AxisKind::Upcast => "UPCAST",
        AxisKind::Unroll => "UNROLL",
        AxisKind::Thread => "THREAD",
    }
}

fn list(v: impl IntoIterator<Item = usize>) -> String {
    v.into_iter().map(|x| x.to_string()).collect::<Vec<_>>().join(",")
}

fn arg_text(a: &Arg) -> String {
    match a {
        Arg::None => "-".into(),
        Arg::Device(d) => format!("device:{d}"),
        Arg::Variable(name, lo, hi) => format!("var:{name}:{lo}:{hi}"),
        Arg::Index(i) => format!("index:{i}"),
        Arg::Range(axis, kind) => format!("range:{axis}:{}", axis_text(*kind)),
        Arg::ParamBuffer(slot, numel) => format!("param:{slot}:{numel}"),
        Arg::ParamScalar(slot) => format!("scalar:{slot}"),
        Arg::Float(f) => format!("float:{:016x}", f.to_bits()),
        Arg::Int(i) => format!("int:{i}"),
        Arg::Bool(b) => format!("bool:{}", u8::from(*b)),
        Arg::Bounds(b) => format!("bounds:{}", list(b.iter().copied())),
        Arg::Shape(s) => format!("shape:{}", list(s.iter().copied())),
        Arg::Axes(a) => format!("axes:{}", list(a.iter().copied())),
        Arg::Lanes(l) => format!("lanes:{}", list(l.iter().flat_map(|&(axis, n)| [axis, n]))),
        Arg::Reduce(op, axes) => format!("reduce:{op:?}:{}", list(axes.iter().copied())),
        Arg::Buffer(_) => panic!("a kernel refers to memory by ParamBuffer slot, never by Buffer"),
    }
}

/// The fg-kernel text of a rangeified kernel: "fg-kernel 1", then for node i
/// of `sink.toposort()` the line `<Op> <dtype> <arg> [#tag] <source ids>`.
#[must_use]
pub fn kernel_text(sink: &UOp) -> String {
    let order = sink.toposort();
    let mut id: HashMap<*const (), usize> = HashMap::with_capacity(order.len());
    let mut out = String::from("fg-kernel 1\n");
    for (i, n) in order.iter().enumerate() {
        let _ = write!(out, "{:?} {} {}", n.op(), dtype_text(n.dtype()), arg_text(n.arg()));
        if let Some(tag) = n.0.tag {
            let _ = write!(out, " #{tag}");
        }
        for s in n.srcs() {
            let _ = write!(out, " {}", id[&(Rc::as_ptr(&s.0).cast::<()>())]);
        }
        out.push('\n');
        id.insert(Rc::as_ptr(&n.0).cast::<()>(), i);
    }
    out
}

// ── Device half ─────────────────────────────────────────────────────────────

/// Device memory of one HIP buffer, freed when the last Storage clone drops.
#[derive(Debug)]
pub struct HipAlloc {
    ctx: *mut sys::fg_ctx,
    pub ptr: *mut c_void,
    pub len: usize,
}

impl Drop for HipAlloc {
    fn drop(&mut self) {
        // SAFETY: `ptr` came from fg_hip_alloc on `ctx` and is freed once.
        unsafe { sys::fg_hip_free(self.ctx, self.ptr) };
    }
}

/// A rendered, compiled and loaded kernel (`Program::Hip`).
#[derive(Debug)]
pub struct HipKernel {
    kernel: *mut sys::fg_kernel,
    kinds: Vec<i32>,
}

impl Drop for HipKernel {
    fn drop(&mut self) {
        // SAFETY: `kernel` came from fg_hip_kernel_load and is freed once.
        unsafe { sys::fg_hip_kernel_free(self.kernel) };
    }
}

/// The MI355X device: one HIP context (stream) and the program cache.
pub struct HipDevice {
    ctx: sys::Context,
    cache: RefCell<HashMap<UOp, Rc<Program>>>,
}

impl HipDevice {
    /// # Panics
    /// Panics with the runtime's message when no usable GPU is present.
    #[must_use]
    pub fn new() -> Self {
        let ordinal = std::env::var("FG_HIP_DEVICE").ok().and_then(|v| v.parse().ok()).unwrap_or(0);
        let ctx = sys::Context::new(ordinal).unwrap_or_else(|e| panic!("hip: {e}"));
        Self { ctx, cache: RefCell::new(HashMap::new()) }
    }

    fn ptr_of(b: &Buffer) -> *mut c_void {
        match b.0.storage.borrow().as_ref() {
            Some(Storage::Hip(a)) => a.ptr,
            Some(_) => panic!("buffer {} does not live on the HIP device", b.id()),
            None => panic!("buffer {} is not realized", b.id()),
        }
    }
}

impl Default for HipDevice {
    fn default() -> Self {
        Self::new()
    }
}

fn hip_err(e: &sys::Error) -> DeviceError {
    DeviceError::Hip(e.to_string())
}

impl Device for HipDevice {
    fn id(&self) -> DeviceId {
        DeviceId::Hip
    }

    fn reserve_buffer(&self, dtype: DType, numel: usize) -> Buffer {
        Buffer::reserved(DeviceId::Hip, dtype, numel)
    }

    /// Zero-filled, as the trait requires (device.rs:282).
    fn allocate(&self, dtype: DType, numel: usize) -> Buffer {
        let len = dtype.size_bytes() * numel;
        let mut ptr = std::ptr::null_mut();
        // SAFETY: `ptr` is a valid out-pointer; the context is live.
        sys::hip_result(unsafe { sys::fg_hip_alloc(self.ctx.0, len, 1, &mut ptr) })
            .unwrap_or_else(|e| panic!("hip: {e}"));
        Buffer::new(DeviceId::Hip, dtype, numel, Storage::Hip(Rc::new(HipAlloc { ctx: self.ctx.0, ptr, len })))
    }

    /// Panics on a size mismatch with the CPU backend's message (cpu.rs:294-300).
    fn copy_from_host(&self, buffer: &Buffer, src: &[u8]) {
        assert_eq!(buffer.device(), DeviceId::Hip, "copy_from_host: buffer is not on the HIP device");
        assert_eq!(src.len(), buffer.nbytes(), "copy_from_host: expected {} bytes, got {}", buffer.nbytes(), src.len());
        buffer.ensure_allocated();
        // SAFETY: the device buffer holds `src.len()` bytes.
        sys::hip_result(unsafe { sys::fg_hip_copy_h2d(self.ctx.0, Self::ptr_of(buffer), src.as_ptr().cast(), src.len()) })
            .unwrap_or_else(|e| panic!("hip: {e}"));
    }

    /// Waits for the stream, then copies (device.rs:302-308).
    fn copy_to_host(&self, buffer: &Buffer) -> Vec<u8> {
        let mut out = vec![0u8; buffer.nbytes()];
        // SAFETY: `out` holds the buffer's byte size.
        sys::hip_result(unsafe {
            sys::fg_hip_copy_d2h(self.ctx.0, out.as_mut_ptr().cast(), Self::ptr_of(buffer), out.len())
        })
        .unwrap_or_else(|e| panic!("hip: {e}"));
        out
    }

    /// `source` is HipRenderer's kernel text: render for gfx950, compile with
    /// hiprtc (the library's code-object cache applies) and load. The launch
    /// geometry travels inside the loaded kernel.
    fn compile(&self, source: &str, _func_name: &str, num_args: usize) -> Result<Program, DeviceError> {
        let rendered = sys::Rendered::new(source).map_err(|e| hip_err(&e))?;
        let (_, _, num_params, _, _) = rendered.info().map_err(|e| hip_err(&e))?;
        if num_params != num_args {
            return Err(DeviceError::Hip(format!("kernel takes {num_params} arguments, caller passes {num_args}")));
        }
        let kinds = (0..num_params).map(|s| rendered.param_kind(s)).collect::<Result<Vec<_>, _>>()
            .map_err(|e| hip_err(&e))?;
        let kernel = sys::Kernel::load(&self.ctx, &rendered).map_err(|e| hip_err(&e))?;
        let raw = kernel.0;
        std::mem::forget(kernel); // owned by HipKernel from here on
        Ok(Program::Hip { kernel: HipKernel { kernel: raw, kinds }, num_args })
    }

    /// Queues every launch pass on the context's stream (no host wait).
    fn execute(&self, program: &Program, args: &mut [KernelArg]) -> Result<(), DeviceError> {
        let Program::Hip { kernel, num_args } = program else {
            return Err(DeviceError::Hip("not a HIP program".into()));
        };
        assert_eq!(args.len(), *num_args, "kernel expects {num_args} args, got {}", args.len());
        let a: Vec<sys::fg_arg> = args
            .iter()
            .zip(&kernel.kinds)
            .map(|(arg, &kind)| match arg {
                KernelArg::Buffer(b) => {
                    b.ensure_allocated();
                    sys::fg_arg::ptr(Self::ptr_of(b))
                }
                KernelArg::I32(i) => sys::fg_arg::i32(*i),
                KernelArg::F32(f) => sys::fg_arg::f32(*f),
                KernelArg::Bool(b) => {
                    debug_assert_eq!(kind, sys::FG_ARG_BOOL);
                    sys::fg_arg::boolean(*b)
                }
            })
            .collect();
        // SAFETY: `a` holds one argument per kernel parameter, in slot order.
        sys::hip_result(unsafe { sys::fg_hip_kernel_run(self.ctx.0, kernel.kernel, a.as_ptr(), a.len() as i32) })
            .map_err(|e| hip_err(&e))
    }

    fn cached_program(&self, sink: &UOp) -> Option<Rc<Program>> {
        self.cache.borrow().get(sink).cloned()
    }

    fn insert_program(&self, sink: UOp, program: Rc<Program>) {
        self.cache.borrow_mut().insert(sink, program);
    }

    #[cfg(test)]
    fn clear_for_tests(&self) {
        self.cache.borrow_mut().clear();
    }
}
