// Device layer: Buffer identity, kernel arguments, compiled programs and the
// device interface that backends implement (src/device.rs:96-354).
//
// The reference trait compiles a source string with no launch geometry
// (device.rs:309-314) and hard-codes the clang renderer at the call site
// (tensor.rs:850). Here each device owns its lowering: `optimize` runs the
// device's kernel passes on a rangeified kernel, `render` produces source plus
// launch geometry, and `compile`/`execute` mirror the reference trait.
#pragma once

#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "ir.hpp"

namespace fg {

class Device;

struct BufferInner {
  size_t id = 0;
  DeviceId device = DeviceId::Hip;
  DType dtype;
  size_t numel = 0;
  void* storage = nullptr;  // device pointer for HIP, host pointer for CPU
  bool realized = false;
  // Holds the zeros `allocate` produced and nothing has written it since
  // (allocation contract: device.rs:282, cpu.rs:277-280).
  bool known_zero = false;
  // Allocated as zeros but storage not created yet (the HIP device
  // materialises zero-filled allocations on first use).
  bool zero_init = false;
  size_t nbytes() const { return dtype.size_bytes() * numel; }
  bool is_realized() const { return realized; }
  void ensure_allocated();  // device.rs:191-213
  ~BufferInner();
};

size_t next_buffer_id();

// device.rs:242-251
struct KernelArg {
  enum class Kind : uint8_t { Buffer, I32, F32, Bool } kind = Kind::I32;
  Buffer buffer;
  int32_t i = 0;
  float f = 0.f;
  bool b = false;
  static KernelArg buf(const Buffer& x) { KernelArg a; a.kind = Kind::Buffer; a.buffer = x; return a; }
  static KernelArg i32(int32_t x) { KernelArg a; a.kind = Kind::I32; a.i = x; return a; }
  static KernelArg f32(float x) { KernelArg a; a.kind = Kind::F32; a.f = x; return a; }
  static KernelArg boolean(bool x) { KernelArg a; a.kind = Kind::Bool; a.b = x; return a; }
};

// One kernel launch of a program.
struct LaunchSpec {
  std::string func;
  unsigned grid[3] = {1, 1, 1};
  unsigned block[3] = {1, 1, 1};
  unsigned lds_bytes = 0;
};

// What a renderer hands to `Device::compile`: the source and everything the
// launch needs that the reference's `compile(source, name, num_args)` lacks.
struct RenderedKernel {
  std::string source;
  std::string name;
  unsigned grid[3] = {1, 1, 1};
  unsigned block[3] = {1, 1, 1};
  unsigned lds_bytes = 0;
  std::string kind;  // lowering class, for debug output and tests
  std::vector<std::pair<int, DType>> params;  // (slot, dtype) in launch order
  int out_slot = -1;                           // the parameter slot the kernel stores to
  bool reads_output = false;                   // whether it also loads from that parameter (in place)
  size_t out_count = 0;                        // elements of that parameter it stores
  // Multi-kernel programs: when non-empty these launches run in order instead
  // of the single (name, grid, block) launch. With scratch_bytes > 0 the
  // program owns a device scratch buffer passed as the last argument of every
  // launch (partial results between passes; nothing needs zeroing).
  std::vector<LaunchSpec> launches;
  size_t scratch_bytes = 0;
  // Block kernels (one workgroup): the device function the kernel calls, its
  // parameter types in slot order, and its source, so a device can run a run
  // of them as one launch (render_block_batch).
  std::string stage_fn, stage_src;
  std::vector<std::string> stage_types;
  // Kernels whose body is a device function of its block index (the small
  // GEMM): the function, its source and its parameter types in slot order,
  // so a device can run two independent ones in one launch (render_hfused).
  std::string hbody_fn, hbody_src;
  std::vector<std::string> hbody_types;
};

struct Program {
  virtual ~Program() = default;
  size_t num_args = 0;
  RenderedKernel meta;
};

class Device {
 public:
  virtual ~Device() = default;
  virtual DeviceId id() const = 0;

  // device.rs:280 — identity only, no storage.
  Buffer reserve_buffer(DType dtype, size_t numel);
  // device.rs:283 — zero-initialised storage.
  virtual Buffer allocate(DType dtype, size_t numel) = 0;
  // Give a reserved buffer storage. `zero` asks for zero-filled memory; kernel
  // outputs that overwrite every element pass false.
  virtual void realize_storage(BufferInner& b, bool zero) = 0;
  // realize_storage preferring the storage at `hint` (a replayed plan asks for
  // the blocks its outputs had last time). Devices without the notion ignore it.
  virtual void realize_storage_at(BufferInner& b, bool zero, void* hint) {
    (void)hint;
    realize_storage(b, zero);
  }
  virtual void release(BufferInner& b) = 0;
  virtual void copy_from_host(const Buffer& b, const void* src, size_t nbytes) = 0;
  virtual std::vector<uint8_t> copy_to_host(const Buffer& b) = 0;
  // copy_to_host into the caller's `nbytes` (which must be the buffer's
  // size), with no intermediate vector.
  virtual void copy_to_host_into(const Buffer& b, void* dst, size_t nbytes);
  // A read-back that need not finish before the caller queues more work:
  // read_async takes the buffer's bytes (as copy_to_host would) into `slot`
  // once the device has run what is already queued; read_wait returns them.
  // A device that runs synchronously, as the default does, copies at once.
  virtual void read_async(const Buffer& b, int slot);
  virtual std::vector<uint8_t> read_wait(int slot);

  // Kernel pipeline after rangeify.
  virtual UOp optimize(const UOp& rangeified) = 0;
  // The optimized kernel made ready to render against the scheduled one it
  // came from (the HIP device keeps every parameter in its signature).
  virtual UOp bind_params(const UOp& optimized, const UOp& scheduled) {
    (void)scheduled;
    return optimized;
  }
  virtual RenderedKernel render(const UOp& optimized, const std::string& name) = 0;
  virtual std::shared_ptr<Program> compile(const RenderedKernel& rk, size_t num_args) = 0;
  virtual void execute(Program& p, std::vector<KernelArg>& args) = 0;
  // Run a recorded sequence of launches (a replayed realisation plan) in
  // order. `state` is a slot owned by the sequence's record, in which the
  // device may keep replay state between calls; it is dropped with the record.
  virtual void execute_sequence(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                                std::shared_ptr<void>& state) {
    (void)state;
    for (size_t i = 0; i < progs.size(); i++) execute(*progs[i], args[i]);
  }
  // execute_sequence, then `result` read back into `slot` as read_async
  // does. A device may fold the copy into the sequence itself.
  virtual void execute_sequence_read(const std::vector<Program*>& progs, std::vector<std::vector<KernelArg>>& args,
                                     std::shared_ptr<void>& state, const Buffer& result, int slot) {
    execute_sequence(progs, args, state);
    read_async(result, slot);
  }
  virtual void synchronize() {}
  // Brackets a loop that only replays recorded sequences (the native train
  // loop's captured steps): a device may launch them on a faster path in
  // between. Everything queued is ordered as without the brackets.
  virtual void begin_replay_loop() {}
  virtual void end_replay_loop() {}
  // Whether schedule-time value-preserving fusion (shared elementwise
  // subexpressions inlined into one kernel, zero buffers folded) is enabled.
  virtual bool fuse_elementwise() const { return false; }
  // Whether relu may take its zeros from one never-written buffer per
  // (dtype, shape) instead of allocating fresh zeros per call as the
  // reference does (tensor.rs:517-531); same values, no allocation.
  virtual bool shares_relu_zeros() const { return false; }

  // device.rs:323-327
  std::shared_ptr<Program> cached_program(const UOp& sink);
  void insert_program(const UOp& sink, std::shared_ptr<Program> p);
  void clear_for_tests();
  size_t cache_size() const { return programs_.size(); }

 protected:
  UOpMap<std::shared_ptr<Program>> programs_;

 private:
  std::vector<std::pair<int, std::vector<uint8_t>>> read_slots_;
};

// Registry (device.rs:334-354). The HIP device is built in; the CPU device is
// provided by the test oracle, which registers itself at load time.
Device& get_device(DeviceId id);
bool has_device(DeviceId id);
// The device programs use when they name none: the reference's tensor::cpu()
// (tensor.rs:1122-1127) with the choice moved to the DEVICE environment
// variable, "hip" (the default, MI355X) or "cpu" (registered only by the test
// oracle). Read once per process; any other value is an error.
DeviceId default_device();
void register_device(DeviceId id, Device* dev);
Device* make_hip_device();
// Replayed launch sequences of at least this many launches run as one HIP
// graph (default 2); shorter ones are launched one by one. The setter returns
// the previous value.
int graph_min_launches();
int set_graph_min_launches(int n);
// The HIP device's runtime context (an fg_ctx*), created on first use.
void* hip_context_raw();

}  // namespace fg
