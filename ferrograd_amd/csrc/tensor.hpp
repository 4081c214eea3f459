// Tensor front end, autograd, nn::Linear and optim::Sgd
// (src/tensor.rs, src/gradient.rs, src/nn.rs, src/optim.rs).
#pragma once

#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "device.hpp"
#include "ir.hpp"
#include "schedule.hpp"

namespace fg {

struct TensorInner;

// A shared handle to lazy graph state (tensor.rs:84-97): clones alias one
// identity so realisation and in-place updates are visible through all handles.
class Tensor {
 public:
  Tensor() = default;
  explicit Tensor(std::shared_ptr<TensorInner> p) : p_(std::move(p)) {}

  // Constructors (tensor.rs:260-312).
  static Tensor from_bytes(const void* data, size_t nbytes, const Shape& shape, DType dtype, DeviceId dev);
  static Tensor new_f32(const std::vector<float>& data, const Shape& shape, DeviceId dev);
  static Tensor zeros(const Shape& shape, DeviceId dev, DType dtype);
  static Tensor ones(const Shape& shape, DeviceId dev, DType dtype);
  static Tensor full_f32(const Shape& shape, float value, DeviceId dev);
  static Tensor scalar_f32(float value, DeviceId dev);
  static Tensor from_uop(const UOp& u, bool requires_grad);

  DeviceId device() const;
  DType dtype() const;
  Shape shape() const;
  const Shape& shape_ref() const;  // no copy; valid while the tensor's graph node lives
  size_t numel() const;
  size_t ndim() const;
  bool is_realized() const;
  bool requires_grad() const;
  std::optional<Tensor> grad() const;
  void clear_grad() const;
  Tensor with_requires_grad(bool rg) const;
  Tensor detach() const;
  Tensor replace(const Tensor& other) const;
  Tensor assign(const Tensor& other) const;

  // Elementwise (tensor.rs:442-531).
  Tensor add(const Tensor& o) const;
  Tensor mul(const Tensor& o) const;
  Tensor neg() const;
  Tensor sub(const Tensor& o) const;
  Tensor reciprocal() const;
  Tensor exp2() const;
  Tensor log2() const;
  Tensor sqrt() const;
  Tensor relu() const;
  Tensor exp() const;
  Tensor log() const;

  // Movement (tensor.rs:539-657).
  Tensor reshape(const Shape& s) const;
  Tensor narrow(size_t dim, size_t start, size_t len) const;
  Tensor permute(const std::vector<size_t>& order) const;
  Tensor contiguous() const;
  Tensor expand(const Shape& s) const;

  // Reductions and composites (tensor.rs:665-778).
  Tensor sum(const std::vector<size_t>& axes) const;
  Tensor max(const std::vector<size_t>& axes) const;
  Tensor log_softmax(size_t axis) const;
  Tensor cross_entropy(const Tensor& targets) const;
  Tensor matmul(const Tensor& other) const;

  // Realisation (tensor.rs:781-930).
  static void realize_many(const std::vector<Tensor>& tensors);
  Tensor realize() const;
  std::vector<float> to_vec() const;
  std::vector<uint8_t> to_bytes() const;
  Buffer realized_buffer() const;

  // Autograd (tensor.rs:938-998).
  std::vector<Tensor> gradient(const std::vector<Tensor>& targets) const;
  void backward() const;

  UOp uop() const;
  void set_uop(const UOp& u) const;
  bool ptr_eq(const Tensor& o) const { return p_ == o.p_; }
  TensorInner* raw() const { return p_.get(); }
  explicit operator bool() const { return static_cast<bool>(p_); }

 private:
  Tensor unary(Op op) const;
  Tensor binary(const Tensor& o, Op op, DType out) const;
  Tensor broadcasted(const Tensor& o, Op op, DType out) const;
  UOp target_uop() const;
  std::shared_ptr<TensorInner> p_;
};

struct TensorInner {
  UOp uop;
  bool requires_grad = false;
  std::shared_ptr<TensorInner> grad;
};

// gradient.rs:20-58
UOpMap<UOp> compute_gradient(const UOp& root, const UOp& root_grad, const std::vector<UOp>& targets);
// compute_gradient with the root's toposort already computed (root = its last node).
UOpMap<UOp> compute_gradient_ordered(const std::vector<UOp>& order, const UOp& root_grad,
                                     const std::vector<UOp>& targets);

// nn.rs — seeded Kaiming-normal init and Linear.
void reset_init_seed(uint64_t seed = 42);
Tensor kaiming_normal(const Shape& shape, size_t fan_in, DeviceId dev);
struct Linear {
  Tensor weight;
  std::optional<Tensor> bias;
  static Linear create(size_t in_features, size_t out_features, DeviceId dev, bool with_bias = true);
  Tensor forward(const Tensor& x) const;
  std::vector<Tensor> parameters() const;
};

// optim.rs:16-71
struct Sgd {
  std::vector<Tensor> params;
  float lr;
  // The learning rate as a 1-element buffer per device, uploaded on the first
  // step and only ever read (optim.rs:62 builds Tensor::scalar(lr) for every
  // parameter on every step; the values are the same, without a host->device
  // copy per parameter per step).
  mutable std::vector<std::pair<DeviceId, Tensor>> lr_buffers;
  Sgd(const std::vector<Tensor>& params, float lr);
  void zero_grad() const;
  void step() const;
};

// The nodes live tensors point at (tensor.rs:201-214), as a lookup map and a
// list, for the HIP schedule's fusions to leave to the reference's rules.
void collect_held_nodes(PtrIndexMap* held, std::vector<const UOpInner*>* list);

// The examples/mnist.rs:84-101 loop body run `steps` times from native code,
// as a compiled caller of the reference runs it: logits = layers through ReLU
// between them (mnist.rs:30-54 generalised to any depth), loss =
// cross_entropy, zero_grad, backward, step, then the loss read back. Returns
// each step's loss. With `batch` > 0, `x` and `targets` are whole datasets and
// step i trains on rows [s, s + batch) through narrow(), s = ((first_batch +
// i) mod (rows / batch)) * batch, as mnist.rs:84-87 batches an epoch.
std::vector<float> train_steps(const std::vector<const Linear*>& layers, const Sgd& opt, const Tensor& x,
                               const Tensor& targets, int steps, int64_t batch = 0, int64_t first_batch = 0);

// Offline MNIST IDX files (dataset.rs:116-161): images as f32 [count, 784]
// scaled by 1/255 on `dev`, labels as bytes.
Tensor idx_images(const std::string& path, DeviceId dev);
std::vector<uint8_t> idx_labels(const std::string& path);

// Per-process statistics used by tests and the benchmark.
struct RealizeStats {
  size_t kernels_launched = 0;
  size_t programs_compiled = 0;
  size_t lowering_cache_hits = 0;
  // Host time (ns) spent in each stage of realize_many / backward.
  uint64_t ns_schedule = 0, ns_lower = 0, ns_launch = 0, ns_apply_map = 0, ns_backward = 0;
  // Replayed plans that ran as one HIP graph launch, and the launches inside
  // them whose arguments had to be updated first.
  size_t graph_replays = 0, graph_updates = 0;
  // Native training loops: steps captured, and steps launched from a capture
  // without rebuilding their graphs.
  size_t steps_captured = 0, steps_replayed = 0;
};
RealizeStats& realize_stats();
int debug_level();
// Drops every cached program, lowering and realisation plan on all devices.
void clear_kernel_caches();
// Realisation plan cache (structure of the lazy graph -> recorded kernel
// launches and replacements). On by default.
void set_plan_cache_enabled(bool on);
void clear_plan_cache();
void plan_cache_stats(uint64_t* hits, uint64_t* misses, uint64_t* entries);

}  // namespace fg
