// Scheduling and rangeify (src/schedule.rs, src/schedule/rangeify.rs,
// src/schedule/indexing.rs).
#pragma once

#include "device.hpp"
#include "ir.hpp"

namespace fg {

// schedule.rs:32-41
struct ScheduleItem {
  UOp sink;                        // Sink(Store(Param(0), expr)) or Sink(Store(dest, expr))
  std::vector<KernelArg> inputs;   // runtime inputs in slot order, excluding output slot 0
  Buffer output_buffer;            // null for in-place stores
  Shape out_shape;
};

// schedule.rs:45-50
struct SchedulePlan {
  std::vector<ScheduleItem> items;
  UOpMap<UOp> replacements;
};

struct ScheduleOptions {
  // Value-preserving fusion used by the HIP device: an elementwise node whose
  // consumers all reconverge on one elementwise node is computed inside that
  // node's kernel instead of being materialised (its loads are shared through
  // interning, so nothing is recomputed), and buffers still holding the zeros
  // `allocate` produced become a literal 0.
  bool fuse = false;
  // Nodes that live tensors point at. The reference materialises a node by
  // its structure alone and then repoints every live tensor at that node to
  // the buffer (tensor.rs:222-252), so the fusions above leave held nodes to
  // the reference's rules: a held tensor is realised exactly when the
  // reference's would be.
  const PtrIndexMap* held = nullptr;
};

SchedulePlan schedule_many(const std::vector<UOp>& exprs, const ScheduleOptions& opt = {});
std::vector<ScheduleItem> schedule(const UOp& expr, const ScheduleOptions& opt = {});
ScheduleItem parameterize_store(const UOp& store, const ScheduleOptions& opt = {});

// rangeify.rs:204-206
UOp rangeify(const UOp& sink);

// Tag carried by literal zeros that replaced a zero-filled buffer. The
// symbolic folds leave such literals alone so the arithmetic stays identical
// to loading the zeros.
constexpr uint64_t kZeroBufferTag = 0x5a45524fULL;  // "ZERO"
// Tags the Contiguous that Tensor::matmul makes of its transposed right operand
// (tensor.rs:771-777). No tensor a caller holds points at it, so the HIP
// schedule may read its source in place when the copy would not change the
// layout; a contiguous() the caller asked for is materialised as in the
// reference.
constexpr uint64_t kMatmulCopyTag = 0x4d4d4350ULL;  // "MMCP"

}  // namespace fg
