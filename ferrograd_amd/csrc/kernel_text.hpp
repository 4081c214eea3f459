// Text form of one rangeified kernel: what a caller outside this library
// (a Rust `Renderer`, tests) hands to fg_hip_render across the C-ABI.
//
// The reference renders a kernel from its UOp graph (codegen.rs:17-20;
// tensor.rs:845-852). The HIP lowering replaces optimize/expand/devectorize/
// linearize, so it takes the graph rangeify produces (rangeify.rs:42-206,
// after parameterize: schedule.rs:131-170). Format, one node per line in
// topological order (sources before users), node i being line i after the
// header:
//
//   fg-kernel 1
//   <Op> <dtype> <arg> [#<tag>] [<source line numbers>...]
//
//   Op     the uop.rs:26-339 variant name (Add, Range, ParamBuffer, ...)
//   dtype  f32 | i32 | bool | void, with xN for an N-lane vector (f32x4)
//   arg    -                 none
//          device:<hip|cpu>  int:<i64>  bool:<0|1>
//          float:<16 hex digits of the f64 bit pattern>
//          range:<axis>:<LOOP|GLOBAL|LOCAL|REDUCE|GROUP_REDUCE|UPCAST|UNROLL|THREAD>
//          param:<slot>:<numel>   scalar:<slot>   index:<tag>
//          reduce:<Op>:<a,b,...>  axes:<...>  shape:<...>  bounds:<...>  lanes:<...>
//          var:<name>:<min>:<max>
//   #tag   an optional node tag (a u64; the HIP schedule tags literal zeros
//          that stand for allocate()'s zero buffers)
//
// The last line is the kernel's Sink. Buffer args cannot cross: a kernel
// refers to memory through ParamBuffer slots only.
#pragma once

#include <string>

#include "ir.hpp"

namespace fg {

std::string kernel_to_text(const UOp& sink);
// Parses the text back into the same (interned) nodes. Malformed input
// raises fg::Error naming the line.
UOp kernel_from_text(const std::string& text);

}  // namespace fg
