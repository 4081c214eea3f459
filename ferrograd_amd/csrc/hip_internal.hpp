// Internal hooks between the HIP runtime (hip_runtime.cpp) and the kernel
// entry points (hip_kernel.cpp). Not part of the public C-ABI.
#pragma once

#include "../../include/ferrograd_hip.h"

extern "C" {
// Sets fg_hip_last_error() and returns `code`.
int fg_hip_set_error(int code, const char* msg);
// The device ordinal a context was created on.
int fg_hip_context_device(const fg_ctx* c);
// fg_hip_launch without launch profiling: one hipModuleLaunchKernel, nothing
// allocated or recorded.
int fg_hip_launch_direct(fg_ctx* c, fg_prog* p, const fg_arg* args, int nargs, const unsigned grid[3],
                         const unsigned block[3], unsigned lds);
// Workgroups of `block` threads (plus `lds` bytes of dynamic LDS) of program
// `p` that the context's device holds at once: per-CU occupancy times CUs.
int fg_hip_program_resident(fg_ctx* c, fg_prog* p, unsigned block, unsigned lds, long* out);
// Per-device set-up of the kernel entry points, run by fg_hip_init with the
// device current.
int fg_hip_kernel_device_setup(int ordinal);
}
