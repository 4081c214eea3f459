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
// Direct dispatch into the context's own HSA queue (AQL packets written by
// the host), for replay loops whose launch cost on the host matters. Between
// fg_hip_aql_begin and fg_hip_aql_end, fg_hip_aql_launch queues a kernel
// there: it runs after everything queued before it on the queue and on the
// context's stream (the stream is synchronised before the first packet),
// and every stream operation issued meanwhile first waits for the queue to
// drain. With signal_slot >= 0 the packet completes read-back slot
// `signal_slot` (fg_hip_read_queued then marks the slot as pending on it).
// A kernel whose argument segment holds more than its explicit arguments
// (hidden arguments), or more than fits a packet's argument slot, returns
// FG_AQL_UNSUPPORTED with nothing queued; it then takes fg_hip_launch.
#define FG_AQL_UNSUPPORTED 100
int fg_hip_aql_begin(fg_ctx* c);
int fg_hip_aql_end(fg_ctx* c);
int fg_hip_aql_active(const fg_ctx* c);
int fg_hip_aql_launch(fg_ctx* c, fg_prog* p, const fg_arg* args, int nargs, const unsigned grid[3],
                      const unsigned block[3], unsigned lds, int signal_slot);
// Per-device set-up of the kernel entry points, run by fg_hip_init with the
// device current.
int fg_hip_kernel_device_setup(int ordinal);
}
