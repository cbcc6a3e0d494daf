// vs_host.h - host-side helpers shared by the entry points (error text, device properties).
#pragma once
#include <hip/hip_runtime.h>

#include <string>

namespace vs {

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

struct DevInfo {
  int device;
  int cus;
  size_t lds_per_block;
  int coop;
};
// Properties of the current device (cached per device).
const DevInfo* dev_info();

// Polls of an inter-workgroup wait before it gives up (0: the default). Set by vs_set_spin_limit.
extern unsigned g_spin_limit;
// Non-zero: the calling thread launches sampling kernels cooperatively (set by vs_set_cooperative, per thread).
extern thread_local int g_cooperative;
// VS_DEBUG_* testing flags (set by vs_set_debug).
extern unsigned g_debug;

// Phase-timestamp buffer of development builds (VS_TRACE); always null in the shipped library.
extern unsigned long long* g_trace;

}  // namespace vs
