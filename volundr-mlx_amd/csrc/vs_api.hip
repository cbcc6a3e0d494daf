// vs_api.hip - library-wide C entry points: error text, workspace zeroing, version; cached device properties.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "../../include/volundr_sampling.h"
#include "vs_host.h"

namespace vs {

static thread_local std::string g_err;
unsigned long long* g_trace = nullptr;
unsigned g_spin_limit = 0;
thread_local int g_cooperative = 0;
unsigned g_debug = 0;

void set_error(const std::string& msg) { g_err = msg; }
int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}
int hip_fail(hipError_t e, const char* what) {
  g_err = std::string(what) + ": " + hipGetErrorString(e);
  return VS_EHIP;
}

static std::mutex g_mu;
static DevInfo g_dev[64];
static bool g_have[64];

const DevInfo* dev_info() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return nullptr;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_have[d]) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, d) != hipSuccess) return nullptr;
    g_dev[d].device = d;
    g_dev[d].cus = p.multiProcessorCount;
    g_dev[d].lds_per_block = p.sharedMemPerBlock;
    g_dev[d].coop = p.cooperativeLaunch;
    g_have[d] = true;
  }
  return &g_dev[d];
}

}  // namespace vs

namespace {
// An empty kernel: the launch-floor measurement of vs_launch_floor (what a launch of a given shape costs with no
// work in it, back to back on one stream).
__global__ void vs_empty_kernel(int) {}

// Streaming read: workgroup b reads its contiguous share of n16 16-byte words, eight loads per lane in flight, and
// folds them into one word (written only on an impossible value, so the loads stay live). The rate a kernel whose
// bytes stream in once, such as the lm_head weight of vs_lmhead_verify_greedy, can reach on the device.
__global__ __launch_bounds__(512) void vs_stream_read_kernel(const uint4* __restrict__ p, size_t n16, uint32_t* out) {
  const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const size_t b0 = (size_t)blockIdx.x * per, b1 = b0 + per < n16 ? b0 + per : n16;
  uint32_t acc = 0;
  for (size_t i = b0 + threadIdx.x; i < b1; i += (size_t)512 * 8) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const size_t j = i + (size_t)u * 512;
      v[u] = p[j < b1 ? j : i];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) out[blockIdx.x] = acc;
}
// The XCD (XCC id hardware register) each workgroup runs on: the placement check of vs_xcd_ids.
__global__ void vs_xcd_ids_kernel(uint32_t* out) {
  uint32_t id;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(id));
  if (threadIdx.x == 0) out[blockIdx.x] = id & 0xFu;
}
}  // namespace

extern "C" {

int vs_xcd_ids(uint32_t* out, int blocks, int threads, vs_stream_t stream) {
  if (!out || blocks < 1 || threads < 1 || threads > 1024) return vs::fail(VS_EINVAL, "vs_xcd_ids: bad arguments");
  hipLaunchKernelGGL(vs_xcd_ids_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)stream, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return vs::hip_fail(e, "vs_xcd_ids: launch");
  return VS_OK;
}

int vs_stream_read(const void* p, size_t bytes, int blocks, uint32_t* out, vs_stream_t stream) {
  if (!p || !out || blocks < 1 || bytes % 16 != 0 || (uintptr_t)p % 16 != 0)
    return vs::fail(VS_EINVAL, "vs_stream_read: need a 16-byte aligned buffer of whole 16-byte words and blocks >= 1");
  hipLaunchKernelGGL(vs_stream_read_kernel, dim3(blocks), dim3(512), 0, (hipStream_t)stream, (const uint4*)p,
                     bytes / 16, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return vs::hip_fail(e, "vs_stream_read: launch");
  return VS_OK;
}

int vs_launch_floor(int blocks, int threads, size_t lds_bytes, int reps, vs_stream_t stream) {
  if (blocks < 1 || threads < 1 || threads > 1024 || reps < 1) return vs::fail(VS_EINVAL, "vs_launch_floor: bad shape");
  for (int i = 0; i < reps; ++i)
    hipLaunchKernelGGL(vs_empty_kernel, dim3(blocks), dim3(threads), lds_bytes, (hipStream_t)stream, 0);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return vs::hip_fail(e, "vs_launch_floor: launch");
  return VS_OK;
}

const char* vs_last_error(void) { return vs::g_err.c_str(); }

int vs_version(void) { return 10; }

int vs_set_spin_limit(unsigned polls) {
  vs::g_spin_limit = polls;
  return VS_OK;
}

int vs_set_debug(unsigned flags) {
  vs::g_debug = flags;
  return VS_OK;
}

int vs_set_cooperative(int on) {
  const int prev = vs::g_cooperative;
  vs::g_cooperative = on ? 1 : 0;
  return prev;
}

#ifdef VS_TRACE
void vs_debug_set_trace(void* p) { vs::g_trace = (unsigned long long*)p; }
#endif

int vs_workspace_init(void* ws, size_t bytes, vs_stream_t stream) {
  if (!ws && bytes) return vs::fail(VS_EINVAL, "vs_workspace_init: null workspace");
  if (!bytes) return VS_OK;
  hipError_t e = hipMemsetAsync(ws, 0, bytes, (hipStream_t)stream);
  if (e != hipSuccess) return vs::hip_fail(e, "vs_workspace_init: hipMemsetAsync");
  return VS_OK;
}

}  // extern "C"
