// vs_common.h - device helpers shared by the sampling and verify kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#include "../../include/volundr_sampling.h"

// Exact IEEE fp32 semantics for the arithmetic that has to match NumPy bit for bit: no contraction of a*b+c
// into an FMA anywhere in these sources (the build also passes -ffp-contract=off).
#pragma clang fp contract(off)

// Phase timestamps for development builds (-DVS_TRACE): workgroup 0-thread writes the 100 MHz wall clock into
// trace[blockIdx.x * 32 + id]. Compiled out of the shipped library.
#ifdef VS_TRACE
// Phase stamps go to LDS (a global store per stamp would make the stamping wave wait on store completion at
// every vmcnt wait) and are written out once at the end of the workgroup.
__shared__ unsigned long long vs_tr_lds[64];
#define VS_TR_DECL(A)                               \
  if (threadIdx.x < 64) vs_tr_lds[threadIdx.x] = 0; \
  __syncthreads()
#define VS_TRX(id)                                            \
  do {                                                        \
    if (threadIdx.x == 0) vs_tr_lds[id] = wall_clock64();     \
  } while (0)
#define VS_TR(A, id)                                                 \
  do {                                                               \
    if ((A).trace && threadIdx.x == 0) vs_tr_lds[id] = wall_clock64(); \
  } while (0)
#define VS_TRV(A, id, val)                                  \
  do {                                                      \
    if ((A).trace && threadIdx.x == 0) vs_tr_lds[id] = (val); \
  } while (0)
#define VS_TRC(A, id)                                           \
  do {                                                          \
    if ((A).trace && threadIdx.x == 0) vs_tr_lds[id] = clock64(); \
  } while (0)
#define VS_TR_FLUSH(A)                                                                             \
  do {                                                                                             \
    if ((A).trace && threadIdx.x == 0)                                                             \
      for (int i_ = 0; i_ < 64; ++i_) (A).trace[(size_t)blockIdx.x * 64 + i_] = vs_tr_lds[i_];     \
  } while (0)
#else
#define VS_TRX(id) \
  do {             \
  } while (0)
#define VS_TR_DECL(A) \
  do {                \
  } while (0)
#define VS_TRV(A, id, val) \
  do {                     \
  } while (0)
#define VS_TR_FLUSH(A) \
  do {                 \
  } while (0)
#define VS_TRC(A, id) \
  do {                \
  } while (0)
#define VS_TR(A, id) \
  do {               \
  } while (0)
#endif

namespace vs {

typedef unsigned long long u64;

constexpr int WAVE = 64;

// ---------------------------------------------------------------------------------------------------------------
// Order-preserving keys.
//   ord32(x): uint32 whose unsigned order equals the float order of x; -0 and +0 map to the same key (NumPy compares
//             them equal, so np.argmax and lexsort treat them as ties).
//   key64(x, i) = ord32(x) << 32 | (0xFFFFFFFF - i): descending key order == (x descending, index ascending), the
//             order of `np.lexsort((idx, -x[idx]))` (volundr-mlx/sampler.py:140). Keys are unique per row.
//   amkey(x, i): same with NaN ranked above +inf, so the maximum key is np.argmax's answer (first NaN, else first
//             maximum).
// Real values never produce key 0, which therefore means "none".
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ord32(float f) {
  uint32_t b = __float_as_uint(f);
  if (f == 0.0f) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float inv_ord32(uint32_t k) {
  return (k & 0x80000000u) ? __uint_as_float(k & 0x7FFFFFFFu) : __uint_as_float(~k);
}
__device__ __forceinline__ u64 key64(float x, uint32_t idx) {
  return ((u64)ord32(x) << 32) | (u64)(0xFFFFFFFFu - idx);
}
// xorshift64* of Sampler.uniform (volundr-mlx/sampler.py:67-73): one state step, and the uniform of a stepped state
// (the top 53 bits of the multiplied state over 2^53).
__host__ __device__ __forceinline__ u64 xorshift64s_step(u64 r) {
  r ^= r >> 12;
  r ^= r << 25;
  r ^= r >> 27;
  return r;
}
__host__ __device__ __forceinline__ double xorshift64s_uniform(u64 r) {
  return (double)((r * 0x2545F4914F6CDD1DULL) >> 11) / 9007199254740992.0;
}

__device__ __forceinline__ u64 amkey64(float x, uint32_t idx) {
  uint32_t o = (x != x) ? 0xFFFFFFFFu : ord32(x);
  return ((u64)o << 32) | (u64)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ uint32_t key_index(u64 k) { return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFull); }
__device__ __forceinline__ float key_value(u64 k) { return inv_ord32((uint32_t)(k >> 32)); }
__device__ __forceinline__ bool am_is_nan(u64 k) { return (uint32_t)(k >> 32) == 0xFFFFFFFFu; }

__device__ __forceinline__ bool is_finite(float x) { return (__float_as_uint(x) & 0x7F800000u) != 0x7F800000u; }

// bf16 / f16 widening (exact).
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

// ---------------------------------------------------------------------------------------------------------------
// Wave64 cross-lane primitives on DPP row moves and the gfx950 permlane swaps: these stay in the VALU (a few cycles
// each), unlike ds_bpermute (__shfl), whose ~90-cycle latency dominated every dependent reduction chain.
//   lane_xor<J>(v): the value of lane (lane ^ J), J in {1,2,4,8,16,32}
//   wave_max/min/sum(v): butterfly all-reduce (every lane gets the result)
//   wave_scan(v): inclusive prefix sum (row_shr 1,2,4,8 then row_bcast 15/31)
//   lane_bcast(v, L): the value of lane L (L uniform) via readlane
// 64-bit values move as two 32-bit halves.
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return threadIdx.x & (WAVE - 1); }

// v_max3_f32 / v_min3_f32 (a quiet NaN operand is passed over: callers test for NaNs apart), without the
// canonicalising operations the compiler adds around fmaxf / fminf; v_max3_u32; a packed 16-bit maximum.
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float min3f(float a, float b, float c) {
  float r;
  asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ uint32_t max3u(uint32_t a, uint32_t b, uint32_t c) {
  const uint32_t m = a > b ? a : b;
  return m > c ? m : c;
}
__device__ __forceinline__ uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}

template <int CTRL, int ROWM = 0xF, int BANKM = 0xF>
__device__ __forceinline__ uint32_t dpp32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWM, BANKM, false);
}

template <int J>
__device__ __forceinline__ uint32_t xor32(uint32_t u) {
  if constexpr (J == 1) {
    return dpp32<0xB1>(u, u);  // quad_perm [1,0,3,2]
  } else if constexpr (J == 2) {
    return dpp32<0x4E>(u, u);  // quad_perm [2,3,0,1]
  } else if constexpr (J == 4 || J == 8) {
    const uint32_t up = dpp32<0x100 + J>(u, u);   // row_shl:J -> lane + J
    const uint32_t dn = dpp32<0x110 + J>(u, u);   // row_shr:J -> lane - J
    return (lane_id() & J) ? dn : up;
  } else if constexpr (J == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return (lane_id() & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
  } else {
    static_assert(J == 32, "lane_xor: J in {1,2,4,8,16,32}");
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return (lane_id() & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
  }
}

template <typename T, typename F>
__device__ __forceinline__ T lanemove(T v, F f) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lane values");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, f(__builtin_bit_cast(uint32_t, v)));
  } else {
    const u64 u = __builtin_bit_cast(u64, v);
    const uint32_t lo = f((uint32_t)u), hi = f((uint32_t)(u >> 32));
    return __builtin_bit_cast(T, ((u64)hi << 32) | lo);
  }
}

template <int J, typename T>
__device__ __forceinline__ T lane_xor(T v) {
  return lanemove(v, [](uint32_t u) { return xor32<J>(u); });
}

// lane_xor with a run-time J (a power of two below 64)
template <typename T>
__device__ __forceinline__ T lane_xor_rt(T v, int j) {
  switch (j) {
    case 1: return lane_xor<1>(v);
    case 2: return lane_xor<2>(v);
    case 4: return lane_xor<4>(v);
    case 8: return lane_xor<8>(v);
    case 16: return lane_xor<16>(v);
    default: return lane_xor<32>(v);
  }
}

template <typename T>
__device__ __forceinline__ T lane_bcast(T v, int L) {
  const int l = __builtin_amdgcn_readfirstlane(L);
  return lanemove(v, [l](uint32_t u) { return (uint32_t)__builtin_amdgcn_readlane((int)u, l); });
}

template <typename T, typename Op>
__device__ __forceinline__ T wave_allreduce(T v, Op op) {
  v = op(v, lane_xor<1>(v));
  v = op(v, lane_xor<2>(v));
  v = op(v, lanemove(v, [](uint32_t u) { return dpp32<0x141>(u, u); }));  // row_half_mirror
  v = op(v, lanemove(v, [](uint32_t u) { return dpp32<0x140>(u, u); }));  // row_mirror
  v = op(v, lane_xor<16>(v));
  v = op(v, lane_xor<32>(v));
  return v;
}
template <typename T>
__device__ __forceinline__ T wave_max(T v) {
  return wave_allreduce(v, [](T a, T b) { return a > b ? a : b; });
}
template <typename T>
__device__ __forceinline__ T wave_min(T v) {
  return wave_allreduce(v, [](T a, T b) { return a < b ? a : b; });
}
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  return wave_allreduce(v, [](T a, T b) { return a + b; });
}
// inclusive scan inside a wave (lanes with no source in a step add the identity 0)
template <typename T>
__device__ __forceinline__ T wave_scan(T v) {
  v += lanemove(v, [](uint32_t u) { return dpp32<0x111>(0u, u); });  // row_shr:1
  v += lanemove(v, [](uint32_t u) { return dpp32<0x112>(0u, u); });  // row_shr:2
  v += lanemove(v, [](uint32_t u) { return dpp32<0x114>(0u, u); });  // row_shr:4
  v += lanemove(v, [](uint32_t u) { return dpp32<0x118>(0u, u); });  // row_shr:8
  v += lanemove(v, [](uint32_t u) { return dpp32<0x142, 0xA>(0u, u); });  // row_bcast:15 -> rows 1, 3
  v += lanemove(v, [](uint32_t u) { return dpp32<0x143, 0xC>(0u, u); });  // row_bcast:31 -> rows 2, 3
  return v;
}

// Wave-aggregated append: lanes with `pred` get consecutive slots of *counter (an LDS counter), with one atomic per
// wave instead of one per lane (same-address atomics serialise). Works on LDS or device counters. Returns the
// slot, or -1.
template <typename C>
__device__ __forceinline__ int wave_append(bool pred, C* counter) {
  const unsigned long long m = __ballot(pred);
  if (!m) return -1;
  const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
  const int leader = __ffsll((long long)m) - 1;
  int base = 0;
  if (lane_id() == leader) base = (int)atomicAdd(counter, (C)__popcll(m));
  base = __builtin_amdgcn_readlane(base, leader);
  return pred ? base + below : -1;
}

// Reserve n consecutive slots of *counter for this lane (one atomic per wave): returns the lane's first slot.
template <typename C>
__device__ __forceinline__ int wave_alloc(int n, C* counter) {
  const int incl = wave_scan(n);
  const int total = __builtin_amdgcn_readlane(incl, WAVE - 1);
  int base = 0;
  if (lane_id() == 0 && total) base = (int)atomicAdd(counter, (C)total);
  base = __builtin_amdgcn_readlane(base, 0);
  return base + incl - n;
}

// Block-wide reductions for a block of NT threads; `red` is LDS scratch of >= NT/64 elements of T.
// Every thread receives the result.
template <int NT, typename T>
__device__ __forceinline__ T block_max(T v, T* red) {
  v = wave_max(v);
  const int w = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int i = 1; i < NT / WAVE; ++i) r = red[i] > r ? red[i] : r;
  return r;
}
template <int NT, typename T>
__device__ __forceinline__ T block_min(T v, T* red) {
  v = wave_min(v);
  const int w = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int i = 1; i < NT / WAVE; ++i) r = red[i] < r ? red[i] : r;
  return r;
}
// Sum in a fixed order (wave tree, then waves 0..NW-1): deterministic for a given launch shape.
template <int NT, typename T>
__device__ __forceinline__ T block_sum(T v, T* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int i = 1; i < NT / WAVE; ++i) r += red[i];
  return r;
}
// Inclusive block scan; also returns the block total through *total.
template <int NT, typename T>
__device__ __forceinline__ T block_scan(T v, T* red, T* total) {
  T s = wave_scan(v);
  const int w = threadIdx.x / WAVE, lane = threadIdx.x & (WAVE - 1);
  __syncthreads();
  if (lane == WAVE - 1) red[w] = s;
  __syncthreads();
  T off = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NT / WAVE; ++i) {
    if (i < w) off += red[i];
    tot += red[i];
  }
  *total = tot;
  return s + off;
}

// ---------------------------------------------------------------------------------------------------------------
// Cross-workgroup data exchange.
// gfx950 keeps one L2 per XCD; an agent-scope release/acquire compiles to a write-back / invalidate of that whole
// L2 (several microseconds each). This code never needs either: every datum that another workgroup reads is written
// and read with agent-scope relaxed atomics (stores and loads that go to the device-coherent level, `sc1`), and the
// order "data, then counter" is enforced in hardware by waiting for the wave's outstanding memory operations to be
// acknowledged before the counter RMW (publish_wait). Readers observe the counter first and only then issue their
// (coherent) data loads.
// ---------------------------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void st_dev(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_dev(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Exchange inside one XCD. When every workgroup that reads a datum runs on the XCD of the workgroup that wrote it,
// the XCD's L2 is a coherence point they share: the writer's workgroup-scope store (`sc0`) passes this CU's
// write-through L1 and is acknowledged by that L2, and a non-temporal load (`nt`) skips the reader's L1 and reads
// that L2, about half the latency of a device-coherent round trip (~0.5 us against ~1 us per hop, measured on
// MI355X; a plain or workgroup-scope load can hit a stale line of the reader's own L1). Only data that was written
// by such stores in the same launch may be read this way; counters and sums built with atomics (which act at the
// device-coherent level) keep ld_dev. XL = false selects the device-coherent forms.
template <bool XL, typename T>
__device__ __forceinline__ void st_row(T* p, T v) {
  if constexpr (XL)
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  else
    st_dev(p, v);
}
template <bool XL, typename T>
__device__ __forceinline__ T ld_row(const T* p) {
  if constexpr (XL)
    return __builtin_nontemporal_load(p);
  else
    return ld_dev(p);
}
__device__ __forceinline__ uint32_t ld_relaxed(const uint32_t* p) { return ld_dev(p); }
__device__ __forceinline__ u64 ld_relaxed64(const u64* p) { return ld_dev(p); }
__device__ __forceinline__ double ld_relaxed_f64(const double* p) { return ld_dev(p); }
// Wait until every memory operation this wave issued has completed (stores acknowledged by the coherent level).
// The s_waitcnt orders the hardware; the two signal fences order the compiler: no load or store may be moved
// across the wait in either direction (a signal fence emits no instruction). Without them nothing in the
// language would stop the compiler from sinking a data store below the wait, and hence below the counter RMW
// that follows it, since the wait builtin is not a memory operation.
__device__ __forceinline__ void publish_wait() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ uint32_t ctr_add(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide arrival: all waves' prior device-coherent writes complete, then thread 0 adds `add` to *ctr. Returns
// the old counter value in every thread (through *lds).
__device__ __forceinline__ uint32_t block_arrive(uint32_t* ctr, uint32_t* lds, uint32_t add = 1u) {
  publish_wait();
  __syncthreads();
  if (threadIdx.x == 0) *lds = ctr_add(ctr, add);
  __syncthreads();
  const uint32_t old = *lds;
  __syncthreads();
  return old;
}

// Wait until *ctr >= target after arriving. Thread 0 spins; the whole block calls it. The wait is bounded twice:
// by `ticks` of the constant 100 MHz real-time counter (s_memrealtime, 10 ns per tick; the normal bound) and by
// `limit` polls (a testing hook: a tiny limit forces the timeout path). Returns false (for every thread) when a
// bound was hit, so a wave can never wait forever.
__device__ __forceinline__ bool row_barrier(uint32_t* ctr, uint32_t target, uint32_t limit, uint64_t ticks,
                                            int* flag_lds) {
  publish_wait();
  __syncthreads();
  if (threadIdx.x == 0) {
    ctr_add(ctr, 1u);
    uint32_t polls = 0;
    int ok = 1;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (ld_dev(ctr) < target) {  // at most `limit` polls
      if (++polls >= limit || __builtin_amdgcn_s_memrealtime() - t0 > ticks) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    *flag_lds = ok;
  }
  __syncthreads();
  return *flag_lds != 0;
}

// Row barrier inside one XCD (the XL exchange of st_row / ld_row): workgroup g stores `want` in its own flag word
// (flags[g]), then one wave polls the G words with non-temporal loads until each holds `want` or a later value of the
// same call. A flag is ((u64)epoch << 32) | barrier number, where epoch counts the calls of the row (so a word left
// by an earlier call, still in memory or in a stale L2 line, never passes) and barrier numbers grow within a call (a
// workgroup that has passed may already have stored the next one). Every prior store and atomic of the
// workgroup is acknowledged before its flag is stored (publish_wait). Bounded like row_barrier; `unreachable`
// (a testing flag) makes every wait run to its bound.
__device__ __forceinline__ bool flag_barrier(u64* flags, int g, int G, u64 want, bool unreachable, uint32_t limit,
                                             uint64_t ticks, int* flag_lds) {
  publish_wait();
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(&flags[g], want, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (threadIdx.x < WAVE) {
    const int L = threadIdx.x;
    const uint32_t ep = (uint32_t)(want >> 32);
    uint32_t polls = 0;
    int ok = 1;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
      asm volatile("" ::: "memory");  // each trip loads the flags again
      const u64 f = L < G ? __builtin_nontemporal_load(&flags[L]) : want;
      const bool here = (uint32_t)(f >> 32) == ep && (uint32_t)f >= (uint32_t)want;
      if (__all(here) && !unreachable) break;
      if (++polls >= limit || __builtin_amdgcn_s_memrealtime() - t0 > ticks) {  // at most `limit` polls
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (L == 0) *flag_lds = ok;
  }
  __syncthreads();
  return *flag_lds != 0;
}

}  // namespace vs
