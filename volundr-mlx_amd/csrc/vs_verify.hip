// vs_verify.hip - greedy speculative verify for gfx950: first-max argmax over the valid vocabulary, the accept
// prefix, and the chosen-token logprob, in one pass over [B, T, V] logits.
//
// Reference: tok = argmax(logits[..., :vv]) (volundr-mlx/spec/specdec.py:326, scheduler.py:462);
//            nacc = sum(cumprod(inp[:, 1:] == tok[:, :-1])) (specdec.py:327, scheduler.py:463);
//            logprob = x[tok] - logsumexp(x[:vv]) (log-softmax form of spec/check_verify.py:27-30; build-defined).
//
// Each (b, t) row is split into G chunks, one 256-thread workgroup each, so B*T = 17..68 rows still fill the
// 256 CUs. A workgroup reads its chunk once with 16-byte loads into VGPRs, reduces (first-max key, finite max) with
// wave64 reductions, then sum(exp(x - max)). No atomics: every word a workgroup publishes carries a tag, an epoch
// + 1 read from the workspace; the row's last workgroup (g = G - 1) reloads the row's partials (one per wave, or
// one per workgroup) until each shows the tag and merges them, and the finisher of a request's last row reloads the
// request's other tokens the same way and computes the accept length. Each slot's epoch is advanced only by its reader, after it has read the slot
// in the call (its writers read the epoch before they store), and a slot is only ever written for one row (partial
// slot (row, s), token slot row), so no word a previous call or graph replay left can pass for the current one's,
// whatever shapes the calls had. A launch holds only as many rows as the device keeps resident at once, so every
// workgroup a finisher waits for is running or done.
#include "vs_common.h"
#include "vs_host.h"

#pragma clang fp contract(off)

namespace vs {

constexpr int VNT = 256;
constexpr int VNW = VNT / WAVE;
constexpr int VNV_MAX = 64;  // 16-byte loads per lane (streamed, not held)
constexpr int VNF = 8;       // 16-byte loads per lane held in VGPRs by the fast path
constexpr int VGMAX = 64;
constexpr int VRMAX = 8192;  // rows (B*T) per call: the slots of the row-token area

// A workgroup's partial slot: five 64-bit words, each the tag (high half) over 32 bits of payload: the first-max
// key (high, low), the finite maximum's bits, sum-exp's float64 bits (high, low); word 7 is the slot's epoch, and
// tag = epoch + 1. A 64-bit store is single-copy atomic, so a word that shows the tag holds this call's payload.
struct VPart {
  u64 w[8];
};
constexpr int VEPW = 7;  // the epoch word
static_assert(sizeof(VPart) == 64, "VPart layout");
constexpr int VPW = 5;  // words in use
// Wall-clock bound (100 MHz ticks, 100 ms) on a finisher's wait: a launch's workgroups are all resident on an
// otherwise idle device, so it is reached only if other work held CUs for that long; the row then reports token -1
// (which no draft matches).
constexpr uint64_t VWAIT_TICKS = 10000000;

struct VerifyArgs {
  const void* logits;
  int64_t ld;
  int B, T, V, vv;
  int G, CH, NV, vec_ok;
  const int32_t* drafts;
  int32_t* out_argmax;
  int32_t* out_accept;
  float* out_lp;
  int row0;  // first row of this launch
  char* ws;  // [VRMAX] token slots (tag | token, epoch) | [R][VGMAX] VPart
  unsigned long long* trace;  // development builds only (VS_TRACE); null otherwise
};

template <int DT>
struct VTraits;
template <>
struct VTraits<VS_F32> {
  static constexpr int VEC = 4;
  static constexpr uint32_t NEG_INF_WORD = 0xFF800000u;
  __device__ static uint4 gather(const void* p, int base, int hi) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = base + q < hi ? ((const uint32_t*)p)[base + q] : 0xFF800000u;
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ static float get(const uint4& r, int q) { return ((const float*)&r)[q]; }
  __device__ static float one(const void* p, int64_t i) { return ((const float*)p)[i]; }
  // best = max(best, the four values); mag = max(mag, their magnitude bits); a NaN has magnitude > NAN_MAG
  static constexpr uint32_t NAN_MAG = 0x7F800000u;
  __device__ static void max_mag(const uint4& r, float& best, uint32_t& mag) {
    best = max3f(best, __uint_as_float(r.x), __uint_as_float(r.y));
    best = max3f(best, __uint_as_float(r.z), __uint_as_float(r.w));
    mag = max3u(mag, r.x & 0x7FFFFFFFu, r.y & 0x7FFFFFFFu);
    mag = max3u(mag, r.z & 0x7FFFFFFFu, r.w & 0x7FFFFFFFu);
  }
  __device__ static bool has_nan(uint32_t mag) { return mag > NAN_MAG; }
};
template <>
struct VTraits<VS_BF16> {
  static constexpr int VEC = 8;
  static constexpr uint32_t NEG_INF_WORD = 0xFF80FF80u;
  __device__ static uint4 gather(const void* p, int base, int hi) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = base + 2 * q < hi ? ((const uint16_t*)p)[base + 2 * q] : 0xFF80u;
      const uint32_t b = base + 2 * q + 1 < hi ? ((const uint16_t*)p)[base + 2 * q + 1] : 0xFF80u;
      w[q] = a | (b << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ static float get(const uint4& r, int q) {
    const uint32_t w = q < 2 ? r.x : q < 4 ? r.y : q < 6 ? r.z : r.w;  // q is a constant after unrolling
    return __uint_as_float((q & 1) ? (w & 0xFFFF0000u) : (w << 16));
  }
  __device__ static float one(const void* p, int64_t i) { return bf16_to_f32(((const uint16_t*)p)[i]); }
  // as for float32, with the two 16-bit magnitudes of a word kept apart (one packed maximum per word)
  __device__ static void max_mag(const uint4& r, float& best, uint32_t& mag) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      best = max3f(best, __uint_as_float(w[i] << 16), __uint_as_float(w[i] & 0xFFFF0000u));
      mag = pk_max_u16(mag, w[i] & 0x7FFF7FFFu);
    }
  }
  __device__ static bool has_nan(uint32_t mag) { return (mag & 0xFFFFu) > 0x7F80u || (mag >> 16) > 0x7F80u; }
};
template <>
struct VTraits<VS_F16> {
  static constexpr int VEC = 8;
  static constexpr uint32_t NEG_INF_WORD = 0xFC00FC00u;
  __device__ static uint4 gather(const void* p, int base, int hi) {
    uint32_t w[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = base + 2 * q < hi ? ((const uint16_t*)p)[base + 2 * q] : 0xFC00u;
      const uint32_t b = base + 2 * q + 1 < hi ? ((const uint16_t*)p)[base + 2 * q + 1] : 0xFC00u;
      w[q] = a | (b << 16);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
  __device__ static float get(const uint4& r, int q) {
    const uint32_t w = q < 2 ? r.x : q < 4 ? r.y : q < 6 ? r.z : r.w;  // q is a constant after unrolling
    return f16_to_f32((uint16_t)((q & 1) ? (w >> 16) : (w & 0xFFFFu)));
  }
  __device__ static float one(const void* p, int64_t i) { return f16_to_f32(((const uint16_t*)p)[i]); }
  __device__ static void max_mag(const uint4& r, float& best, uint32_t& mag) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      best = max3f(best, get(r, 2 * i), get(r, 2 * i + 1));
      mag = pk_max_u16(mag, w[i] & 0x7FFF7FFFu);
    }
  }
  __device__ static bool has_nan(uint32_t mag) { return (mag & 0xFFFFu) > 0x7C00u || (mag >> 16) > 0x7C00u; }
};

template <int DT>
__global__ __launch_bounds__(VNT) void vs_verify_kernel(VerifyArgs A) {
  typedef VTraits<DT> TR;
  constexpr int VEC = TR::VEC;
  constexpr int U = 4;  // 16-byte loads in flight per lane
  __shared__ u64 red64[VNW];
  __shared__ float redf[VNW];
  __shared__ double redd[VNW];
  const int t = threadIdx.x;
  const int G = A.G;
  const int nb = gridDim.x, b = blockIdx.x;
  const int l = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
  const int row = A.row0 + l / G, g = l % G;
  u64* rowtok = (u64*)A.ws;  // token slot r: words 2r (tag | token) and 2r + 1 (epoch)
  VPart* parts = (VPart*)(A.ws + 16 * VRMAX) + (size_t)row * VGMAX;  // this row's partial slots (written for it only)
  // Epochs: each slot's epoch is advanced only by its reader, after it has read the slot in the call; its writer
  // reads it before it stores (so both use the same value), and the tag is epoch + 1 (never the 0 of a zeroed
  // workspace). Each workgroup reads its own partial slot's epoch, the row's finisher also its token slot's, and the
  // second wave of a request's last-row finisher the request's first 64 token slots'. They are loaded right after
  // the logits (issued after them, so that the waits for the logits do not wait for these); every epoch sits in its
  // own slot, so no address is read by many workgroups at once.
  const int req = row / A.T, tp = row - req * A.T;
  uint32_t ep = 0, tep = 0;
  u64 qep = 0;
  // Partial slots: one per wave when the row's waves fit one merging wave (G * VNW <= 64: no workgroup reduction),
  // else one per workgroup.
  const bool per_wave = G * VNW <= WAVE;
  const int nslots = per_wave ? G * VNW : G;
  VPart* myslot = parts + (per_wave ? g * VNW + t / WAVE : g);
  auto load_epochs = [&]() {
    ep = (uint32_t)ld_dev(&myslot->w[VEPW]);
    if (g == G - 1) {
      tep = (uint32_t)ld_dev(&rowtok[2 * (size_t)row + 1]);
      if (tp == A.T - 1 && t >= WAVE && t < 2 * WAVE && t - WAVE < A.T - 1)
        qep = ld_dev(&rowtok[2 * ((size_t)req * A.T + (t - WAVE)) + 1]);
    }
  };

  const int lo = g * A.CH;
  const int hi = min(A.vv, lo + A.CH);
  const char* rowp = (const char*)A.logits + (int64_t)row * A.ld * (DT == VS_F32 ? 4 : 2);
  VS_TR_DECL(A);
  VS_TR(A, 0);

  u64 am = 0;
  float m = -__builtin_inff();
  double se = 0.0;
  if (A.NV <= VNF) {
    // Fast path: the whole chunk fits in VGPRs (<= VNF 16-byte loads per lane, all issued at once). Pass 1: the
    // lane's first maximum (strict > in increasing index order), its finite maximum and its first NaN; pass 2:
    // sum(exp(x - m)) from the registers as exp2((x - m) * log2(e)) (one v_exp_f32 per element). Keys are built
    // once per lane: np.argmax's order (NaN first, then the value, then the lower index) is kept.
    uint4 rv[VNF];
#pragma unroll
    for (int u = 0; u < VNF; ++u) {
      int base = lo + (u * VNT + t) * VEC;
      base = (u < A.NV && base < hi) ? base : lo;  // clamped into the row: the values are masked below
      rv[u] = A.vec_ok ? *(const uint4*)(rowp + (int64_t)base * (DT == VS_F32 ? 4 : 2)) : make_uint4(0, 0, 0, 0);
    }
    load_epochs();
    // a vector that is not whole inside the chunk (the row's last, or any when unaligned) is assembled element by
    // element, -inf past the end, so both passes below read registers only
#pragma unroll
    for (int u = 0; u < VNF; ++u) {
      const int base = lo + (u * VNT + t) * VEC;
      if (u < A.NV && base < hi && !(A.vec_ok && base + VEC <= hi)) rv[u] = TR::gather(rowp, base, hi);
      // a vector wholly past the chunk reads as -inf (a select, not a branch)
      const bool past = base >= hi;
      rv[u].x = past ? TR::NEG_INF_WORD : rv[u].x;
      rv[u].y = past ? TR::NEG_INF_WORD : rv[u].y;
      rv[u].z = past ? TR::NEG_INF_WORD : rv[u].z;
      rv[u].w = past ? TR::NEG_INF_WORD : rv[u].w;
    }
#ifdef VS_TRACE
    __builtin_amdgcn_s_waitcnt(0);
    VS_TR(A, 5);
#endif
    // Every element past the chunk now reads -inf, and a lane's elements inside the chunk come first in its (u, q)
    // order, so no element needs a range test. A lane with no element inside the chunk contributes no key.
    // np.argmax ranks a NaN first, so the lane's maximum matters only when it holds none: the maximum comes from
    // three-input max instructions (two elements each; a quiet NaN operand is passed over) and the NaN flag from
    // the largest magnitude bits, then a backward sweep of equality selects leaves the first index holding the maximum
    // (with every element -inf, the first element, as np.argmax has it).
    const int base0 = lo + t * VEC;
    const bool any_in = base0 < hi;
    float best = -__builtin_inff();
    uint32_t mag = 0;
#pragma unroll
    for (int u = 0; u < VNF; ++u) {
      if (u >= A.NV) break;  // uniform: the work scales with the chunk, not with the register budget
      TR::max_mag(rv[u], best, mag);
    }
    const bool anynan = TR::has_nan(mag);
    int bi = base0;
#pragma unroll
    for (int u = VNF - 1; u >= 0; --u) {
      if (u >= A.NV) continue;
#pragma unroll
      for (int q = VEC - 1; q >= 0; --q) bi = TR::get(rv[u], q) == best ? base0 + u * VNT * VEC + q : bi;
    }
    // the finite maximum: the maximum itself unless it is +inf (then a sweep over the finite elements) or NaN
    if (is_finite(best)) {
      m = best;
    } else if (best > 0.0f) {
#pragma unroll
      for (int u = 0; u < VNF; ++u) {
        if (u >= A.NV) break;
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const float x = TR::get(rv[u], q);
          m = __builtin_fmaxf(m, is_finite(x) ? x : -__builtin_inff());
        }
      }
    }
    VS_TR(A, 6);
    int nani = -1;
    if (anynan) {
#pragma unroll
      for (int u = 0; u < VNF; ++u) {
        if (u >= A.NV) break;
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
          const float x = TR::get(rv[u], q);
          nani = ((x != x) & (nani < 0)) ? base0 + u * VNT * VEC + q : nani;
        }
      }
    }
    if (any_in && nani >= 0)
      am = amkey64(__builtin_nanf(""), (uint32_t)nani);
    else if (any_in)
      am = amkey64(best, (uint32_t)bi);
    // the raw registers are declared changed here, so the compiler re-widens them in pass 2 instead of keeping
    // every widened value of pass 1 live (VGPRs, hence occupancy)
#pragma unroll
    for (int u = 0; u < VNF; ++u) asm volatile("" : "+v"(rv[u].x), "+v"(rv[u].y), "+v"(rv[u].z), "+v"(rv[u].w));
    if (is_finite(m)) {
      const float L2E = 1.44269504088896340736f;
      float acc0 = 0.0f, acc1 = 0.0f;  // two chains of additions
      if (!anynan & is_finite(best)) {
        // no NaN and no +inf: a -inf element gives exp2(-inf) = 0 without a test
#pragma unroll
        for (int u = 0; u < VNF; ++u) {
          if (u >= A.NV) break;
#pragma unroll
          for (int q = 0; q < VEC; q += 2) {
            acc0 += __builtin_amdgcn_exp2f((TR::get(rv[u], q) - m) * L2E);
            acc1 += __builtin_amdgcn_exp2f((TR::get(rv[u], q + 1) - m) * L2E);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
#pragma unroll
        for (int u = 0; u < VNF; ++u) {
          if (u >= A.NV) break;
#pragma unroll
          for (int q = 0; q < VEC; ++q) {
            const float x = TR::get(rv[u], q);
            const float d = is_finite(x) ? (x - m) * L2E : -__builtin_inff();
            acc0 += __builtin_amdgcn_exp2f(d);  // exp2(-inf) = 0: masked terms add nothing, without a branch
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      se = (double)acc0 + (double)acc1;
    }
  } else {
  // General path (chunks longer than the register budget): one streaming pass with the first-max key, a running
  // finite maximum m and s = sum(exp(x - m)) rescaled whenever m grows (float32 exp per element, float64 sums).
  auto load = [&](uint4* r, int j0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int base = lo + ((j0 + u) * VNT + t) * VEC;
      r[u] = make_uint4(0, 0, 0, 0);
      if (j0 + u < A.NV && A.vec_ok && base + VEC <= hi)
        r[u] = *(const uint4*)(rowp + (int64_t)base * (DT == VS_F32 ? 4 : 2));
    }
  };
  uint4 cur[U], nxt[U];
  load(cur, 0);
  load_epochs();
  for (int j0 = 0; j0 < A.NV; j0 += U) {
    if (j0 + U < A.NV) load(nxt, j0 + U);  // the next batch is in flight while this one is reduced
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + u >= A.NV) continue;
      const int base = lo + ((j0 + u) * VNT + t) * VEC;
      const bool full = A.vec_ok && base + VEC <= hi;
      float xs[VEC];
#pragma unroll
      for (int q = 0; q < VEC; ++q)
        xs[q] = full ? TR::get(cur[u], q) : (base + q < hi ? TR::one(rowp, base + q) : -__builtin_inff());
      float vm = -__builtin_inff();
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        if (base + q < hi) {
          const u64 k = amkey64(xs[q], (uint32_t)(base + q));
          am = k > am ? k : am;
          if (is_finite(xs[q])) vm = xs[q] > vm ? xs[q] : vm;
        }
      }
      if (vm > m) {
        if (se > 0.0) se *= exp((double)m - (double)vm);
        m = vm;
      }
      if (is_finite(m)) {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < VEC; ++q)
          if (base + q < hi && is_finite(xs[q])) acc += expf(xs[q] - m);
        se += (double)acc;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) cur[u] = nxt[u];
  }
  }
  VS_TR(A, 1);
  // each wave reduces its lanes (the key's maximum, the maximum, then the sum rescaled to it); with a slot per wave
  // lane 0 publishes the wave's partial, else one LDS exchange and one barrier, then thread 0 merges the VNW waves
  auto publish = [&](VPart* pp, u64 kb, float mb, double sb) {
    const u64 tag = (u64)(ep + 1u) << 32;
    const u64 sbits = (u64)__double_as_longlong(sb);
    st_dev(&pp->w[0], tag | (kb >> 32));
    st_dev(&pp->w[1], tag | (kb & 0xFFFFFFFFull));
    st_dev(&pp->w[2], tag | (u64)__float_as_uint(mb));
    st_dev(&pp->w[3], tag | (sbits >> 32));
    st_dev(&pp->w[4], tag | (sbits & 0xFFFFFFFFull));
  };
  {
    const int wv = t / WAVE;
    const u64 kw = wave_max(am);
    const float mw = wave_max(m);
    const float L2E = 1.44269504088896340736f;
    const double sw = wave_sum((se > 0.0 && is_finite(mw)) ? se * (double)__builtin_amdgcn_exp2f((m - mw) * L2E) : 0.0);
    if (per_wave) {
      if (lane_id() == 0) publish(myslot, kw, mw, sw);
    } else if (lane_id() == 0) {
      red64[wv] = kw;
      redf[wv] = mw;
      redd[wv] = sw;
    }
    if (!per_wave) __syncthreads();  // uniform
    if (!per_wave && t == 0) {
      u64 kb = red64[0];
      float mb = redf[0];
#pragma unroll
      for (int w = 1; w < VNW; ++w) {
        kb = red64[w] > kb ? red64[w] : kb;
        mb = redf[w] > mb ? redf[w] : mb;
      }
      double sb = 0.0;
#pragma unroll
      for (int w = 0; w < VNW; ++w)
        sb += (redd[w] > 0.0 && is_finite(mb)) ? redd[w] * (double)__builtin_amdgcn_exp2f((redf[w] - mb) * L2E) : 0.0;
      publish(myslot, kb, mb, sb);
    }
  }
  VS_TR(A, 2);
  if (g != G - 1) {
    VS_TR_FLUSH(A);
    return;
  }
  // this row's token slot: the request's finisher advances its epoch after it has read the token
  const u64 qtag = (u64)(tep + 1u) << 32;
  // the row's finisher: merge the row's partials in one wave (<= 64), each reloaded until all its words show the tag
  if (t < WAVE) {
    u64 k = 0;
    float mm = -__builtin_inff();
    double e = 0.0;
    bool ok = true;
    if (t < nslots) {
      VPart* pp = parts + t;
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      u64 w[VPW];
      const uint32_t se = (uint32_t)ld_dev(&pp->w[VEPW]);  // the slot's epoch: only this lane changes it
      const u64 stag = (u64)(se + 1u) << 32;
      for (;;) {
#pragma unroll
        for (int i = 0; i < VPW; ++i) w[i] = ld_dev(&pp->w[i]);
        ok = true;
#pragma unroll
        for (int i = 0; i < VPW; ++i) ok = ok && (w[i] & 0xFFFFFFFF00000000ull) == stag;
        if (ok || __builtin_amdgcn_s_memrealtime() - t0 > VWAIT_TICKS) break;
        __builtin_amdgcn_s_sleep(1);
      }
      pp->w[VEPW] = se + 1u;  // read in this call (a plain store: read by later calls only)
      k = (w[0] << 32) | (w[1] & 0xFFFFFFFFull);
      mm = __uint_as_float((uint32_t)w[2]);
      e = __longlong_as_double((long long)((w[3] << 32) | (w[4] & 0xFFFFFFFFull)));
    }
    if (__builtin_expect(!__all(ok), 0)) {  // the time bound was reached: token -1
      k = 0;
      mm = __builtin_nanf("");
      e = 0.0;
    }
    VS_TR(A, 3);
    const u64 bam = wave_max(k);
    const int32_t tok = bam ? (int32_t)key_index(bam) : -1;
    if (t == 0) {  // the token first: the request's finisher waits for it, not for the logprob
      if (tp < A.T - 1) st_dev(&rowtok[2 * (size_t)row], qtag | (u64)(uint32_t)tok);
      A.out_argmax[row] = tok;
    }
    const float M = wave_max(mm);
    // the rescaling factors and the logarithm in float (the logprob's tolerance is 1e-5 relative): v_exp_f32 of
    // (m - M) log2 e, and log(S) = log1p(S - 1) with S >= 1 (it holds the maximum's own term), which keeps the float
    // log1p's relative accuracy when one token dominates
    const float L2E = 1.44269504088896340736f;
    const double S =
        wave_sum((e > 0.0 && is_finite(M)) ? e * (double)__builtin_amdgcn_exp2f((mm - M) * L2E) : 0.0);
    if (t == 0 && A.out_lp) {
      const float xj = am_is_nan(bam) ? __builtin_nanf("") : key_value(bam);
      A.out_lp[row] =
          (is_finite(xj) && S > 0.0) ? (float)((double)xj - ((double)M + (double)log1pf((float)(S - 1.0)))) : 0.0f;
    }
  } else if (t < 2 * WAVE && tp == A.T - 1) {
    // the request's last row: its accept length (specdec.py:327), computed by the finisher's second wave while the
    // first merges the row (row T - 1 has no draft of its own): the other rows' tokens reloaded until they show the
    // tag, 64 positions per ballot, the accept length at the first mismatch
    const int ln = t - WAVE;
    const int32_t* dr = A.drafts + (size_t)req * (A.T - 1);
    int nacc = 0;
    bool found = false;
    for (int base = 0; base < A.T - 1; base += WAVE) {
      const int i = base + ln;
      bool stop = i >= A.T - 1;
      if (!stop) {
        const size_t ti = (size_t)req * A.T + i;
        const uint32_t te = (uint32_t)(base == 0 ? qep : ld_dev(&rowtok[2 * ti + 1]));
        const u64 ttag = (u64)(te + 1u) << 32;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        u64 w;
        for (;;) {
          w = ld_dev(&rowtok[2 * ti]);
          if ((w & 0xFFFFFFFF00000000ull) == ttag || __builtin_amdgcn_s_memrealtime() - t0 > VWAIT_TICKS) break;
          __builtin_amdgcn_s_sleep(1);
        }
        rowtok[2 * ti + 1] = te + 1u;  // read in this call (a plain store: read by later calls only)
        stop = (w & 0xFFFFFFFF00000000ull) != ttag || dr[i] != (int32_t)(uint32_t)w;
      }
      // every token slot is read (and its epoch advanced), also past the first mismatch: a slot left unread would
      // keep an epoch whose tag this call's token carries
      const unsigned long long mb2 = __ballot(stop);
      if (!found) {
        if (mb2) {
          nacc += __ffsll((long long)mb2) - 1;
          found = true;
        } else {
          nacc += WAVE;
        }
      }
    }
    if (ln == 0) A.out_accept[req] = nacc;
  }
  VS_TR_FLUSH(A);
}

}  // namespace vs

using namespace vs;

extern "C" size_t vs_verify_workspace_bytes(int B, int T, int V) {
  (void)V;
  size_t R = (B < 1 || T < 1) ? 1 : (size_t)B * T;
  return 16 * (size_t)VRMAX + sizeof(VPart) * R * VGMAX;  // token slots, partial slots
}

extern "C" int vs_verify_greedy(const void* logits, int dtype, int B, int T, int V, int64_t ld, int vocab_valid,
                                const int32_t* drafts, int32_t* out_argmax, int32_t* out_accept, float* out_logprob,
                                void* ws, size_t ws_bytes, vs_stream_t stream) {
  if (B < 0 || T < 1) return fail(VS_EINVAL, "vs_verify_greedy: B < 0 or T < 1");
  if (B == 0) return VS_OK;
  if (V < 1 || vocab_valid < 1 || vocab_valid > V) return fail(VS_EINVAL, "vs_verify_greedy: need 1 <= vocab_valid <= V");
  if (ld < V) return fail(VS_EINVAL, "vs_verify_greedy: ld < V");
  if (dtype != VS_F32 && dtype != VS_BF16 && dtype != VS_F16) return fail(VS_EINVAL, "vs_verify_greedy: bad dtype");
  if (!logits || !out_argmax || !out_accept || !ws || (T > 1 && !drafts))
    return fail(VS_EINVAL, "vs_verify_greedy: null pointer argument");
  if ((long long)B * T > VRMAX) return fail(VS_EINVAL, "vs_verify_greedy: B*T above 8192 rows");
  if (ws_bytes < vs_verify_workspace_bytes(B, T, V)) return fail(VS_EWORKSPACE, "vs_verify_greedy: workspace too small");
  const DevInfo* dv = dev_info();
  if (!dv) return fail(VS_EHIP, "vs_verify_greedy: no HIP device");
  const int VEC = dtype == VS_F32 ? 4 : 8;
  const int unit = VNT * VEC;
  const int R = B * T;
  const int chmax = VNV_MAX * unit;
  int gmin = (vocab_valid + chmax - 1) / chmax;
  if (gmin > VGMAX) return fail(VS_EINVAL, "vs_verify_greedy: vocab_valid too large");
  // About NVT 16-byte loads per lane (measured best on MI355X: less work per workgroup
  // adds merge overhead, more lengthens each workgroup's chain), but never more workgroups than are
  // resident at once (a second wave would start only after the first finished).
  constexpr int NVT = 6;
  const void* kfn = dtype == VS_F32 ? (const void*)vs_verify_kernel<VS_F32>
                    : dtype == VS_BF16 ? (const void*)vs_verify_kernel<VS_BF16>
                                       : (const void*)vs_verify_kernel<VS_F16>;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kfn, VNT, 0) != hipSuccess || per_cu < 1) per_cu = 1;
  int G = (vocab_valid + NVT * unit - 1) / (NVT * unit);
  const int gres = (per_cu * dv->cus) / R;
  if (G > gres) G = gres;
  const int gf = (vocab_valid + VNF * unit - 1) / (VNF * unit);  // the fewest workgroups the fast path allows
  if (G < gf) G = gf;
  if (G < 1) G = 1;
  if (G > VGMAX) G = VGMAX;
  if (G < gmin) G = gmin;
  int CH = (vocab_valid + G - 1) / G;
  CH = (CH + unit - 1) / unit * unit;
  G = (vocab_valid + CH - 1) / CH;
  VerifyArgs a;
  a.logits = logits;
  a.ld = ld;
  a.B = B;
  a.T = T;
  a.V = V;
  a.vv = vocab_valid;
  a.G = G;
  a.CH = CH;
  a.NV = CH / unit;
  a.vec_ok = ((uintptr_t)logits % 16 == 0) && (ld % VEC == 0);
  a.drafts = drafts;
  a.out_argmax = out_argmax;
  a.out_accept = out_accept;
  a.out_lp = out_logprob;
  a.ws = (char*)ws;
  a.trace = g_trace;
  // rows per launch: all of a launch's workgroups resident at once (finishers wait for their row's workgroups)
  const int cap = per_cu * dv->cus;
  int rpl = cap / G;
  if (rpl < 1) rpl = 1;
  for (int r0 = 0; r0 < R; r0 += rpl) {
    const int n = (R - r0) < rpl ? (R - r0) : rpl;
    a.row0 = r0;
    void* kargs[] = {&a};
    const hipError_t e = hipLaunchKernel(kfn, dim3((unsigned)(n * G)), dim3(VNT), kargs, 0, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "vs_verify_greedy: launch");
  }
  return VS_OK;
}
