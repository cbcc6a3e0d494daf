// vs_lmhead.hip - the bf16 lm_head GEMM with the greedy-verify epilogue fused in, for gfx950: logits are never
// written to HBM; each workgroup reduces its slice of the vocabulary to per-position (first-max key, max, sum-exp)
// partials; workgroup p merges position p from tagged partials (no atomics, no second launch; a second launch
// merges them when the vocabulary gives fewer workgroups than positions), into argmax, accept length and logprob.
//
// Reference: logits = lm_head(h) in bf16 (volundr-mlx/volundr.py:958-968, bf16 weight [vocab_size, hidden]; spec
// verify's head call, spec/verify.py:223), then tok = argmax(logits[:, :vv]) and nacc = sum(cumprod(inp[1:] ==
// tok[:-1])) (spec/specdec.py:326-327, scheduler.py:462-463). The logits here are bf16(fp32 sum of products), as a
// bf16 matmul produces them; the epilogue is the verify kernel's (first-max argmax over the bf16 values, logprob =
// x[tok] - logsumexp(x[:vv])).
//
// Shape of the work: R = B*T positions (<= 80) x N vocabulary rows x K hidden, R tiny. The weight (N*K*2 bytes,
// 2.54 GB at 248320 x 5120) is read exactly once and dominates: the kernel is HBM-bound. Design:
//  * one 512-thread workgroup per CU (persistent over a contiguous range of 16-row vocabulary tiles);
//  * v_mfma_f32_16x16x32_bf16 with the weight as the A operand, loaded straight from HBM into registers: lane
//    (m = l%16, g = l/16) holds W[row m][k + 8g .. 8g + 7]; the loads are arranged so that each instruction reads
//    whole 128-byte runs of 8 rows, and the operands are rebuilt with one DPP lane rotation; one two-step group of
//    loads per tile is in flight per wave;
//  * the hidden rows (B operand) are staged through LDS in 256-wide k-chunks, double-buffered, shared by the 8 waves
//    (each workgroup reads h once: 256 x R x K x 2 bytes of L2 traffic in all);
//  * accumulators stay in VGPRs for the whole K loop; the epilogue rounds each to bf16 and folds it into running
//    per-lane partials.
#include "vs_common.h"
#include "vs_host.h"
#include "vs_lmsample.h"

#pragma clang fp contract(off)

namespace vs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int LNT = 512;            // threads per workgroup
constexpr int LNW = LNT / WAVE;     // waves per workgroup
constexpr int KS = 32;              // k per MFMA
constexpr int LRMAX = 80;           // positions per call (5 tiles of 16)
constexpr int LPMAX = 2048;         // workgroups per launch
constexpr size_t LWS_HEAD = 256;    // workspace head (unused)
constexpr int LMPW = 4;             // positions one wave of the merging workgroup reduces at a time

// Workgroup partials, position-major and one array per field ([R][P] each), so that the merge's lanes, which walk
// the workgroups of one position, read consecutive words: (first-max key, float64 sum-exp, float32 max).
struct LParts {
  u64* amkey;
  double* se;
  float* mf;
};
__device__ __forceinline__ LParts lparts(char* ws, int R) {
  LParts q;
  q.amkey = (u64*)(ws + LWS_HEAD);
  q.se = (double*)(q.amkey + (size_t)R * LPMAX);
  q.mf = (float*)(q.se + (size_t)R * LPMAX);
  return q;
}

// merge_in partials: five 64-bit words per (position, workgroup), [R][LNT] at the workspace's partial area (slot
// (p, wg) is only ever written by workgroup wg for position p, whatever the grid size of the call), each
// the tag (high half) over 32 bits of payload (first-max key high/low, maximum, sum-exp high/low); a 64-bit store
// is single-copy atomic, so a word that shows the tag holds this call's payload. Tag = the slot's epoch (word 7)
// + 1; the merging workgroup advances it once it has read the slot, and the writer reads it before it stores, so
// that calls, and a captured graph's replays, tag their words apart whatever shapes they have.
constexpr int LTW = 8;  // words per partial slot (5 used)
// (after the position-major arrays of the second-launch merge, so that the two layouts never share words)
__device__ __forceinline__ u64* ltparts(char* ws, int R) {
  return (u64*)(ws + LWS_HEAD + (size_t)(8 + 8 + 4) * LPMAX * R);
}
// Wall-clock bound (100 MHz ticks, 100 ms) on a merging workgroup's wait for the other workgroups' partials: every
// workgroup of the launch is resident on an otherwise idle device (one per CU), so it is reached only if other
// work held CUs for that long; the position then reports token -1 (no draft matches it) and logprob NaN.
constexpr uint64_t LWAIT_TICKS = 10000000;

struct LHArgs {
  const uint16_t* h;  // [R, ldh] bf16
  int64_t ldh;
  const uint16_t* W;  // [N, ldw] bf16
  int64_t ldw;
  int N, vv, K, B, T, R, ntiles;
  int merge_in;  // workgroup p merges position p from tagged partials (else vs_lmhead_merge_kernel does)
  const int32_t* drafts;  // [B, T-1]
  int32_t* out_argmax;    // [R]
  int32_t* out_accept;    // [B]
  float* out_lp;          // [R] or null
  uint16_t* out_logits;   // [R, ldo] bf16 or null
  int64_t ldo;
  char* ws;  // [LWS_HEAD bytes] then the workgroup partials (LParts, or tagged words when merge_in); sampling: LSParts
  const vs_row_params* params;  // sampling epilogue: one row per position
  unsigned long long* trace;  // development builds only (VS_TRACE); null otherwise
};

// Sampling epilogue. Each round, a top-k position's values go to LDS as 16-bit ordered values (the bf16 logit's
// ord32 >> 16: equal values compare equal, zero = not finite) at fixed slots; after the last round one wave per
// position selects its largest ones. ls_ord16 / ls_key64 convert between the two.
constexpr int LS_VROUNDS = 4;  // rounds a workgroup may run (its tiles <= LS_VROUNDS * LNW * NTW)
__device__ __forceinline__ uint32_t ls_ord16(float x) { return is_finite(x) ? ord32(x) >> 16 : 0u; }
__device__ __forceinline__ u64 ls_key64(uint32_t v, uint32_t id) {
  const uint32_t o = (v << 16) | ((v & 0x8000u) ? 0u : 0xFFFFu);  // a bf16 value's ord32 (see ord32)
  return ((u64)o << 32) | (u64)(0xFFFFFFFFu - id);
}

// The kept keys of one position, written to list[0, LS_KMAX) (zero padded) with the largest to *head: every key
// whose value reaches the k-th largest (a superset of the k largest when values tie), reduced to exactly the k
// largest (ties to the lower id) only when they would not fit. vbuf holds the position's values, 4 per word (nw
// words); `id` maps a slot to its vocabulary row. One wave; counts are ballots or lane sums.
//  1. L = the k-th largest lane maximum (a lower bound of the k-th largest value: >= k lanes reach it), by a
//     bisection with one compare per lane;
//  2. the values >= L (usually k to 2k) become keys in the position's own LDS row (already read);
//  3. the kept keys are selected among those few (ls_keep). Only when more than LS_CAND values reach L does the
//     selection run over all the values.
constexpr int LS_CAND = 512;
template <int C>
__device__ __forceinline__ void ls_keep(const u64* cb, int n, int k, u64* list, u64* head) {
  constexpr int PER = C / WAVE;
  const int ln = lane_id();
  u64 kk[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int i = ln + WAVE * u;
    kk[u] = i < n ? cb[i] : (u64)0;
  }
  auto count_ge = [&](u64 c) -> int {  // keys >= c (c > 0: zeros never count)
    int m = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) m += (int)__popcll(__ballot(kk[u] >= c));
    return m;
  };
  u64 T = 1;
  if (n > k) {
    uint32_t H = 0;
    for (int b = 15; b >= 0; --b) {
      const uint32_t c = H | (1u << b);
      H = count_ge((u64)c << 48) >= k ? c : H;
    }
    T = (u64)H << 48;
    if (count_ge(T) > LS_KMAX) {  // ties beyond the slots: the k-th largest key itself
      for (int b = 47; b >= 0; --b) {
        const u64 c = T | ((u64)1 << b);
        T = count_ge(c) >= k ? c : T;
      }
    }
  }
  int m = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u) m += kk[u] >= T ? 1 : 0;
  const int incl = wave_scan(m);
  const int tot = __builtin_amdgcn_readlane(incl, WAVE - 1);
  int p = incl - m;
  u64 best = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (kk[u] >= T) {
      list[p++] = kk[u];
      best = kk[u] > best ? kk[u] : best;
    }
  for (int i = tot + ln; i < LS_KMAX; i += WAVE) list[i] = 0;
  best = wave_max(best);
  if (ln == 0) *head = best;
}

template <int NW, typename IdOf>
__device__ __forceinline__ void ls_select(uint16_t* vbuf, int nw, int k, IdOf id, u64* list, u64* head) {
  const int ln = lane_id();
  uint32_t v[NW][4];
  uint32_t lm = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u) {
    const int w = ln + WAVE * u;
    const uint2 d = w < nw ? *(const uint2*)(vbuf + 4 * w) : make_uint2(0u, 0u);
    v[u][0] = d.x & 0xFFFFu;
    v[u][1] = d.x >> 16;
    v[u][2] = d.y & 0xFFFFu;
    v[u][3] = d.y >> 16;
    lm = max3u(lm, max3u(v[u][0], v[u][1], 0u), max3u(v[u][2], v[u][3], 0u));
  }
  uint32_t L = 1;
  if ((int)__popcll(__ballot(lm != 0)) >= k) {
    L = 0;
    for (int b = 15; b >= 0; --b) {
      const uint32_t c = L | (1u << b);
      L = (int)__popcll(__ballot(lm >= c)) >= k ? c : L;
    }
  }
  int m = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) m += v[u][e] >= L ? 1 : 0;
  const int incl = wave_scan(m);
  const int tot = __builtin_amdgcn_readlane(incl, WAVE - 1);
  if (tot <= LS_CAND) {
    u64* cb = (u64*)vbuf;  // the row has been read into registers: its space holds the candidate keys
    int p = incl - m;
#pragma unroll
    for (int u = 0; u < NW; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (v[u][e] >= L) cb[p++] = ls_key64(v[u][e], id(4 * (ln + WAVE * u) + e));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (tot <= 2 * WAVE)
      ls_keep<2 * WAVE>(cb, tot, k, list, head);  // the usual case: two candidates per lane
    else
      ls_keep<LS_CAND>(cb, tot, k, list, head);
    return;
  }
  // Many values reach L (one lane held most of the largest): the selection runs over all of them. H = the largest
  // 16-bit value with >= k values at or above it; ties at H beyond the slots keep their lowest ids.
  auto count_ge = [&](uint32_t c) -> int {  // values >= c (c >= 1: zeros never count)
    int cnt = 0;
#pragma unroll
    for (int u = 0; u < NW; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) cnt += v[u][e] >= c ? 1 : 0;
    return wave_sum(cnt);
  };
  uint32_t H = 0;
  for (int b = 15; b >= 0; --b) {
    const uint32_t c = H | (1u << b);
    H = count_ge(c) >= k ? c : H;
  }
  uint32_t idmax = 0xFFFFFFFFu;
  if (count_ge(H) > LS_KMAX) {
    const int need = k - count_ge(H + 1);  // ties to keep (>= 1)
    auto ties_below = [&](uint32_t c) -> int {  // ties with id < c
      int cnt = 0;
#pragma unroll
      for (int u = 0; u < NW; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) cnt += (v[u][e] == H && id(4 * (ln + WAVE * u) + e) < c) ? 1 : 0;
      return wave_sum(cnt);
    };
    idmax = 0;  // the largest c with fewer than `need` ties below it: the need-th smallest tie id
    for (int b = 30; b >= 0; --b) {
      const uint32_t c = idmax | (1u << b);
      idmax = ties_below(c) < need ? c : idmax;
    }
  }
  m = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      m += (v[u][e] > H || (v[u][e] == H && (idmax == 0xFFFFFFFFu || id(4 * (ln + WAVE * u) + e) <= idmax))) ? 1 : 0;
  const int incl2 = wave_scan(m);
  const int tot2 = __builtin_amdgcn_readlane(incl2, WAVE - 1);
  int p = incl2 - m;
  u64 best = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t slot = 4 * (ln + WAVE * u) + e;
      if (v[u][e] > H || (v[u][e] == H && (idmax == 0xFFFFFFFFu || id(slot) <= idmax))) {
        const u64 key = ls_key64(v[u][e], id(slot));
        list[p++] = key;
        best = key > best ? key : best;
      }
    }
  for (int i = tot2 + ln; i < LS_KMAX; i += WAVE) list[i] = 0;
  best = wave_max(best);
  if (ln == 0) *head = best;
}

// (m, s) pairs: s = sum exp(x - m) over finite x, accumulated in float64; the rescale factor exp(m - mm) <= 1 is
// v_exp_f32 of (m - mm) log2 e (relative error a few 1e-7, far inside the logprob tolerance; a float64 exp per
// merge step made the cross-lane and cross-workgroup merges cost tens of microseconds)
__device__ __forceinline__ float exp_le0(float d) { return __builtin_amdgcn_exp2f(d * 1.44269504088896340736f); }
__device__ __forceinline__ void lse_merge(float& m, double& s, float m2, double s2) {
  const float mm = m2 > m ? m2 : m;
  double r = 0.0;
  if (s > 0.0 && is_finite(mm)) r += s * (double)exp_le0(m - mm);
  if (s2 > 0.0 && is_finite(mm)) r += s2 * (double)exp_le0(m2 - mm);
  m = mm;
  s = r;
}

// SAMPLE: the sampling epilogue (one tile of <= 16 positions): besides the (first-max key, max, sum-exp) partials,
// every position of a top-k row keeps its workgroup's largest keys, and the partials go to LSParts for
// vs_lmhead_sample_merge_kernel instead of an in-launch merge.
template <int NTT, int NTW, int KC, bool SAMPLE>
__global__ __launch_bounds__(LNT) __attribute__((amdgpu_waves_per_eu(LNT / 256))) void vs_lmhead_verify_kernel(
    LHArgs A) {
  static_assert(!SAMPLE || NTT == 1, "the sampling epilogue serves one tile of positions");
  static_assert(LS_KMAX == WAVE, "a wave writes a position's kept keys");
  constexpr int RP = 16 * NTT;  // positions padded to whole MFMA tiles
  // sampling: per position, every round's values (LNW waves x 4 lanes x NTW x 4 per round) as 16-bit ordered values;
  // rows padded by 8 bytes, so that the 16 positions a wave writes at once fall in different LDS banks
  constexpr int LS_RV = LNW * 4 * NTW * 4;
  constexpr int LS_VSTR = LS_VROUNDS * LS_RV + 4;
  __shared__ __attribute__((aligned(16))) uint16_t vbuf[SAMPLE ? 16 : 1][SAMPLE ? LS_VSTR : 1];
  __shared__ int scls[16], svlim[16];
  __shared__ uint32_t rn[SAMPLE ? LNW : 1][SAMPLE ? RP : 1];
  constexpr int SPC = KC / KS;
  constexpr int HSTR = KC + 8;
  __shared__ __attribute__((aligned(16))) uint16_t hs[2][RP][HSTR];
  __shared__ u64 rk[LNW][RP];
  __shared__ float rm[LNW][RP];
  __shared__ double rs[LNW][RP];
  const int t = threadIdx.x, wv = t / WAVE, ln = lane_id();
  const int m16 = ln & 15, kg = ln >> 4;
  const int P = gridDim.x, wg = blockIdx.x;
  const int R = A.R, K = A.K;
  const int nchunks = K / KC;
  const int t0 = (int)((long long)wg * A.ntiles / P), t1 = (int)((long long)(wg + 1) * A.ntiles / P);
  const int rounds = (t1 - t0 + LNW * NTW - 1) / (LNW * NTW);
  const LParts parts = lparts(A.ws, A.R);
  VS_TR_DECL(A);
  VS_TR(A, 0);
  // accept lengths start at T-1 (every draft accepted); the merge lowers them to the first mismatch. A coherent
  // store, waited for: the merging workgroups run on other XCDs, and each merges only after it has seen workgroup
  // 0's partials, so every atomicMin follows it (a second merge launch follows it anyway).
  if (!SAMPLE && wg == 0) {
    for (int b = t; b < A.B; b += LNT) st_dev(&A.out_accept[b], A.T - 1);
    publish_wait();  // complete before this workgroup's partials (stored much later) can release a merge
  }

  if constexpr (SAMPLE) {
    if (t < 16) {
      int vl = 0, c = LS_UNSUPPORTED;
      if (t < R) c = ls_class(A.params[t], A.N, &vl);
      scls[t] = c;
      svlim[t] = vl;
    }
  }
  uint32_t nfc[NTT];  // finite values of the lane's positions (sampling)
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) nfc[tt] = 0;

  // padded positions R..RP-1 read as zeros in both buffers
  {
    const int per = (RP - R) * (KC / 8);
    for (int i = t; i < 2 * per; i += LNT) {
      const int b = i / per, rem = i - b * per;
      *(uint4*)&hs[b][R + rem / (KC / 8)][(rem % (KC / 8)) * 8] = make_uint4(0, 0, 0, 0);
    }
  }
  // per-lane running partials of its positions tt*16 + m16
  u64 pk[NTT];
  float pm[NTT];
  double ps[NTT];
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) {
    pk[tt] = 0;
    pm[tt] = -__builtin_inff();
    ps[tt] = 0.0;
  }
  const int hpieces = R * (KC / 8);  // 16-byte pieces of one hidden chunk
  constexpr int HPT = RP * (KC / 8) / LNT;  // pieces per thread (R <= RP rows)
  static_assert(HPT * LNT == RP * (KC / 8), "the threads cover a padded chunk exactly");
  // this thread's pieces: (row, column) in the chunk, clamped into range (the clamped ones are not stored)
  int hrow[HPT], hcol[HPT];
  bool hin[HPT];
#pragma unroll
  for (int q = 0; q < HPT; ++q) {
    const int i0 = q * LNT + t;
    hin[q] = i0 < hpieces;
    const int i = hin[q] ? i0 : hpieces - 1;
    hrow[q] = i / (KC / 8);
    hcol[q] = (i % (KC / 8)) * 8;
  }
  // Weight fetch, two MFMA steps (64 k = 128 bytes of a row) at a time, so that every load instruction reads whole
  // 128-byte runs of 8 rows (an instruction reading 64 bytes from each of 16 rows streams at ~60% of the rate):
  // half 0 reads rows 0-7 of the tile, half 1 rows 8-15; lane (m, g) reads, of row m & 7 (+ 8 in half 1), the
  // 16-byte piece g if it is its own row's half (m < 8 for half 0), else piece 4 + g, which belongs to its partner
  // lane m ^ 8 in the second step. Step 0 takes the own-half register; step 1 takes the other register from the
  // partner lane (DPP row rotate by 8 inside each 16-lane row).
  // Addresses: a 64-bit base per round (the round's first tile, uniform) plus 32-bit byte offsets per lane and tile
  // (a round spans < 4 GB: LNW*NTW tiles of 16 rows of at most ldw*2 bytes, checked on the host).
  // The stream never stops between rounds: the last group of a round fetches the next round's first group, and the
  // last chunk stages the next round's first hidden chunk, so a round's epilogue overlaps those loads.
  const bool lo8 = m16 < 8;
  auto round_offsets = [&](int rr, const char*& base, uint32_t (&o0)[NTW], uint32_t (&o1)[NTW]) {
    const int tb = t0 + rr * LNW * NTW;
    base = (const char*)(A.W + (int64_t)tb * 16 * A.ldw);
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      int tl = tb + j * LNW + wv;
      // a tile past the range reads the range's last tile (its lines are being fetched for another wave anyway)
      tl = tl < t1 ? tl : t1 - 1;
      int r0 = tl * 16 + (m16 & 7), r1 = r0 + 8;
      r0 = (r0 < A.N ? r0 : A.N - 1) - tb * 16;
      r1 = (r1 < A.N ? r1 : A.N - 1) - tb * 16;
      o0[j] = (uint32_t)((int64_t)r0 * A.ldw * 2) + (uint32_t)((lo8 ? kg : 4 + kg) * 16);
      o1[j] = (uint32_t)((int64_t)r1 * A.ldw * 2) + (uint32_t)((lo8 ? 4 + kg : kg) * 16);
    }
  };
  const char* wbase;
  uint32_t wo0[NTW], wo1[NTW];
  round_offsets(0, wbase, wo0, wo1);
  // the staged pieces live in named registers (an array of them was kept in scratch memory)
  uint4 hr0, hr1, hr2, hr3, hr4;
  static_assert(HPT <= 5, "at most five staged pieces per thread");
#define LH_HLOAD(cc)                                                                                          \
  {                                                                                                           \
    const uint16_t* hbase = A.h + (int64_t)(cc) * KC;                                                         \
    hr0 = *(const uint4*)(hbase + (int64_t)hrow[0] * A.ldh + hcol[0]);                                        \
    if constexpr (HPT > 1) hr1 = *(const uint4*)(hbase + (int64_t)hrow[HPT > 1 ? 1 : 0] * A.ldh + hcol[HPT > 1 ? 1 : 0]); \
    if constexpr (HPT > 2) hr2 = *(const uint4*)(hbase + (int64_t)hrow[HPT > 2 ? 2 : 0] * A.ldh + hcol[HPT > 2 ? 2 : 0]); \
    if constexpr (HPT > 3) hr3 = *(const uint4*)(hbase + (int64_t)hrow[HPT > 3 ? 3 : 0] * A.ldh + hcol[HPT > 3 ? 3 : 0]); \
    if constexpr (HPT > 4) hr4 = *(const uint4*)(hbase + (int64_t)hrow[HPT > 4 ? 4 : 0] * A.ldh + hcol[HPT > 4 ? 4 : 0]); \
  }
#define LH_HSTORE(bb)                                                                                          \
  {                                                                                                            \
    if (hin[0]) *(uint4*)&hs[bb][hrow[0]][hcol[0]] = hr0;                                                      \
    if constexpr (HPT > 1) if (hin[HPT > 1 ? 1 : 0]) *(uint4*)&hs[bb][hrow[HPT > 1 ? 1 : 0]][hcol[HPT > 1 ? 1 : 0]] = hr1; \
    if constexpr (HPT > 2) if (hin[HPT > 2 ? 2 : 0]) *(uint4*)&hs[bb][hrow[HPT > 2 ? 2 : 0]][hcol[HPT > 2 ? 2 : 0]] = hr2; \
    if constexpr (HPT > 3) if (hin[HPT > 3 ? 3 : 0]) *(uint4*)&hs[bb][hrow[HPT > 3 ? 3 : 0]][hcol[HPT > 3 ? 3 : 0]] = hr3; \
    if constexpr (HPT > 4) if (hin[HPT > 4 ? 4 : 0]) *(uint4*)&hs[bb][hrow[HPT > 4 ? 4 : 0]][hcol[HPT > 4 ? 4 : 0]] = hr4; \
  }
  LH_HLOAD(0)
  uint4 wb[NTW][2];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    wb[j][0] = *(const uint4*)(wbase + wo0[j]);
    wb[j][1] = *(const uint4*)(wbase + wo1[j]);
  }
  // merge_in: the epoch of this workgroup's slot for position t (this thread stores the partial), loaded after the
  // first weights (so that their waits do not wait for it)
  const uint32_t ep_t =
      (!SAMPLE && A.merge_in && t < R) ? (uint32_t)ld_dev(ltparts(A.ws, R) + ((size_t)t * LNT + wg) * LTW + 7) : 0u;
  __syncthreads();  // the padded rows are zeroed
  LH_HSTORE(0)
  __syncthreads();
  int cg = 0;  // chunks processed so far (all rounds): the LDS buffer of the current chunk is cg & 1
  for (int r = 0; r < rounds; ++r) {
    int tile[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) tile[j] = t0 + r * LNW * NTW + j * LNW + wv;
    // the next round's addresses (this round's again on the last round: its final prefetch is a spare)
    const char* nbase;
    uint32_t no0[NTW], no1[NTW];
    round_offsets(r + 1 < rounds ? r + 1 : r, nbase, no0, no1);
    f32x4_t acc[NTW][NTT];
#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
      for (int tt = 0; tt < NTT; ++tt) acc[j][tt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    VS_TR(A, 1 + 3 * r);
    for (int c = 0; c < nchunks; ++c, ++cg) {
      const int b = cg & 1;
      // the next chunk's hidden rows (chunk 0 again after the last: the next round's first) are fetched now and
      // stored into the idle buffer after this chunk's steps
      const int cn = c + 1 < nchunks ? c + 1 : 0;
      LH_HLOAD(cn)
      const bool last_chunk = c + 1 == nchunks;
#pragma unroll
      for (int gq = 0; gq < SPC / 2; ++gq) {
        bf16x8_t hb0[NTT], hb1[NTT];
#pragma unroll
        for (int tt = 0; tt < NTT; ++tt) {
          hb0[tt] = *(const bf16x8_t*)&hs[b][tt * 16 + m16][(2 * gq) * KS + kg * 8];
          hb1[tt] = *(const bf16x8_t*)&hs[b][tt * 16 + m16][(2 * gq + 1) * KS + kg * 8];
        }
        // the group fetched now: the next one of this round, or the next round's first
        const bool wrap = last_chunk && gq == SPC / 2 - 1;
        const int gn = wrap ? 0 : c * (SPC / 2) + gq + 1;
        const char* fb = wrap ? nbase : wbase;
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const uint4 a0 = wb[j][0], a1 = wb[j][1];
          const uint4 s0 = lo8 ? a0 : a1;
          const uint4 o = lo8 ? a1 : a0;
          uint4 s1;
          s1.x = dpp32<0x128>(o.x, o.x);  // row_ror:8 -> the value of lane m ^ 8
          s1.y = dpp32<0x128>(o.y, o.y);
          s1.z = dpp32<0x128>(o.z, o.z);
          s1.w = dpp32<0x128>(o.w, o.w);
          const uint32_t f0 = wrap ? no0[j] : wo0[j], f1 = wrap ? no1[j] : wo1[j];
          wb[j][0] = *(const uint4*)(fb + (f0 + (uint32_t)gn * 4 * KS));
          wb[j][1] = *(const uint4*)(fb + (f1 + (uint32_t)gn * 4 * KS));
          __builtin_amdgcn_sched_barrier(0);  // keep the next group's loads here, one group ahead of their use
#pragma unroll
          for (int tt = 0; tt < NTT; ++tt) {
            acc[j][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, s0), hb0[tt],
                                                                 acc[j][tt], 0, 0, 0);
            acc[j][tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, s1), hb1[tt],
                                                                 acc[j][tt], 0, 0, 0);
          }
        }
      }
      LH_HSTORE(b ^ 1)
      __syncthreads();
    }
    wbase = nbase;
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      wo0[j] = no0[j];
      wo1[j] = no1[j];
    }
    VS_TR(A, 2 + 3 * r);
    // epilogue of the round: lane holds vocabulary rows tile*16 + 4*kg + q of positions tt*16 + m16. The values
    // are rounded to bf16 (the hardware conversion, round to nearest even); a lane whose in-range values are all
    // finite (magnitude bits below +inf's) takes the short path: the maximum by three-input instructions, its first
    // vocabulary row by a backward sweep of equality selects (rows grow with j and q), and exp2 sums; otherwise the
    // exact per-value path.
    const float L2E = 1.44269504088896340736f;
#pragma unroll
    for (int tt = 0; tt < NTT; ++tt) {
      const int pos = tt * 16 + m16;
      const int vlim = SAMPLE ? svlim[m16] : A.vv;  // sampling: the row's own range ([0, vv) or the whole row)
      float xs[NTW][4];
      float best = -__builtin_inff();
      uint32_t mag = 0;
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int v = tile[j] * 16 + kg * 4 + q;
          const bool in = (tile[j] < t1) & (v < vlim);
          const float x = (float)(__bf16)acc[j][tt][q];
          xs[j][q] = in ? x : -__builtin_inff();
          mag = in ? max3u(mag, __float_as_uint(x) & 0x7FFFFFFFu, 0u) : mag;
        }
        best = max3f(best, max3f(xs[j][0], xs[j][1], xs[j][2]), xs[j][3]);
      }
      if (A.out_logits) {
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int v = tile[j] * 16 + kg * 4 + q;
            if (tile[j] < t1 && v < A.N && pos < R)
              A.out_logits[(int64_t)pos * A.ldo + v] = __builtin_bit_cast(uint16_t, (__bf16)acc[j][tt][q]);
          }
      }
      if (mag < 0x7F800000u) {
        if (best > -__builtin_inff()) {  // some value in range
          int bi = 0;
#pragma unroll
          for (int j = NTW - 1; j >= 0; --j)
#pragma unroll
            for (int q = 3; q >= 0; --q) bi = xs[j][q] == best ? tile[j] * 16 + kg * 4 + q : bi;
          const u64 k = amkey64(best, (uint32_t)bi);
          pk[tt] = k > pk[tt] ? k : pk[tt];
          if (best > pm[tt]) {
            if (ps[tt] > 0.0) ps[tt] *= (double)__builtin_amdgcn_exp2f((pm[tt] - best) * L2E);
            pm[tt] = best;
          }
        }
        if (is_finite(pm[tt])) {
          float s0 = 0.0f, s1 = 0.0f;  // two chains of additions; exp2(-inf) = 0 for the values out of range
#pragma unroll
          for (int j = 0; j < NTW; ++j) {
            s0 += __builtin_amdgcn_exp2f((xs[j][0] - pm[tt]) * L2E);
            s1 += __builtin_amdgcn_exp2f((xs[j][1] - pm[tt]) * L2E);
            s0 += __builtin_amdgcn_exp2f((xs[j][2] - pm[tt]) * L2E);
            s1 += __builtin_amdgcn_exp2f((xs[j][3] - pm[tt]) * L2E);
          }
          ps[tt] += (double)s0 + (double)s1;
        }
      } else {
        float vm = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int v = tile[j] * 16 + kg * 4 + q;
            const float x = xs[j][q];
            if ((tile[j] < t1) & (v < A.vv)) {
              const u64 k = amkey64(x, (uint32_t)v);
              pk[tt] = k > pk[tt] ? k : pk[tt];
              if (is_finite(x)) vm = x > vm ? x : vm;
            }
          }
        }
        if (vm > pm[tt]) {
          if (ps[tt] > 0.0) ps[tt] *= (double)expf(pm[tt] - vm);
          pm[tt] = vm;
        }
        if (is_finite(pm[tt])) {
          float sacc = 0.0f;
#pragma unroll
          for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (is_finite(xs[j][q])) sacc += expf(xs[j][q] - pm[tt]);
          ps[tt] += (double)sacc;
        }
      }
      if constexpr (SAMPLE) {
        // the finite count, and for a top-k row this round's values (sampler.py:130-136 keeps finite logits only)
        const int kc = scls[m16];
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) nfc[tt] += is_finite(xs[j][q]) ? 1u : 0u;
        if (kc >= 1) {
#pragma unroll
          for (int j = 0; j < NTW; ++j) {
            const uint2 d = make_uint2(ls_ord16(xs[j][0]) | (ls_ord16(xs[j][1]) << 16),
                                       ls_ord16(xs[j][2]) | (ls_ord16(xs[j][3]) << 16));
            *(uint2*)&vbuf[m16][r * LS_RV + ((wv * 4 + kg) * NTW + j) * 4] = d;
          }
        }
      }
    }
  }
#undef LH_HLOAD
#undef LH_HSTORE

  // lanes of one position (same m16): xor 16, 32; then the waves through LDS; then the workgroup partial
#pragma unroll
  for (int tt = 0; tt < NTT; ++tt) {
#pragma unroll
    for (int sh = 16; sh <= 32; sh *= 2) {
      const u64 ok = sh == 16 ? lane_xor<16>(pk[tt]) : lane_xor<32>(pk[tt]);
      const float om = sh == 16 ? lane_xor<16>(pm[tt]) : lane_xor<32>(pm[tt]);
      const double os = sh == 16 ? lane_xor<16>(ps[tt]) : lane_xor<32>(ps[tt]);
      pk[tt] = ok > pk[tt] ? ok : pk[tt];
      lse_merge(pm[tt], ps[tt], om, os);
    }
    if constexpr (SAMPLE) {
      nfc[tt] += lane_xor<16>(nfc[tt]);
      nfc[tt] += lane_xor<32>(nfc[tt]);
      if (kg == 0) rn[wv][tt * 16 + m16] = nfc[tt];
    }
    if (kg == 0) {
      rk[wv][tt * 16 + m16] = pk[tt];
      rm[wv][tt * 16 + m16] = pm[tt];
      rs[wv][tt * 16 + m16] = ps[tt];
    }
  }
  __syncthreads();
  if (t < R) {
    u64 k = rk[0][t];
    float m = rm[0][t];
    double s = rs[0][t];
#pragma unroll
    for (int w = 1; w < LNW; ++w) {
      k = rk[w][t] > k ? rk[w][t] : k;
      lse_merge(m, s, rm[w][t], rs[w][t]);
    }
    if constexpr (SAMPLE) {
      // the merge runs as a later launch: plain stores
      const LSParts q = ls_parts(A.ws, R);
      uint32_t nf = 0;
#pragma unroll
      for (int w = 0; w < LNW; ++w) nf += rn[w][t];
      const size_t ix = (size_t)t * LS_PMAX + wg;
      q.amkey[ix] = k;
      q.mf[ix] = m;
      q.se[ix] = s;
      q.nfin[ix] = nf;
    } else if (A.merge_in) {
      u64* w = ltparts(A.ws, R) + ((size_t)t * LNT + wg) * LTW;
      const u64 tg = (u64)(ep_t + 1u) << 32;
      const u64 sb = (u64)__double_as_longlong(s);
      st_dev(&w[0], tg | (k >> 32));
      st_dev(&w[1], tg | (k & 0xFFFFFFFFull));
      st_dev(&w[2], tg | (u64)__float_as_uint(m));
      st_dev(&w[3], tg | (sb >> 32));
      st_dev(&w[4], tg | (sb & 0xFFFFFFFFull));
    } else {
      const size_t ix = (size_t)t * LPMAX + wg;
      st_dev(&parts.amkey[ix], k);
      st_dev(&parts.mf[ix], m);
      st_dev(&parts.se[ix], s);
    }
  }
  if constexpr (SAMPLE) {
    // each wave selects the kept keys of its positions (w, w + 8) from every round's values (the barrier above
    // ordered the rounds' LDS writes): the list and its largest key
    VS_TR(A, 12);
    const LSParts q = ls_parts(A.ws, R);
    const int nw = rounds * LS_RV / 4;
    // slot -> vocabulary row: slot = r * LS_RV + ((w * 4 + g) * NTW + j) * 4 + e holds row tile * 16 + g * 4 + e of
    // tile t0 + r * LNW * NTW + j * LNW + w
    auto id_of = [&](uint32_t slot) -> uint32_t {
      const uint32_t rr = slot / LS_RV, rem = slot % LS_RV;
      const uint32_t e = rem & 3, jj = (rem >> 2) % NTW, wk = (rem >> 2) / NTW;
      const uint32_t tl = (uint32_t)t0 + rr * LNW * NTW + jj * LNW + (wk >> 2);
      return tl * 16 + (wk & 3) * 4 + e;
    };
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const int pos = wv + pp * LNW;
      const int kc = pos < R ? scls[pos] : 0;
      if (kc >= 1)
        ls_select<LS_VROUNDS * LS_RV / 4 / WAVE>(vbuf[pos], nw, kc, id_of,
                                                 q.lists + ((size_t)pos * LS_PMAX + wg) * LS_KMAX,
                                                 q.heads + (size_t)pos * LS_PMAX + wg);
      VS_TR(A, 14 + pp);
    }
    VS_TR(A, 13);
    VS_TR_FLUSH(A);
    return;
  }
  VS_TR(A, 20);
  if (!A.merge_in || wg >= R) {
    VS_TR_FLUSH(A);
    return;
  }
  // Workgroup p merges position p (no atomics): thread i reloads workgroup i's partial until its five words show
  // the call's tag, then the block takes the first-max key, the maximum, and the sum-exp rescaled to it; the
  // accept length is lowered to the first mismatching draft position (specdec.py:327) by one atomicMin per
  // mismatching position.
  __syncthreads();  // the workgroup reduction above is done with rk / rm / rs
  {
    const int p = wg;
    u64 k = 0;
    float m = -__builtin_inff();
    double sv = 0.0;
    int ok = 1;
    if (t < P) {
      u64* w = ltparts(A.ws, R) + ((size_t)p * LNT + t) * LTW;
      const uint32_t se = (uint32_t)ld_dev(&w[7]);  // the slot's epoch: only this thread changes it
      const u64 tg = (u64)(se + 1u) << 32;
      const uint64_t c0 = __builtin_amdgcn_s_memrealtime();
      u64 v[5];
      for (;;) {
        // one word polled while the workgroup is still streaming (a merging workgroup waits ~10 us for the last
        // ones, and its reloads share the fabric with their weight reads), then all five
        v[4] = ld_dev(&w[4]);
        if ((v[4] & 0xFFFFFFFF00000000ull) != tg) {
          if (__builtin_amdgcn_s_memrealtime() - c0 > LWAIT_TICKS) {
            ok = 0;
            break;
          }
          __builtin_amdgcn_s_sleep(2);
          continue;
        }
#pragma unroll
        for (int i = 0; i < 5; ++i) v[i] = ld_dev(&w[i]);
        bool all = true;
#pragma unroll
        for (int i = 0; i < 5; ++i) all = all && (v[i] & 0xFFFFFFFF00000000ull) == tg;
        if (all) break;
        if (__builtin_amdgcn_s_memrealtime() - c0 > LWAIT_TICKS) {
          ok = 0;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      w[7] = se + 1u;  // read in this call (a plain store: read by later calls only)
      k = (v[0] << 32) | (v[1] & 0xFFFFFFFFull);
      m = __uint_as_float((uint32_t)v[2]);
      sv = __longlong_as_double((long long)((v[3] << 32) | (v[4] & 0xFFFFFFFFull)));
    }
    VS_TR(A, 21);
    const u64 kw = wave_max(k);
    const float mw = wave_max(m);
    const int okw = __all(ok) ? 1 : 0;
    __shared__ int okf[LNW];
    if (ln == 0) {
      rk[wv][0] = kw;
      rm[wv][0] = mw;
      okf[wv] = okw;
    }
    __syncthreads();
    u64 K0 = rk[0][0];
    float M = rm[0][0];
    bool good = okf[0] != 0;
#pragma unroll
    for (int q = 1; q < LNW; ++q) {
      K0 = rk[q][0] > K0 ? rk[q][0] : K0;
      M = rm[q][0] > M ? rm[q][0] : M;
      good = good && okf[q] != 0;
    }
    if (t == 0) {  // the token and the accept length first (their stores complete while the logprob is computed)
      const int32_t tok = good ? (int32_t)key_index(K0) : -1;
      A.out_argmax[p] = tok;
      const int b = p / A.T, tp = p % A.T;
      if (tp < A.T - 1 && A.drafts[(size_t)b * (A.T - 1) + tp] != tok) atomicMin(&A.out_accept[b], tp);
    }
    const float L2E = 1.44269504088896340736f;
    const double sw =
        wave_sum((sv > 0.0 && is_finite(M)) ? sv * (double)__builtin_amdgcn_exp2f((m - M) * L2E) : 0.0);
    if (ln == 0) rs[wv][0] = sw;
    __syncthreads();
    if (t == 0 && A.out_lp) {
      double S = 0.0;
#pragma unroll
      for (int q = 0; q < LNW; ++q) S += rs[q][0];
      VS_TR(A, 24);
      const float xj = am_is_nan(K0) ? __builtin_nanf("") : key_value(K0);
      // log(S) = log1p(S - 1): S >= 1 (the maximum's own term), so the float log keeps its relative accuracy also
      // when one token dominates (S - 1 tiny)
      A.out_lp[p] = !good ? __builtin_nanf("")
                          : (is_finite(xj) && S > 0.0)
                                ? (float)((double)xj - ((double)M + (double)log1pf((float)(S - 1.0))))
                                : 0.0f;
    }
  }
  VS_TR(A, 22);
  VS_TR_FLUSH(A);
}


// Merge for many positions (a separate launch, one 256-thread workgroup per position, so that the positions merge
// in parallel on as many CUs): the position's P partials, the maximum first, then each sum rescaled to it once.
constexpr int MNT = 256;
constexpr int MPT = LPMAX / MNT;  // partials per thread at most
__global__ __launch_bounds__(MNT) void vs_lmhead_merge_kernel(LHArgs A, int P) {
  __shared__ u64 rk[MNT / WAVE];
  __shared__ float rm[MNT / WAVE];
  __shared__ double rs[MNT / WAVE];
  const int pos = blockIdx.x, t = threadIdx.x, wv = t / WAVE, ln = lane_id();
  const LParts parts = lparts(A.ws, A.R);
  u64 kk[MPT];
  float mm[MPT];
  double ss[MPT];
#pragma unroll
  for (int u = 0; u < MPT; ++u) {  // every load issued before the first is used (clamped, masked below)
    const int i0 = u * MNT + t;
    const size_t ix = (size_t)pos * LPMAX + (i0 < P ? i0 : P - 1);
    kk[u] = ld_dev(&parts.amkey[ix]);
    mm[u] = ld_dev(&parts.mf[ix]);
    ss[u] = ld_dev(&parts.se[ix]);
  }
  u64 k = 0;
  float m = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < MPT; ++u) {
    const bool in = u * MNT + t < P;
    k = (in && kk[u] > k) ? kk[u] : k;
    m = (in && mm[u] > m) ? mm[u] : m;
  }
  k = wave_max(k);
  m = wave_max(m);
  if (ln == 0) {
    rk[wv] = k;
    rm[wv] = m;
  }
  __syncthreads();
#pragma unroll
  for (int w = 0; w < MNT / WAVE; ++w) {
    k = rk[w] > k ? rk[w] : k;
    m = rm[w] > m ? rm[w] : m;
  }
  double sm = 0.0;
#pragma unroll
  for (int u = 0; u < MPT; ++u)
    sm += (u * MNT + t < P && ss[u] > 0.0 && is_finite(m)) ? ss[u] * (double)exp_le0(mm[u] - m) : 0.0;
  sm = wave_sum(sm);
  if (ln == 0) rs[wv] = sm;
  __syncthreads();
  if (t == 0) {
    sm = 0.0;
#pragma unroll
    for (int w = 0; w < MNT / WAVE; ++w) sm += rs[w];
    const float xj = am_is_nan(k) ? __builtin_nanf("") : key_value(k);
    const int32_t tok = (int32_t)key_index(k);
    A.out_argmax[pos] = tok;
    // log(sm) = log1p(sm - 1): sm >= 1 (the maximum's own term) keeps the float log1p's relative accuracy
    if (A.out_lp)
      A.out_lp[pos] =
          (is_finite(xj) && sm > 0.0) ? (float)((double)xj - ((double)m + (double)log1pf((float)(sm - 1.0)))) : 0.0f;
    const int b = pos / A.T, tp = pos % A.T;
    if (tp < A.T - 1 && A.drafts[(size_t)b * (A.T - 1) + tp] != tok) atomicMin(&A.out_accept[b], tp);
  }
}

// Positions up to which the launch's own workgroups merge them (beyond, a second launch does).
constexpr int LMERGE_IN = LRMAX;

template <int NTT, int NTW, int KC>
static int lmhead_launch(const LHArgs& a, int P, hipStream_t stream) {
  hipLaunchKernelGGL((vs_lmhead_verify_kernel<NTT, NTW, KC, false>), dim3(P), dim3(LNT), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "vs_lmhead_verify_greedy: launch");
  if (!a.merge_in) {
    hipLaunchKernelGGL(vs_lmhead_merge_kernel, dim3(a.R), dim3(MNT), 0, stream, a, P);
    e = hipGetLastError();
  }
  return e == hipSuccess ? VS_OK : hip_fail(e, "vs_lmhead_verify_greedy: merge launch");
}

template <int KC>
static int lmhead_sample_launch(const LHArgs& a, int P, hipStream_t stream) {
  hipLaunchKernelGGL((vs_lmhead_verify_kernel<1, 4, KC, true>), dim3(P), dim3(LNT), 0, stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VS_OK : hip_fail(e, "vs_lmhead_sample: launch");
}

}  // namespace vs

using namespace vs;

extern "C" size_t vs_lmhead_sample_workspace_bytes(int R) { return ls_workspace_bytes(R < 1 ? 1 : R); }

extern "C" int vs_lmhead_sample(const void* h, int64_t ldh, const void* W, int64_t ldw, int N, int K, int R,
                                const vs_row_params* params, int32_t* out_ids, float* out_logprob,
                                uint32_t* out_flags, int32_t* out_keep, void* ws, size_t ws_bytes,
                                vs_stream_t stream) {
  if (R < 0 || R > LS_RMAX) return fail(VS_EINVAL, "vs_lmhead_sample: need 0 <= R <= 16 rows");
  if (R == 0) return VS_OK;
  if (N < 1) return fail(VS_EINVAL, "vs_lmhead_sample: N < 1");
  if (K < 256 || K % 256 != 0) return fail(VS_EINVAL, "vs_lmhead_sample: K must be a positive multiple of 256");
  if (ldh < K || ldw < K || ldh % 8 != 0 || ldw % 8 != 0)
    return fail(VS_EINVAL, "vs_lmhead_sample: row strides must be >= K and multiples of 8");
  if (!h || !W || !params || !out_ids || !out_logprob || !ws)
    return fail(VS_EINVAL, "vs_lmhead_sample: null pointer argument");
  if ((uintptr_t)h % 16 != 0 || (uintptr_t)W % 16 != 0)
    return fail(VS_EINVAL, "vs_lmhead_sample: h and W must be 16-byte aligned");
  if ((int64_t)LNW * 8 * 16 * ldw * 2 >= ((int64_t)1 << 32))
    return fail(VS_EINVAL, "vs_lmhead_sample: weight rows too long (ldw)");
  if (ws_bytes < vs_lmhead_sample_workspace_bytes(R)) return fail(VS_EWORKSPACE, "vs_lmhead_sample: workspace too small");
  const DevInfo* dv = dev_info();
  if (!dv) return fail(VS_EHIP, "vs_lmhead_sample: no HIP device");
  LHArgs a = {};
  a.h = (const uint16_t*)h;
  a.ldh = ldh;
  a.W = (const uint16_t*)W;
  a.ldw = ldw;
  a.N = N;
  a.vv = N;
  a.K = K;
  a.B = R;
  a.T = 1;
  a.R = R;
  a.ntiles = (N + 15) / 16;
  a.merge_in = 0;
  a.ws = (char*)ws;
  a.params = params;
  a.trace = g_trace;
  int P = dv->cus;
  if (P > a.ntiles) P = a.ntiles;
  if (P > LS_PMAX) P = LS_PMAX;
  if ((a.ntiles + P - 1) / P > LS_VROUNDS * LNW * 4)
    return fail(VS_EINVAL, "vs_lmhead_sample: N too large for the workgroups' value buffers");
  const int rc = K % 512 == 0 ? lmhead_sample_launch<512>(a, P, (hipStream_t)stream)
                              : lmhead_sample_launch<256>(a, P, (hipStream_t)stream);
  if (rc != VS_OK) return rc;
  return ls_merge_launch(params, R, N, P, (char*)ws, out_ids, out_logprob, out_flags, out_keep, (hipStream_t)stream);
}

extern "C" size_t vs_lmhead_workspace_bytes(int B, int T) {
  const size_t R = (B < 1 || T < 1) ? 1 : (size_t)B * T;
  return LWS_HEAD + (size_t)(8 + 8 + 4) * LPMAX * R + (size_t)LTW * 8 * LNT * R;  // arrays, then tagged slots
}

extern "C" int vs_lmhead_verify_greedy(const void* h, int64_t ldh, const void* W, int64_t ldw, int N, int K,
                                       int vocab_valid, int B, int T, const int32_t* drafts, int32_t* out_argmax,
                                       int32_t* out_accept, float* out_logprob, void* out_logits, int64_t ldo,
                                       void* ws, size_t ws_bytes, vs_stream_t stream) {
  if (B < 0 || T < 1) return fail(VS_EINVAL, "vs_lmhead_verify_greedy: B < 0 or T < 1");
  if (B == 0) return VS_OK;
  const long long R = (long long)B * T;
  if (R > LRMAX) return fail(VS_EINVAL, "vs_lmhead_verify_greedy: B*T above 80 positions");
  if (N < 1 || vocab_valid < 1 || vocab_valid > N)
    return fail(VS_EINVAL, "vs_lmhead_verify_greedy: need 1 <= vocab_valid <= N");
  if (K < 256 || K % 256 != 0) return fail(VS_EINVAL, "vs_lmhead_verify_greedy: K must be a positive multiple of 256");
  const bool kc512 = R <= 32 && K % 512 == 0;
  if (ldh < K || ldw < K || ldh % 8 != 0 || ldw % 8 != 0)
    return fail(VS_EINVAL, "vs_lmhead_verify_greedy: row strides must be >= K and multiples of 8");
  if (!h || !W || !out_argmax || !out_accept || !ws || (T > 1 && !drafts))
    return fail(VS_EINVAL, "vs_lmhead_verify_greedy: null pointer argument");
  if ((uintptr_t)h % 16 != 0 || (uintptr_t)W % 16 != 0)
    return fail(VS_EINVAL, "vs_lmhead_verify_greedy: h and W must be 16-byte aligned");
  if ((int64_t)LNW * 8 * 16 * ldw * 2 >= ((int64_t)1 << 32))
    return fail(VS_EINVAL, "vs_lmhead_verify_greedy: weight rows too long (ldw)");
  if (out_logits && ldo < N) return fail(VS_EINVAL, "vs_lmhead_verify_greedy: ldo < N");
  if (ws_bytes < vs_lmhead_workspace_bytes(B, T))
    return fail(VS_EWORKSPACE, "vs_lmhead_verify_greedy: workspace too small");
  const DevInfo* dv = dev_info();
  if (!dv) return fail(VS_EHIP, "vs_lmhead_verify_greedy: no HIP device");
  LHArgs a;
  a.h = (const uint16_t*)h;
  a.ldh = ldh;
  a.W = (const uint16_t*)W;
  a.ldw = ldw;
  a.N = N;
  a.vv = vocab_valid;
  a.K = K;
  a.B = B;
  a.T = T;
  a.R = (int)R;
  a.ntiles = (N + 15) / 16;
  a.drafts = drafts;
  a.out_argmax = out_argmax;
  a.out_accept = out_accept;
  a.out_lp = out_logprob;
  a.out_logits = (uint16_t*)out_logits;
  a.ldo = ldo;
  a.ws = (char*)ws;
  a.trace = g_trace;
  int P = dv->cus;  // one workgroup per CU, each over a contiguous range of vocabulary tiles
  if (P > a.ntiles) P = a.ntiles;
  if (P > LPMAX) P = LPMAX;
  a.merge_in = R <= LMERGE_IN && R <= P && P <= LNT;  // one merging workgroup per position, one thread per partial
  const int ntt = (int)((R + 15) / 16);
  switch (ntt) {
    case 1: return kc512 ? lmhead_launch<1, 4, 512>(a, P, (hipStream_t)stream)
                         : lmhead_launch<1, 4, 256>(a, P, (hipStream_t)stream);
    case 2: return kc512 ? lmhead_launch<2, 4, 512>(a, P, (hipStream_t)stream)
                         : lmhead_launch<2, 4, 256>(a, P, (hipStream_t)stream);
    case 3: return lmhead_launch<3, 4, 256>(a, P, (hipStream_t)stream);
    case 4: return lmhead_launch<4, 2, 256>(a, P, (hipStream_t)stream);
    default: return lmhead_launch<5, 2, 256>(a, P, (hipStream_t)stream);
  }
}
