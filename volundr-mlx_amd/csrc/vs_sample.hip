// vs_sample.hip - batched Sampler.sample (volundr-mlx/sampler.py:100-156) as one cooperative HIP kernel for gfx950.
//
// Layout: row r of the batch is split into G contiguous vocabulary chunks, one 512-thread workgroup each
// (split-vocab, so that B <= 16 rows still occupy the 256 CUs). A workgroup reads its chunk from HBM exactly once
// with 16-byte loads and keeps it in VGPRs (<= 24 values per lane) for every later pass. The G workgroups of a
// row sit on one XCD (blockIdx -> row mapping below) and talk through a per-row control block in the workspace.
//
// Per row, by class (decided from the row's parameters, identically in every workgroup):
//   GREEDY  (Sampling.greedy)        local first-max argmax + logsumexp partials -> last workgroup merges.
//   TOPK    (1 <= top_k <= kcap)     local top-k by 64-bit key -> last workgroup sorts the G*k candidates and runs
//                                    softmax / top-p / min-p / draw on the k survivors in one wave, in the order
//                                    sampler.py:140-156 uses.
//   FULL    (top-k off or large)     row max + finite count over a spin barrier; the kept set (sampler.py:
//                                    133-139) gets a mass histogram; if it has <= 1024 members they are gathered
//                                    and one workgroup finishes as for TOPK, otherwise top-p and the draw are
//                                    resolved by a row-cooperative radix select on the keys, weighted by
//                                    fixed-point probability mass (deterministic integer sums).
// No full-vocabulary sort happens anywhere.
#include "vs_common.h"
#include "vs_host.h"
#include "vs_lmsample.h"

#include <mutex>

#pragma clang fp contract(off)

namespace vs {

constexpr int SNT = 512;         // threads per workgroup
constexpr int SNW = SNT / WAVE;  // waves per workgroup
constexpr int NRED = 16;         // entries of each LDS reduction/broadcast array (>= SNW and >= 6)
static_assert(NRED >= 2 * SNW, "one reduction slot per wave, and the TOPK wave heads at 8 ..");
constexpr int EPT_MAX = 24;      // logits per lane in flight during the load
constexpr int NBIN = 256;        // radix digit = 8 bits
constexpr int MAX_ROUNDS = 32;   // histogram slots per row (8 count + 1 coarse + 4 fine + 1 + 7 + 7 radix rounds)
constexpr int GMAX = 64;         // workgroups per row
constexpr int GCAP = 1024;       // gather area of the FULL path (keys)
constexpr int GSMALL = 128;      // kept sets up to this size are finished in one workgroup
constexpr int GCAP2 = 512;       // elements gathered from the located value bins (<= SNT: one per thread in the final scans)
static_assert(GCAP2 <= SNT, "the final in-bin scans hold one gathered element per thread");
constexpr int NSET = 4;          // coarse value bins refined in the second histogram round
constexpr int BIGCAP = 5120;     // kept logits of the selected coarse bins that one workgroup resolves after a gather
constexpr int RANK_MAX = 512;    // largest set ranked by counting
constexpr int KEYS_CAP = 8192;   // LDS key area (64 KB): the merged candidate lists of a row
constexpr int KCAP = 256;        // largest top_k of the TOPK class
constexpr int RPL_MAX = 64;      // rows per launch (workspace is sized for this many)
constexpr int PAIRS_ALL = 2048;  // (id, count) tables up to this many entries are loaded whole by every workgroup
// Row-barrier time bounds in ticks of the 100 MHz real-time counter. A row's workgroups arrive within ~10 us of one
// another on an idle device; under a plain launch a wait that outlasts 200 us means some workgroup of the row is not
// resident (other streams hold the CUs), and the row gives up so that the host can repeat the call cooperatively.
// Under a cooperative launch every workgroup is resident, so only slowed waves can delay a barrier: 5 ms.
constexpr uint64_t WAIT_TICKS = 20000;        // 200 us
constexpr uint64_t WAIT_TICKS_COOP = 500000;  // 5 ms
// LDS scalar slots (misc): 0-17 single counters and flags, then arrays
constexpr int M_SEGC = 24;                         // [SNW] candidates per wave (TOPK)
constexpr int M_CNTS = M_SEGC + SNW;               // [GMAX] kept count per workgroup (FULL, small kept set)
constexpr int M_OFFS = M_CNTS + GMAX;              // [GMAX] their offsets
constexpr int M_XCH = (M_OFFS + GMAX + 1) & ~1;    // 2 x u64 exchange slots (8-byte aligned)
constexpr int M_STAT1 = M_XCH + 4;                 // [SNW] block_stats maxima
constexpr int M_STAT2 = M_STAT1 + SNW;             // [SNW]
constexpr int M_WB = M_STAT2 + SNW;                // [SNW] lane_max_bound per-wave bounds
constexpr int M_NZ = M_WB + SNW;                   // [SNW] lane_max_bound lanes with a finite logit
constexpr int NMISC = M_NZ + SNW;

enum RowClass { CLS_GREEDY = 0, CLS_TOPK = 1, CLS_FULL = 2 };

// Per-row control block; all zero between calls.
struct RowCtl {
  uint32_t bar;     // spin-barrier arrivals
  uint32_t done;    // workgroups finished (bits 0-15), of them the one that wrote the row's result (bits
                    // 16-23) and those that timed out at a row barrier (bits 24-31)
  uint32_t nfin;    // finite count of the row
  uint32_t mkey;    // ord32 of the largest finite logit
  u64 amkey;        // np.argmax key of the row
  uint32_t gcount;  // gather reservations
  uint32_t mcnt;    // min-p kept count
  u64 mfix;         // min-p kept fixed-point mass
  double mf64;      // min-p kept float64 mass
  uint32_t epoch;   // calls of this row so far (the XL row-barrier flags carry it); cleanup advances it
  uint32_t nminkey; // ~ord32 of the smallest finite logit (max-reduced)
  uint32_t g2count; // second gather reservations
  uint32_t gmax;    // largest per-workgroup kept count
};
static_assert(sizeof(RowCtl) == 64, "RowCtl layout");

struct Part {  // one per workgroup, written with device-coherent stores
  u64 amkey;
  uint32_t nfin;
  uint32_t kc;
  float mf;
  uint32_t pad;
  double se;
  u64 heads[8];  // TOPK lists of the unsorted format: eight of the list's largest keys (0 = none)
};
static_assert(sizeof(Part) == 96, "Part layout");

struct HistSlot {
  uint32_t cnt[NBIN];
  u64 fix[NBIN];
  double f64[NBIN];
  u64 mk[NBIN];
};

// Areas written with workgroup-scope stores (parts, lists, gathers, flags) start on their own 128-byte lines,
// apart from the lines that device-scope atomics update (the control block, the histogram slots).
constexpr size_t OFF_PART = 128;
constexpr size_t OFF_CAND = OFF_PART + sizeof(Part) * GMAX;
constexpr size_t OFF_GATHER = OFF_CAND + sizeof(u64) * KEYS_CAP;
constexpr size_t OFF_HIST = OFF_GATHER + sizeof(u64) * GCAP;
constexpr size_t OFF_BIG = OFF_HIST + sizeof(HistSlot) * MAX_ROUNDS;
constexpr size_t OFF_FLAGS = OFF_BIG + sizeof(u64) * BIGCAP;  // [GMAX] XL row-barrier flags
constexpr size_t ROW_WS = OFF_FLAGS + sizeof(u64) * GMAX;
static_assert(OFF_CAND % 128 == 0 && OFF_GATHER % 128 == 0 && OFF_HIST % 128 == 0 && OFF_BIG % 128 == 0 &&
                  OFF_FLAGS % 128 == 0 && ROW_WS % 128 == 0,
              "row workspace areas on 128-byte lines");

struct SampleArgs {
  const void* logits;
  int64_t ld;
  int B;     // rows in this launch
  int row0;  // first batch row of this launch
  int V;
  int G;
  int CH;
  int NV;      // vector loads per lane
  int vec_ok;  // 16-byte loads allowed
  int has_hist;
  int lds_ch;  // chunk length the LDS areas are sized for
  int kcap;    // candidate-list capacity per workgroup (a power of two)
  int kmax;    // largest top_k of the TOPK class for this launch
  uint32_t spin_limit;  // polls before a row barrier gives up (testing hook; 0xFFFFFFFF: unbounded by polls)
  uint32_t debug;  // VS_DEBUG_* testing flags (vs_set_debug)
  uint64_t spin_ticks;  // real-time ticks (10 ns) before a row barrier gives up
  double fix_scale;  // probability -> fixed point (2^fix_shift)
  int fix_shift;
  double zspan_max;     // ln(fix_scale) - ln(1e6): the kept-value span up to which z comes from fixed point
  const vs_row_params* params;
  vs_row_state* state;  // device-resident request state, or null
  int list_k;           // > 0: top-list mode (vs_topk_batch): every row publishes its list_k largest logits, sorted
  int32_t* list_ids;    // [B, list_k]
  float* list_vals;     // [B, list_k]
  int32_t* pool;        // history pool of the state entry point
  const int32_t* slots;  // state entry point: row r uses params[slots[r]] and state[slots[r]] (null: r)
  const int32_t* tabs;   // state entry point: the (id, count) tables the states point into
  const int32_t* hist;
  const int32_t* bias_ids;
  const float* bias_vals;
  const int32_t* mask_ids;
  int32_t* out_ids;
  float* out_lp;
  uint32_t* out_flags;
  int32_t* out_keep;
  char* ws;
  unsigned long long* trace;  // development builds only (VS_TRACE); null otherwise
};

// LDS layout (dynamic): [xv: CH floats] [keys: max(KEYS_CAP u64, CH u32), the penalty counts during the edits]
// [tk: 2*KCAP u64] [hist] [scratch] [fine bins]. Every class reads its chunk from xv; keys holds candidate lists.
struct Smem {
  uint32_t* cnt;  // penalty counts (during the edits)
  float* xv;      // the processed chunk
  u64* fkeys;     // gathered keys (= keys)
  u64* keys;      // candidate lists
  u64* tk;
  uint32_t* hc;
  u64* hfix;
  double* hf64;
  u64* hmk;
  u64* red64;
  double* redf;
  int* redi;
  int* misc;     // NMISC ints
  uint32_t* fc;  // NSET*256 fine-bin counts
  u64* ffix;     // NSET*256 fine-bin fixed-point masses
  double* ff64;  // NSET*256 fine-bin float64 masses
  uint32_t* rc;  // 256-bin histogram of a workgroup-local radix select (count, fixed-point and float64 mass,
  u64* rfix;     // largest key), used while the other histograms must keep their contents
  double* rf64;
  u64* rmk;
};

__host__ __device__ inline size_t xv_bytes(int CH) { return ((size_t)CH * 4 + 15) & ~(size_t)15; }
__host__ __device__ inline size_t keys_bytes(int CH) {
  const size_t a = (size_t)KEYS_CAP * 8, b = xv_bytes(CH);
  return a > b ? a : b;
}
__host__ __device__ inline size_t region0(int CH) { return xv_bytes(CH) + keys_bytes(CH); }
__device__ __forceinline__ Smem carve(char* base, int CH) {
  Smem s;
  s.xv = (float*)base;
  s.keys = (u64*)(base + xv_bytes(CH));
  s.fkeys = s.keys;
  s.cnt = (uint32_t*)s.keys;  // the penalty counts use the key area before any class needs it
  char* p = base + region0(CH);
  s.tk = (u64*)p;
  p += 2 * KCAP * 8;
  s.hfix = (u64*)p;
  p += NBIN * 8;
  s.hf64 = (double*)p;
  p += NBIN * 8;
  s.hmk = (u64*)p;
  p += NBIN * 8;
  s.hc = (uint32_t*)p;
  p += NBIN * 4;
  s.red64 = (u64*)p;
  p += NRED * 8;
  s.redf = (double*)p;
  p += NRED * 8;
  s.redi = (int*)p;
  p += NRED * 4;
  s.misc = (int*)p;
  p += NMISC * 4;
  s.ffix = (u64*)p;
  p += NSET * NBIN * 8;
  s.ff64 = (double*)p;
  p += NSET * NBIN * 8;
  s.fc = (uint32_t*)p;
  p += NSET * NBIN * 4;
  s.rfix = (u64*)p;
  p += NBIN * 8;
  s.rf64 = (double*)p;
  p += NBIN * 8;
  s.rmk = (u64*)p;
  p += NBIN * 8;
  s.rc = (uint32_t*)p;
  return s;
}
static size_t smem_bytes(int CH) {
  return region0(CH) + 2 * KCAP * 8 + NBIN * (8 + 8 + 8 + 4) + NRED * (8 + 8 + 4) + NMISC * 4 + NSET * NBIN * (8 + 8 + 4) +
         NBIN * (8 + 8 + 8 + 4);
}

// ---------------------------------------------------------------------------------------------------------------
// Histogram scan. One wave walks the 256 bins: lane L owns digits 255-4L .. 252-4L (descending key order), so the
// bins are visited in rank order with one wave-wide scan and a ballot. Finds the first digit whose bin is non-empty
// and whose inclusive cumulative weight reaches `target`; when none does (a target above the total by rounding) the
// lowest non-empty digit, i.e. the last element. Weight = count (count mode) or fixed-point mass. Also returns the
// cumulative sums of all higher digits. The caller has synchronised after filling the bins.
// ---------------------------------------------------------------------------------------------------------------
struct ScanOut {
  int digit;
  u64 cnt_before, fix_before;
  double f64_before;
  u64 cnt, fix;
  double f64;
  u64 mk;
};

__device__ __forceinline__ ScanOut scan256(const Smem& s, const uint32_t* hc, const u64* hfix, const double* hf64,
                                           const u64* hmk, bool count_mode, double target) {
  if (threadIdx.x < WAVE) {
    const int L = threadIdx.x;
    u64 c[4], w[4];
    double f[4];
    u64 lc = 0, lw = 0;
    double lf = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = NBIN - 1 - (4 * L + i);
      c[i] = hc[d];
      w[i] = count_mode ? c[i] : hfix[d];
      f[i] = hf64[d];
      lc += c[i];
      lw += w[i];
      lf += f[i];
    }
    const u64 iw = wave_scan(lw), ic = wave_scan(lc);
    const double iff = wave_scan(lf);
    u64 cw = iw - lw, cc = ic - lc;
    double cf = iff - lf;
    int hit = -1, last = -1;
    u64 hw = 0, hc2 = 0;
    double hf = 0.0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (c[i] > 0) last = i;
      if (hit < 0 && c[i] > 0 && (double)(cw + w[i]) >= target) {
        hit = i;
        hw = cw;
        hc2 = cc;
        hf = cf;
      }
      cw += w[i];
      cc += c[i];
      cf += f[i];
    }
    const unsigned long long hb = __ballot(hit >= 0);
    int lane_sel, i_sel;
    if (hb) {
      lane_sel = __ffsll((long long)hb) - 1;
      i_sel = lane_bcast(hit, lane_sel);
    } else {
      const unsigned long long lb = __ballot(last >= 0);
      lane_sel = lb ? 63 - __clzll((long long)lb) : 0;
      i_sel = lb ? lane_bcast(last, lane_sel) : 0;
      if (i_sel < 0) i_sel = 0;
    }
    if (L == lane_sel) {
      if (!hb) {
        hw = iw - lw;
        hc2 = ic - lc;
        hf = iff - lf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (i < i_sel) {
            hw += w[i];
            hc2 += c[i];
            hf += f[i];
          }
        }
      }
      const int d = NBIN - 1 - (4 * L + i_sel);
      s.misc[0] = d;
      s.red64[0] = hc2;
      s.red64[1] = hw;
      s.redf[0] = hf;
      s.red64[2] = hc[d];
      s.red64[3] = hfix[d];
      s.redf[1] = hf64[d];
      s.red64[4] = hmk ? hmk[d] : 0;
    }
  }
  __syncthreads();
  ScanOut o;
  o.digit = s.misc[0];
  o.cnt_before = s.red64[0];
  o.fix_before = count_mode ? 0 : s.red64[1];
  o.f64_before = s.redf[0];
  o.cnt = s.red64[2];
  o.fix = s.red64[3];
  o.f64 = s.redf[1];
  o.mk = s.red64[4];
  __syncthreads();
  return o;
}

__device__ __forceinline__ ScanOut hist_scan(const Smem& s, bool count_mode, double target) {
  return scan256(s, s.hc, s.hfix, s.hf64, s.hmk, count_mode, target);
}

// Prefix sums of a 256-bin histogram in scan order (digit 255 first, the order scan256 walks): pc[d] and pw[d] hold
// the count and fixed-point sums over digits 255 .. d (inclusive), pf[d] the float64 sum over digits 255 .. d+1
// (exclusive). Called by one whole wave.
__device__ __forceinline__ void hist_prefix(const uint32_t* hc, const u64* hw, const double* hf, u64* pc, u64* pw,
                                            double* pf) {
  const int L = lane_id();
  u64 c[4], w[4];
  double f[4];
  u64 lc = 0, lw = 0;
  double lf = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = NBIN - 1 - (4 * L + i);
    c[i] = hc[d];
    w[i] = hw[d];
    f[i] = hf[d];
    lc += c[i];
    lw += w[i];
    lf += f[i];
  }
  u64 cc = wave_scan(lc) - lc, cw = wave_scan(lw) - lw;
  double cf = wave_scan(lf) - lf;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = NBIN - 1 - (4 * L + i);
    pf[d] = cf;
    cc += c[i];
    cw += w[i];
    cf += f[i];
    pc[d] = cc;
    pw[d] = cw;
  }
}

// The smallest integer >= t (0 for t <= 0, the largest u64 from 2^64 up).
__device__ __forceinline__ u64 ceil_u64(double t) {
  return t <= 0.0 ? (u64)0 : (t >= 18446744073709551616.0 ? ~(u64)0 : (u64)__builtin_ceil(t));
}

// scan256's answer from prefix arrays (hist_prefix): the first digit in scan order whose bin is non-empty and whose
// inclusive weight reaches `target` (the last non-empty digit when none does, which only rounding can cause), with
// the sums before it. Every wave computes it on its own, so no barrier is needed; the caller has synchronised after
// hist_prefix.
__device__ __forceinline__ ScanOut hist_find(const uint32_t* hc, const u64* hw, const double* hf, const u64* pc,
                                             const u64* pw, const double* pf, double target) {
  const int L = lane_id();
  uint32_t c[4];
  u64 w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = NBIN - 1 - (4 * L + i);
    c[i] = hc[d];
    w[i] = pw[d];
  }
  const u64 tg = ceil_u64(target);  // an integer sum reaches target iff it reaches ceil(target)
  int hit = 4, last = -1;
#pragma unroll
  for (int i = 3; i >= 0; --i) {
    hit = (c[i] > 0 && w[i] >= tg) ? i : hit;
    last = (last < 0 && c[i] > 0) ? i : last;
  }
  const unsigned long long hb = __ballot(hit < 4);
  int lane_sel, i_sel;
  if (hb) {
    lane_sel = __ffsll((long long)hb) - 1;
    i_sel = lane_bcast(hit, lane_sel);
  } else {
    const unsigned long long lb = __ballot(last >= 0);
    lane_sel = lb ? 63 - __clzll((long long)lb) : 0;
    i_sel = lb ? lane_bcast(last, lane_sel) : 0;
  }
  const int d = NBIN - 1 - (4 * lane_sel + i_sel);
  ScanOut o;
  o.digit = d;
  o.cnt = hc[d];
  o.fix = hw[d];
  o.f64 = hf[d];
  o.cnt_before = pc[d] - o.cnt;
  o.fix_before = pw[d] - o.fix;
  o.f64_before = pf[d];
  o.mk = 0;
  return o;
}

__device__ __forceinline__ void hist_clear(const Smem& s) {
  const int t = threadIdx.x;
  if (t < NBIN) {
    s.hc[t] = 0;
    s.hfix[t] = 0;
    s.hf64[t] = 0.0;
    s.hmk[t] = 0;
  }
  __syncthreads();
}

__device__ __forceinline__ void hist_add(const Smem& s, u64 key, int shift, u64 fx, double f) {
  const int d = (int)((key >> shift) & 0xFF);
  atomicAdd(&s.hc[d], 1u);
  if (fx) atomicAdd(&s.hfix[d], fx);
  if (f != 0.0) unsafeAtomicAdd(&s.hf64[d], f);
  atomicMax(&s.hmk[d], key);
}

__device__ __forceinline__ bool prefix_match(u64 key, int shift, u64 prefix) {
  return shift >= 56 ? true : ((key >> (shift + 8)) == prefix);
}

// k-th largest of n unique keys in LDS (1 <= k <= n): returns T with |{keys >= T}| == k. Radix select, 8-bit
// digits from the top, stopping as soon as a bin is taken whole.
__device__ __forceinline__ u64 block_kth(const Smem& s, const u64* keys, int n, int k) {
  u64 prefix = 0;
  int shift = 56;
  int krem = k;
  for (;;) {
    hist_clear(s);
    for (int i = threadIdx.x; i < n; i += SNT) {
      const u64 key = keys[i];
      if (prefix_match(key, shift, prefix)) atomicAdd(&s.hc[(key >> shift) & 0xFF], 1u);
    }
    __syncthreads();
    const ScanOut o = hist_scan(s, true, (double)krem);
    const int need = krem - (int)o.cnt_before;
    const u64 np = (prefix << 8) | (u64)o.digit;
    if ((int)o.cnt == need || shift == 0) return np << shift;
    krem = need;
    prefix = np;
    shift -= 8;
  }
}

// Logarithms of the logprob formulas in float32 (the result is a float32 logprob; float log and log1p are
// accurate to a few float ulps, far inside its tolerance), in the forms that keep relative accuracy:
// log(z) for z >= 1 as log1p(z - 1), and log(p / z) for 0 < p <= z as log1p((p - z) / z) when p >= z / 2 (the
// difference is exact) or log(p / z) below.
__device__ __forceinline__ double log_ge1(double z) { return (double)log1pf((float)(z - 1.0)); }
__device__ __forceinline__ double log_ratio(double p, double z) {
  return p >= 0.5 * z ? (double)log1pf((float)((p - z) / z)) : (double)logf((float)(p / z));
}

struct Final {
  int32_t token;
  float lp;
  uint32_t flags;
  int32_t keep;
};

// sampler.py:141-156 on n <= 64 * EM keys sorted descending in LDS (a[0] is the row maximum), in one wave: lane
// L owns positions [L*E, L*E+E), E = ceil(n / 64) <= EM, so every sum and prefix is a lane-sequential loop plus one
// wave scan. Lane 0 leaves the result in LDS for wave_sample.
template <int EM>  // n <= 64 * EM
__device__ __forceinline__ void wave_sample_em(const Smem& s, const u64* a, int n, const vs_row_params& P) {
  {
    const int L = threadIdx.x;
    const int E = EM == 1 ? 1 : (n + WAVE - 1) / WAVE;
    const int i0 = L * E;
    const float tt = P.temperature;
    const float xs0 = key_value(a[0]) / tt;  // sampler.py:141 xs[0]
    double pr[EM];
    double ls = 0.0;
#pragma unroll
    for (int q = 0; q < EM; ++q) {
      pr[q] = 0.0;
      if (q < E && i0 + q < n) {
        const float xs = key_value(a[i0 + q]) / tt;
        const float d = xs - xs0;  // float32 subtraction (:142)
        // exp in float32, widened: relative error <= 2^-23 per mass (the reference's float64 exp of the same d
        // differs by less; sums and cumulative sums inherit that bound, far inside the 1e-6 boundary band and the
        // 1e-5 logprob tolerance; pr[0] = exp(0) = 1 exactly, so a dominant first token's logprob stays exact)
        pr[q] = (double)expf(d);
        ls += pr[q];
      }
    }
    // one scan gives both the total (:143) and each lane's cumulative mass before its first position
    const double incl = wave_scan(ls);
    const double S = lane_bcast(incl, WAVE - 1);
    VS_TRX(40);
#pragma unroll
    for (int q = 0; q < EM; ++q) pr[q] = pr[q] / S;
    const double base = (incl - ls) / S;
    VS_TRX(41);
    int keep = n;
    uint32_t flags = 0;
    if (P.top_p < 1.0) {  // :145-148 first position with cumsum >= top_p
      const double tp = P.top_p;
      double c = base;
      int hit = -1;
      int fb = 0;
#pragma unroll
      for (int q = 0; q < EM; ++q) {
        if (q < E && i0 + q < n) {
          const double prev = c;
          c += pr[q];
          if (hit < 0 && c >= tp) {
            hit = i0 + q;
            fb = fabs(c - tp) < 1e-6 || fabs(prev - tp) < 1e-6;
          }
        }
      }
      const unsigned long long hb = __ballot(hit >= 0);
      if (hb) {
        const int ls2 = __ffsll((long long)hb) - 1;
        keep = lane_bcast(hit, ls2) + 1;
        if (lane_bcast(fb, ls2)) flags |= VS_OUT_TOPP_BOUNDARY;
      }
    }
    if (P.min_p > 0.0) {  // :149-152 first position with pr < pr[0] * min_p
      const double thr = lane_bcast(pr[0], 0) * P.min_p;
      int hit = -1;
#pragma unroll
      for (int q = 0; q < EM; ++q)
        if (hit < 0 && q < E && i0 + q < n && pr[q] < thr) hit = i0 + q;
      const unsigned long long hb = __ballot(hit >= 0);
      int cnt = hb ? lane_bcast(hit, __ffsll((long long)hb) - 1) : n;
      cnt = cnt > 1 ? cnt : 1;
      keep = keep < cnt ? keep : cnt;
    }
    VS_TRX(42);
    double z;  // :153, the cumulative mass through the last kept position (read from the lane that holds it)
    {
      const int owner = (keep - 1) / E, qq = keep - 1 - owner * E;
      double cz = base;
#pragma unroll
      for (int q = 0; q < EM; ++q)
        if (q <= qq && q < E) cz += pr[q];
      z = lane_bcast(cz, owner);
    }
    const double uz = P.u * z;      // :154
    double c = base;
    int hit = -1;
    double hp = 0.0, hc = 0.0;
#pragma unroll
    for (int q = 0; q < EM; ++q) {
      if (q < E && i0 + q < keep) {
        c += pr[q];
        if (hit < 0 && c >= uz) {
          hit = i0 + q;
          hp = pr[q];
          hc = c;
        }
      }
    }
    const unsigned long long hb = __ballot(hit >= 0);
    int j;
    if (hb) {  // :155 searchsorted(cumsum, u*z, 'left')
      const int ls2 = __ffsll((long long)hb) - 1;
      j = lane_bcast(hit, ls2);
      hp = lane_bcast(hp, ls2);
      hc = lane_bcast(hc, ls2);
    } else {  // :156 min(j, keep-1): the last kept position
      j = keep - 1;
      const int owner = j / E, qq = j - owner * E;
      double cc = base, pp = 0.0;
#pragma unroll
      for (int q = 0; q < EM; ++q)
        if (q <= qq && q < E) {
          cc += pr[q];
          pp = pr[q];
        }
      hp = lane_bcast(pp, owner);
      hc = lane_bcast(cc, owner);
    }
    VS_TRX(43);
    if (L == 0) {
      const double tol = 1e-6 * z;
      if (fabs(hc - uz) < tol || (j >= 1 && fabs(hc - hp - uz) < tol)) flags |= VS_OUT_DRAW_BOUNDARY;
      s.misc[1] = (int)key_index(a[j]);
      s.misc[2] = keep;
      s.misc[3] = (int)flags;
      s.redf[0] = log_ratio(hp, z);
    }
  }
}
// sampler.py:141-156 on n <= 256 keys sorted descending in LDS (see wave_sample_em); all threads call it.
__device__ __forceinline__ Final wave_sample(const Smem& s, const u64* a, int n, const vs_row_params& P) {
  if (threadIdx.x < WAVE) {
    if (n <= WAVE) wave_sample_em<1>(s, a, n, P);
    else if (n <= 2 * WAVE) wave_sample_em<2>(s, a, n, P);
    else wave_sample_em<4>(s, a, n, P);
  }
  __syncthreads();
  Final f;
  f.token = s.misc[1];
  f.keep = s.misc[2];
  f.flags = (uint32_t)s.misc[3];
  f.lp = (float)s.redf[0];
  __syncthreads();
  return f;
}


__device__ __forceinline__ int pow2_ceil(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// Descending order by rank: out[#{j : in[j] > in[i]}] = in[i] for ranks below kout (distinct keys get distinct
// ranks). T lanes of one wave share each key's comparisons (T = the largest power of two <= 64 with T * n <= SNT,
// at least 1); each lane reads 8 keys per step, so 8 LDS reads are in flight instead of one per loop trip.
// The caller has synchronised after writing `in`; ends with a barrier.
__device__ __forceinline__ void rank_sort(const u64* in, int n, u64* out, int kout) {
  // T = SNT / 2^ceil(log2 n), clamped to [1, 64]
  const int lg = n > 1 ? 32 - __builtin_clz((unsigned)(n - 1)) : 0;
  int T = lg >= 9 ? 1 : (SNT >> lg);
  T = T > 64 ? 64 : T;
  const int t = threadIdx.x;
  const int sub = t & (T - 1);
  const int step = 8 * T;
  for (int i0 = 0; i0 < n; i0 += SNT / T) {  // uniform trip count
    const int i = i0 + t / T;
    const u64 ki = in[i < n ? i : 0];
    int r = 0;
    for (int j0 = 0; j0 < n; j0 += step) {  // uniform trip count
      u64 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int j = j0 + u * T + sub;
        v[u] = in[j < n ? j : 0];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) r += (j0 + u * T + sub < n && v[u] > ki) ? 1 : 0;
    }
    if (T > 1) r += lane_xor<1>(r);
    if (T > 2) r += lane_xor<2>(r);
    if (T > 4) r += lane_xor<4>(r);
    if (T > 8) r += lane_xor<8>(r);
    if (T > 16) r += lane_xor<16>(r);
    if (T > 32) r += lane_xor<32>(r);
    if (sub == 0 && i < n && r < kout) out[r] = ki;
  }
  __syncthreads();
}

constexpr int SEGW = KEYS_CAP / SNW;  // per-wave candidate segment
// Bits of an ord32 value resolved by the ballot bisections that bound the k-th largest logit from below (sign,
// exponent and 7 mantissa bits).
constexpr int BOUND_BITS = 16;
// Key-area offset (u64 words) of the value-bin prefix sums: above what the final in-bin resolution uses
// (4352 words), 3 * 256 coarse + 3 * NSET * 256 fine words.
constexpr int PFX_OFF = 4352;
static_assert(PFX_OFF + 3 * NBIN * (1 + NSET) <= KEYS_CAP, "prefix sums fit the key area");
// Key-area layout of the value-bin path below the prefix sums: words 0-511 gathered keys, then from word 512 the
// fine-bin id of every chunk position (u16; 0xFFFF = not in the kept set).
constexpr int FID_OFF = 512;
static_assert(FID_OFF * 8 + EPT_MAX * SNT * 2 <= PFX_OFF * 8, "fine-bin ids fit below the prefix sums");

// Sort 64*E keys held by one wave descending (lane L holds positions L + 64*i in e[i]); the bitonic network is
// fully unrolled: partners at distance < 64 are exchanged across lanes (DPP / permlane), the others in-lane.
template <int E>
__device__ __forceinline__ void wave_sort_desc(u64 (&e)[E]) {
  const int L = lane_id();
#pragma unroll
  for (int k = 2; k <= 64 * E; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
        const int d = j / 64;
#pragma unroll
        for (int i = 0; i < E; ++i) {
          if ((i & d) == 0) {
            const int pos = L + 64 * i;
            const bool desc = (pos & k) == 0;
            const u64 a = e[i], b = e[i + d];
            const u64 mx = a > b ? a : b, mn = a > b ? b : a;
            e[i] = desc ? mx : mn;
            e[i + d] = desc ? mn : mx;
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < E; ++i) {
          const u64 o = lane_xor_rt(e[i], j);
          const int pos = L + 64 * i;
          const bool take_max = ((pos & k) == 0) == ((pos & j) == 0);
          e[i] = ((e[i] > o) == take_max) ? e[i] : o;
        }
      }
    }
  }
}

// Sorted copy of n <= 256 keys: out[r] = key of rank r for r < kout. One wave sorts (the others wait at the final
// barrier); larger n falls back to rank counting over the whole workgroup.
__device__ __forceinline__ void small_sort(const u64* in, int n, u64* out, int kout) {
  if (n > 256) {
    rank_sort(in, n, out, kout);
    return;
  }
  if (threadIdx.x < WAVE) {
    const int L = threadIdx.x;
    if (n <= 64) {
      u64 e[1] = {L < n ? in[L] : (u64)0};
      wave_sort_desc<1>(e);
      if (L < kout) out[L] = e[0];
    } else if (n <= 128) {
      u64 e[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) e[i] = L + 64 * i < n ? in[L + 64 * i] : (u64)0;
      wave_sort_desc<2>(e);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        if (L + 64 * i < kout) out[L + 64 * i] = e[i];
    } else {
      u64 e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = L + 64 * i < n ? in[L + 64 * i] : (u64)0;
      wave_sort_desc<4>(e);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (L + 64 * i < kout) out[L + 64 * i] = e[i];
    }
  }
  __syncthreads();
}

// Lower bound for the k-th largest logit of the workgroup, from the lane maxima (ord32 values, 0 for a lane with no
// finite logit): each wave finds its q-th largest lane maximum, q = min(ceil(k/8), its non-zero lanes), by a
// most-significant-bit-first radix select on ballots. Those q lanes of every wave hold values >= the smallest wave's
// result, so when the waves' q add up to >= k the workgroup has >= k logits >= L. L = 0 otherwise (no bound).
// nlanes = lanes holding a finite logit.
struct LaneBound {
  uint32_t L;
  int nlanes;
};
__device__ __forceinline__ LaneBound lane_max_bound(uint32_t tmax, int k, const Smem& s) {
  const int q = (k + SNW - 1) / SNW;
  const int nz = __popcll(__ballot(tmax != 0));
  const int got = nz < q ? nz : q;
  uint32_t wb = 0;
  if (got > 0) {
    // the top BOUND_BITS bits only: the result (low bits zero) is still a valid lower bound, within a factor of
    // 1 + 2^-7 of the exact q-th largest value, for half the dependent ballot steps
    for (int b = 31; b >= 32 - BOUND_BITS; --b) {
      const uint32_t c = wb | (1u << b);
      if ((int)__popcll(__ballot(tmax >= c)) >= got) wb = c;
    }
  }
  VS_TRX(37);
  const int w = threadIdx.x / WAVE;
  uint32_t* wbs = (uint32_t*)(s.misc + M_WB);
  if (lane_id() == 0) {
    wbs[w] = wb;
    s.redi[w] = got;
    s.misc[M_NZ + w] = nz;
  }
  __syncthreads();
  VS_TRX(38);
  LaneBound r;
  uint32_t L = ~0u;
  int tot = 0, nl = 0;
  int gw[SNW], nw[SNW];
  uint32_t bw[SNW];
#pragma unroll
  for (int i = 0; i < SNW; ++i) {  // all reads first, then selects (a guarded read becomes a branch per wave)
    gw[i] = s.redi[i];
    nw[i] = s.misc[M_NZ + i];
    bw[i] = wbs[i];
  }
#pragma unroll
  for (int i = 0; i < SNW; ++i) {
    tot += gw[i];
    nl += nw[i];
    const uint32_t b = gw[i] > 0 ? bw[i] : ~0u;
    L = b < L ? b : L;
  }
  __syncthreads();
  r.L = tot >= k ? L : 0u;
  r.nlanes = nl;
  return r;
}

// One LDS exchange for the per-workgroup statistics: a sum, two 32-bit maxima and a 64-bit maximum.
struct Stats {
  int n;
  uint32_t mx1, mx2;
  u64 am;
};
__device__ __forceinline__ Stats block_stats(int n, uint32_t mx1, uint32_t mx2, const Smem& s) {
  n = wave_sum(n);
  mx1 = wave_max(mx1);
  mx2 = wave_max(mx2);
  const int w = threadIdx.x / WAVE;
  uint32_t* m1 = (uint32_t*)(s.misc + M_STAT1);
  uint32_t* m2 = (uint32_t*)(s.misc + M_STAT2);
  __syncthreads();
  if (lane_id() == 0) {
    s.redi[w] = n;
    m1[w] = mx1;
    m2[w] = mx2;
  }
  __syncthreads();
  Stats r = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < SNW; ++i) {
    r.n += s.redi[i];
    r.mx1 = m1[i] > r.mx1 ? m1[i] : r.mx1;
    r.mx2 = m2[i] > r.mx2 ? m2[i] : r.mx2;
  }
  __syncthreads();
  return r;
}

// The state entry point's Sampler.accept (sampler.py:75-79) and the draw's state advance, by the one thread that
// writes the row's result; the launch boundary orders it before the next call's reads.
__device__ __forceinline__ uint32_t commit_state(const SampleArgs& A, int r, int32_t token, uint32_t flags,
                                                 const vs_row_state& st, uint64_t rng_next) {
  if (!A.state || (flags & VS_OUT_TIMEOUT)) return flags;
  vs_row_state* S = A.state + (A.slots ? A.slots[r] : r);
  if (!(flags & (VS_OUT_GREEDY | VS_OUT_NOFINITE | VS_OUT_FORCED))) S->rng = rng_next;
  if (st.hist_len < st.hist_cap) {
    A.pool[st.hist_off + st.hist_len] = token;
    S->hist_len = st.hist_len + 1;
  } else {
    flags |= VS_OUT_HIST_FULL;
  }
  S->produced = st.produced + 1;
  return flags;
}

__device__ __forceinline__ void write_out(const SampleArgs& A, int row, const Final& f, const vs_row_state& st,
                                          uint64_t rng_next) {
  if (threadIdx.x == 0) {
    const int r = A.row0 + row;
    const uint32_t flags = commit_state(A, r, f.token, f.flags, st, rng_next);
    A.out_ids[r] = f.token;
    A.out_lp[r] = f.lp;
    if (A.out_flags) A.out_flags[r] = flags;
    if (A.out_keep) A.out_keep[r] = f.keep;
  }
}

// round(e * 2^S) to the nearest integer, ties to even, for a float 0 <= e <= 1 and 0 < S <= 63, in float
// arithmetic (sh = 2^(S - 32), sc = 2^S): h = trunc(e * sh) is the part of e * 2^S at and above 2^32 (an integral
// float, exact), and e * sc - h * 2^32 is the rest, exact because it is e's mantissa without its top bits. A rest
// with a fraction is below 2^24, so its rounding cannot carry into h. Equal to rint((double)e * 2^S).
__device__ __forceinline__ u64 fixed_mass(float e, float sh, float sc) {
  const float h = __builtin_truncf(e * sh);
  const float r = __builtin_fmaf(-h, 4294967296.0f, e * sc);
  return ((u64)(uint32_t)h << 32) | (u64)(uint32_t)__builtin_rintf(r);
}

// e^d for d <= 0 with about 2 ulp relative error: 2^(d log2 e) from the hardware base-2 exponential, with the
// rounding error of the product d * log2(e) (exact through an fma, plus the constant's own tail) applied as a
// first-order correction: e^d = 2^y * 2^(lo) ~ 2^y (1 + lo ln 2) for the tiny lo.
// `corr` is ln 2 for that correction (0 drops it: plain 2^(d L)).
__device__ __forceinline__ float exp_nonpos(float d, float corr = 0.693147180559945309f) {
  const float L = 1.44269502162933349609375f;  // log2(e) rounded to float
  const float Llo = 1.9259629891e-8f;          // log2(e) - L
  const float y = d * L;
  const float lo = fmaf(d, L, -y) + d * Llo;
  const float e = __builtin_amdgcn_exp2f(y);
  return fmaf(e, lo * corr, e);
}

// Sorted-id range search: first position in ids[b, e) with ids[p] >= x.
__device__ __forceinline__ int lower_bound_ids(const int32_t* ids, int b, int e, int32_t x) {
  while (b < e) {
    const int m = (b + e) >> 1;
    if (ids[m] < x)
      b = m + 1;
    else
      e = m;
  }
  return b;
}

template <int DT>
struct DTraits;
template <>
struct DTraits<VS_F32> {
  typedef float LT;
  static constexpr int VEC = 4;
  __device__ static float cv(LT v) { return v; }
};
template <>
struct DTraits<VS_BF16> {
  typedef uint16_t LT;
  static constexpr int VEC = 8;
  __device__ static float cv(LT v) { return bf16_to_f32(v); }
};
template <>
struct DTraits<VS_F16> {
  typedef uint16_t LT;
  static constexpr int VEC = 8;
  __device__ static float cv(LT v) { return f16_to_f32(v); }
};

// ---------------------------------------------------------------------------------------------------------------
// History counts (the counts Sampler.accept keeps, sampler.py:77-78) for the tokens in [lo, hi): cnt[tok - lo] += 1
// for every occurrence. The history is read as 16-byte vectors, HB per lane per batch, HD batches in flight; the
// first HD batches are loaded before the logits arrive.
// ---------------------------------------------------------------------------------------------------------------
constexpr int HB = 2;  // 16-byte vectors per lane per batch (8 ids)
struct HistWin {
  int64_t b, e, a, nv;  // [b, e): the ids; a: first 16-byte aligned position; nv: whole vectors from a
};
__device__ __forceinline__ HistWin hist_window(int64_t b, int64_t e) {
  HistWin w;
  w.b = b;
  w.e = e;
  w.a = (b + 3) & ~(int64_t)3;
  if (w.a > e) w.a = e;
  w.nv = (e - w.a) >> 2;
  return w;
}
// Loads vectors v0 + u * SNT (u < HB), the index clamped to the last vector so that every load is unconditional
// (conditional loads make the compiler wait for all loads at the loop latch); the consumer masks by position.
// Requires w.nv >= 1.
__device__ __forceinline__ void hist_load(const int32_t* h, const HistWin& w, int64_t v0, int4 (&r)[HB]) {
  const int4* hv = (const int4*)(h + w.a);
#pragma unroll
  for (int u = 0; u < HB; ++u) {
    const int64_t vi = v0 + (int64_t)u * SNT;
    r[u] = hv[vi < w.nv ? vi : w.nv - 1];
  }
}
// Count N ids per lane into cnt[id - lo] for the ids in [lo, hi).
template <int N>
__device__ __forceinline__ void hist_add_ids(const int32_t (&tk)[N], int lo, int hi, uint32_t* cnt) {
#pragma unroll
  for (int q = 0; q < N; ++q) {
    const uint32_t o = (uint32_t)(tk[q] - lo);
    if (o < (uint32_t)(hi - lo)) atomicAdd(&cnt[o], 1u);
  }
}
constexpr int HD = 4;  // batches in flight
// cnt[tok - lo] += 1 for every history id in [lo, hi).
__device__ __forceinline__ void hist_count(const int32_t* h, const HistWin& w, int4 (&r)[HD][HB], int lo, int hi,
                                           uint32_t* cnt) {
  const int t = threadIdx.x;
  {  // the unaligned head (< 4 ids) and tail (< 4 ids), one id per lane
    const int nh = (int)(w.a - w.b);
    const int64_t tb = w.a + w.nv * 4;
    const int nt = (int)(w.e - tb);
    int32_t one[1] = {-1};
    if (t < nh) one[0] = h[w.b + t];
    else if (t - nh < nt) one[0] = h[tb + (t - nh)];
    hist_add_ids(one, lo, hi, cnt);
  }
  constexpr int64_t BATCH = (int64_t)SNT * HB;  // vectors per batch
  // One group = HD batches: the first was loaded ahead of time; every later group issues all its loads before
  // counting (no registers carried across iterations, so the loads of a group are in flight together).
  auto take = [&](int64_t v0, int4 (&r)[HD][HB]) {
#pragma unroll
    for (int d = 0; d < HD; ++d) {
      const int64_t vb = v0 + d * BATCH;
      if (vb >= w.nv) break;  // uniform
      int32_t tk[4 * HB];
#pragma unroll
      for (int u = 0; u < HB; ++u) {
        const bool ok = vb + (int64_t)u * SNT + t < w.nv;
        tk[4 * u] = ok ? r[d][u].x : -1;
        tk[4 * u + 1] = ok ? r[d][u].y : -1;
        tk[4 * u + 2] = ok ? r[d][u].z : -1;
        tk[4 * u + 3] = ok ? r[d][u].w : -1;
      }
      hist_add_ids(tk, lo, hi, cnt);
    }
  };
  if (w.nv > 0) take(0, r);
  for (int64_t v0 = BATCH * HD; v0 < w.nv; v0 += BATCH * HD) {
    int4 q[HD][HB];
#pragma unroll
    for (int d = 0; d < HD; ++d) hist_load(h, w, v0 + d * BATCH + t, q[d]);
    take(v0, q);
  }
}

// fn(id) for every id of a history window whose whole vectors are all in the prefetched batches r (w.nv <= HD *
// SNT * HB); the unaligned head and tail ids are loaded again. Ids outside the window are not visited.
template <typename Fn>
__device__ __forceinline__ void hist_visit_prefetched(const int32_t* h, const HistWin& w, const int4 (&r)[HD][HB],
                                                      Fn fn) {
  const int t = threadIdx.x;
  {
    const int nh = (int)(w.a - w.b);
    const int64_t tb = w.a + w.nv * 4;
    const int nt = (int)(w.e - tb);
    if (t < nh) fn(h[w.b + t]);
    else if (t - nh < nt) fn(h[tb + (t - nh)]);
  }
  constexpr int64_t BATCH = (int64_t)SNT * HB;
#pragma unroll
  for (int d = 0; d < HD; ++d) {
    const int64_t vb = d * BATCH;
    if (vb >= w.nv) break;  // uniform
#pragma unroll
    for (int u = 0; u < HB; ++u) {
      if (vb + (int64_t)u * SNT + t < w.nv) {
        fn(r[d][u].x);
        fn(r[d][u].y);
        fn(r[d][u].z);
        fn(r[d][u].w);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Penalty counts given as a table (VS_ROW_HIST_PAIRS): n (id, count) pairs sorted by id with unique ids, the form of
// Sampler.counts (sampler.py:77-78, iterated at :113-122). A workgroup needs the entries with ids in [lo, hi) only.
// Thread t loads the id at entry pos(t) = t * n / SNT ahead (with the logits); the block counts the probes below lo
// (c0) and below hi (c1). Every entry with an id in [lo, hi) then lies in [pos(c0 - 1) + 1, pos(c1)) (pos(-1) = -1,
// pos(SNT) = n): at most 2 n / SNT entries beyond the wanted ones, which the range test of the edit skips.
// ---------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int64_t probe_at(int64_t n, int j) { return ((int64_t)j * n) / SNT; }

__device__ __forceinline__ void pair_range(int64_t n, int32_t probe, int lo, int hi, int* red, int64_t* r0,
                                           int64_t* r1) {
  const int w = threadIdx.x / WAVE;
  const int n0 = __popcll(__ballot(probe < lo)), n1 = __popcll(__ballot(probe < hi));
  if (lane_id() == 0) {
    red[w] = n0;
    red[SNW + w] = n1;
  }
  __syncthreads();
  int c0 = 0, c1 = 0;
#pragma unroll
  for (int i = 0; i < SNW; ++i) {
    c0 += red[i];
    c1 += red[SNW + i];
  }
  *r0 = c0 == 0 ? 0 : probe_at(n, c0 - 1) + 1;
  *r1 = c1 == SNT ? n : probe_at(n, c1);
}

template <int DT, bool XL>
__global__ __launch_bounds__(SNT) void vs_sample_kernel(SampleArgs A) {
  typedef DTraits<DT> TR;
  typedef typename TR::LT LT;
  constexpr int VEC = TR::VEC;
  constexpr int NVMAX = EPT_MAX / VEC;
  extern __shared__ __align__(16) char smem_raw[];
  const Smem s = carve(smem_raw, A.lds_ch);
  const int t = threadIdx.x;
  const int G = A.G;

  // blockIdx -> (row, chunk): consecutive workgroups are dealt round-robin to the 8 XCDs, so workgroups with equal
  // blockIdx % 8 share an XCD (and its L2). Give each row G workgroups of one XCD when the grid allows it.
  const int nb = gridDim.x, b = blockIdx.x;
  const int l = (nb % 8 == 0) ? (b % 8) * (nb / 8) + b / 8 : b;
  const int row = l / G, g = l % G;
  const int grow = A.row0 + row;
  const int srow = A.slots ? A.slots[grow] : grow;  // the request's params and state
  vs_row_params P;
  if (A.params) {
    P = A.params[srow];
  } else {  // top-list mode: plain logits, top_k = list_k, no edits
    P = vs_row_params{1.0f, 1.0f, 0.0f, 0.0f, A.list_k, 0u, 1.0, 0.0, 0.0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  }
  // state entry point: the draw, the history range and the stop mask come from the request's device state
  vs_row_state st = {};
  uint64_t rng_next = 0;
  if (A.state) st = A.state[srow];
  // a token forced by the reasoning budget (sampler.py:88-90): the logits are not read, no draw is consumed
  if (__builtin_expect((P.flags & VS_ROW_FORCE) != 0, 0)) {
    if (g == 0) {
      Final f;
      f.token = P.force_token;
      f.lp = 0.0f;
      f.flags = VS_OUT_FORCED;
      f.keep = 0;
      write_out(A, row, f, st, 0);
    }
    return;
  }
  if (A.state) {
    rng_next = xorshift64s_step(st.rng);
    P.u = xorshift64s_uniform(rng_next);
    // the penalty counts: the table (history up to hist_base) plus the tokens recorded since
    P.hist_begin = st.hist_off + st.hist_base;
    P.hist_end = st.hist_off + st.hist_len;
    if (st.produced >= st.min_new_tokens) P.stop_end = P.stop_begin;
  }
  const int64_t tlen = (A.state && A.tabs) ? st.tab_len : 0;  // table entries of a state row
  char* rws = A.ws + (size_t)row * ROW_WS;
  RowCtl* ctl = (RowCtl*)rws;
  Part* parts = (Part*)(rws + OFF_PART);
  u64* cand = (u64*)(rws + OFF_CAND);
  u64* gather = (u64*)(rws + OFF_GATHER);
  HistSlot* hslots = (HistSlot*)(rws + OFF_HIST);
  u64* bflags = (u64*)(rws + OFF_FLAGS);
  const uint32_t epoch = ld_dev(&ctl->epoch);  // used at the row barriers and by the cleanup; lands with the logits
  // XL placement guard: each workgroup tags its partial with (epoch << 4) | the XCD it runs on, and whoever reads
  // the partials checks every tag against its own. A workgroup of the row on another XCD leaves a tag that is stale
  // (its store stayed in its own XCD's L2) or names that XCD, so the row is reported VS_OUT_TIMEOUT instead of
  // being resolved from data that could be stale (the host then repeats it with the device-coherent exchange). The
  // testing flag VS_DEBUG_FAKE_XCD_SPLIT makes every row's last workgroup claim the neighbouring XCD.
  uint32_t xcc = 0;
  if constexpr (XL) {
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 0xFu;
    if ((A.debug & VS_DEBUG_FAKE_XCD_SPLIT) && g == G - 1) xcc ^= 1u;
  }
  auto xtag = [&]() -> uint32_t { return (epoch << 4) | xcc; };

  const int V = A.V;
  // A request that needs no logits (sampler.py:96) reads only [0, vocab_valid) and takes no edits; with its stop
  // mask active it is an ordinary greedy row over the whole vocabulary (sampler.py:123-128).
  const bool argmax_vv = (P.flags & VS_ROW_ARGMAX_VV) && (P.flags & VS_ROW_GREEDY) && P.stop_end == P.stop_begin;
  const int vlim = argmax_vv ? min(V, P.vocab_valid) : V;
  if (argmax_vv) P.bias_end = P.bias_begin, P.supp_end = P.supp_begin, P.hist_end = P.hist_begin;
  const int lo = g * A.CH;
  const int hi = min(vlim, lo + A.CH);
  const int NV = A.NV;
  VS_TR_DECL(A);
  VS_TR(A, 0);
  VS_TRC(A, 30);

  // ---- load the chunk into VGPRs (one HBM read) ----
  float v[EPT_MAX];
  const LT* rowp = (const LT*)A.logits + (int64_t)grow * A.ld;
#pragma unroll
  for (int j = 0; j < NVMAX; ++j) {
    if (j < NV) {
      const int base = lo + (j * SNT + t) * VEC;
      if (A.vec_ok && base + VEC <= hi) {
        const uint4 raw = *(const uint4*)(rowp + base);
        const LT* e = (const LT*)&raw;
#pragma unroll
        for (int q = 0; q < VEC; ++q) v[j * VEC + q] = TR::cv(e[q]);
      } else {
#pragma unroll
        for (int q = 0; q < VEC; ++q) v[j * VEC + q] = (base + q < hi) ? TR::cv(rowp[base + q]) : __builtin_nanf("");
      }
    }
  }
  // ---- while the logits are in flight: the first batch of the history ids, and the count array cleared ----
  const float rep = P.repetition_penalty, fpen = P.frequency_penalty, ppen = P.presence_penalty;
  const bool pairs = (P.flags & VS_ROW_HIST_PAIRS) && !A.state;  // the state pool always holds raw ids
  const int64_t npairs = (P.hist_end - P.hist_begin) >> 1;
  const bool has_pen = A.has_hist && (pairs ? npairs > 0 : (P.hist_end > P.hist_begin || tlen > 0)) &&
                       (rep != 1.0f || fpen != 0.0f || ppen != 0.0f);
  HistWin hw;
  int4 hpre[HD][HB];
  // An (id, count) table (pairs, or a state row's table) of up to PAIRS_ALL entries is loaded whole with the logits,
  // PAIRS_ALL / SNT entries per thread, and each workgroup takes the entries of its range from registers; a longer
  // one is searched (probe: the id at entry t * n / SNT, loaded with the logits) and its bracket loaded after.
  const int2* tabp = (const int2*)(pairs ? A.hist + P.hist_begin : (tlen > 0 ? A.tabs + st.tab_off : nullptr));
  const int64_t tabn = pairs ? npairs : tlen;
  const bool tab_all = tabn > 0 && tabn <= PAIRS_ALL;
  int2 tabe[PAIRS_ALL / SNT];
  int32_t probe = 0;
  if (has_pen && tab_all) {
#pragma unroll
    for (int u = 0; u < PAIRS_ALL / SNT; ++u) {
      const int64_t i = (int64_t)u * SNT + t;
      tabe[u] = tabp[i < tabn ? i : 0];
      tabe[u].x = i < tabn ? tabe[u].x : -1;
    }
  } else if (has_pen && tabn > 0) {
    probe = tabp[probe_at(tabn, t)].x;
  }
  if (has_pen && pairs) {
  } else if (has_pen) {
    hw = hist_window(P.hist_begin, P.hist_end);
    if (hw.nv > 0) {
#pragma unroll
      for (int d = 0; d < HD; ++d) hist_load(A.hist, hw, (int64_t)d * SNT * HB + t, hpre[d]);
    }
    for (int i = t; i < A.CH / 4; i += SNT) ((uint4*)s.cnt)[i] = make_uint4(0, 0, 0, 0);
  }
#define ELEM(j, q) (lo + ((j) * SNT + t) * VEC + (q))
#define FOR_ELEMS(BODY)                                 \
  _Pragma("unroll") for (int j = 0; j < NVMAX; ++j) {   \
    if (j < NV) {                                       \
      _Pragma("unroll") for (int q = 0; q < VEC; ++q) { \
        const int e = ELEM(j, q);                       \
        if (e < hi) {                                   \
          float& x = v[j * VEC + q];                    \
          (void)x;                                      \
          BODY                                          \
        }                                               \
      }                                                 \
    }                                                   \
  }
  VS_TR(A, 1);

  // ---- the chunk moves to LDS (xv): the edits and every class read it from there with compact loops, which keeps
  // the code small enough for the instruction cache and frees the chunk's VGPRs ----
  FOR_ELEMS({ s.xv[e - lo] = x; })
  __syncthreads();
  VS_TR(A, 23);

  // ---- logit edits and penalties (sampler.py:104-126), float32 throughout, applied sparsely ----
  if (P.bias_end > P.bias_begin) {  // :104-109; ids sorted, equal ids in application order: one lane per run
    for (int p = P.bias_begin + t; p < P.bias_end; p += SNT) {
      const int id = A.bias_ids[p];
      if (id >= lo && id < hi && (p == P.bias_begin || A.bias_ids[p - 1] != id)) {
        float y = s.xv[id - lo];
        for (int q = p; q < P.bias_end && A.bias_ids[q] == id; ++q) y = y + A.bias_vals[q];
        s.xv[id - lo] = y;
      }
    }
    __syncthreads();
  }
  if (P.supp_end > P.supp_begin) {  // :110-112
    for (int p = P.supp_begin + t; p < P.supp_end; p += SNT) {
      const int id = A.mask_ids[p];
      if (id >= lo && id < hi) s.xv[id - lo] = -__builtin_inff();
    }
    __syncthreads();
  }
  if (has_pen && pairs && tab_all) {  // :113-122 over the (id, count) table: each entry edits its own logit
#pragma unroll
    for (int u = 0; u < PAIRS_ALL / SNT; ++u) {
      const int id = tabe[u].x;
      const int32_t c = tabe[u].y;
      if ((unsigned)(id - lo) < (unsigned)(hi - lo)) {
        float y = s.xv[id - lo];
        if (rep != 1.0f) {
          const float dv = y / rep, ml = y * rep;
          y = y > 0.0f ? dv : ml;
        }
        const float fc = fpen * (float)c;
        const float sub = fc + (c > 0 ? ppen : 0.0f);
        s.xv[id - lo] = y - sub;
      }
    }
    __syncthreads();
    VS_TR(A, 24);
  } else if (has_pen && pairs) {
    int64_t p0, p1;
    pair_range(npairs, probe, lo, hi, s.redi, &p0, &p1);
    VS_TR(A, 24);
    const int2* hp = (const int2*)(A.hist + P.hist_begin);  // hist_begin is even
    constexpr int PU = 4;  // entries per lane in flight
    for (int64_t p = p0 + t; p < p1; p += (int64_t)PU * SNT) {
      int2 e[PU];
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        const int64_t q = p + (int64_t)u * SNT;
        e[u] = hp[q < p1 ? q : p];
      }
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        const int id = e[u].x;
        const int32_t c = e[u].y;
        // the bracket's entries outside [lo, hi) (and repeats past its end) are skipped
        if (p + (int64_t)u * SNT < p1 && (unsigned)(id - lo) < (unsigned)(hi - lo)) {
          float y = s.xv[id - lo];
          if (rep != 1.0f) {
            const float dv = y / rep, ml = y * rep;
            y = y > 0.0f ? dv : ml;
          }
          const float fc = fpen * (float)c;
          const float sub = fc + (c > 0 ? ppen : 0.0f);
          s.xv[id - lo] = y - sub;
        }
      }
    }
    __syncthreads();
  } else if (has_pen && A.state && hw.nv <= (int64_t)HD * SNT * HB) {
    // A state row whose recent tokens are all prefetched: the recent tokens are counted, then each table entry of
    // the chunk edits its logit with its total count and clears the recent count of its id, then the first visit of
    // each id left among the recent tokens claims its count and edits (sampler.py:113-122). A table longer than
    // PAIRS_ALL is bracketed by the probes and its first entries loaded before the counting.
    constexpr int PU = 4;  // bracket entries per lane in flight
    int64_t p0 = 0, p1 = 0;
    int2 e[PU];
    const int2* tp = (const int2*)(A.tabs + st.tab_off);
    if (!tab_all && tlen > 0) {
      pair_range(tlen, probe, lo, hi, s.redi, &p0, &p1);
#pragma unroll
      for (int u = 0; u < PU; ++u) {
        const int64_t q = p0 + t + (int64_t)u * SNT;
        e[u] = tp[q < p1 ? q : 0];
      }
    }
    hist_count(A.hist, hw, hpre, lo, hi, s.cnt);
    __syncthreads();
    auto edit = [&](int i, uint32_t c) {
      float y = s.xv[i];
      if (rep != 1.0f) {
        const float dv = y / rep, ml = y * rep;
        y = y > 0.0f ? dv : ml;
      }
      const float fc = fpen * (float)c;
      s.xv[i] = y - (fc + ppen);
    };
    if (tab_all) {
#pragma unroll
      for (int u = 0; u < PAIRS_ALL / SNT; ++u)
        if ((unsigned)(tabe[u].x - lo) < (unsigned)(hi - lo)) {
          const int i = tabe[u].x - lo;
          edit(i, (uint32_t)tabe[u].y + s.cnt[i]);
          s.cnt[i] = 0;
        }
      __syncthreads();
    } else if (p1 > p0) {
      for (int64_t p = p0 + t; p < p1; p += (int64_t)PU * SNT) {
        if (p != p0 + t) {
#pragma unroll
          for (int u = 0; u < PU; ++u) {
            const int64_t q = p + (int64_t)u * SNT;
            e[u] = tp[q < p1 ? q : p];
          }
        }
#pragma unroll
        for (int u = 0; u < PU; ++u)  // the bracket's entries outside [lo, hi) are skipped
          if (p + (int64_t)u * SNT < p1 && (unsigned)(e[u].x - lo) < (unsigned)(hi - lo)) {
            const int i = e[u].x - lo;
            edit(i, (uint32_t)e[u].y + s.cnt[i]);
            s.cnt[i] = 0;
          }
      }
      __syncthreads();
    }
    hist_visit_prefetched(A.hist, hw, hpre, [&](int id) {
      if ((unsigned)(id - lo) < (unsigned)(hi - lo)) {
        const uint32_t c = atomicExch(&s.cnt[id - lo], 0u);
        if (c) edit(id - lo, c);
      }
    });
    __syncthreads();
    VS_TR(A, 24);
  } else if (has_pen) {  // :113-122 over the multiset of generated tokens
    hist_count(A.hist, hw, hpre, lo, hi, s.cnt);
    __syncthreads();
    if (tab_all) {  // a state row's table adds its counts (ids unique: plain updates after the counting above)
#pragma unroll
      for (int u = 0; u < PAIRS_ALL / SNT; ++u)
        if ((unsigned)(tabe[u].x - lo) < (unsigned)(hi - lo)) s.cnt[tabe[u].x - lo] += (uint32_t)tabe[u].y;
      __syncthreads();
    } else if (tlen > 0) {
      int64_t p0, p1;
      pair_range(tlen, probe, lo, hi, s.redi, &p0, &p1);
      const int2* tp = (const int2*)(A.tabs + st.tab_off);
      constexpr int PU = 4;
      for (int64_t p = p0 + t; p < p1; p += (int64_t)PU * SNT) {
        int2 e[PU];
#pragma unroll
        for (int u = 0; u < PU; ++u) {
          const int64_t q = p + (int64_t)u * SNT;
          e[u] = tp[q < p1 ? q : p];
        }
#pragma unroll
        for (int u = 0; u < PU; ++u)
          if (p + (int64_t)u * SNT < p1 && (unsigned)(e[u].x - lo) < (unsigned)(hi - lo)) s.cnt[e[u].x - lo] += (uint32_t)e[u].y;
      }
      __syncthreads();
    }
    VS_TR(A, 24);
    auto penalised = [&](float y, uint32_t c) -> float {
      if (rep != 1.0f) {
        const float dv = y / rep, ml = y * rep;  // both, then a select: no divergent branch
        y = y > 0.0f ? dv : ml;
      }
      const float cf = (float)c;
      const float fc = fpen * cf;
      const float sub = fc + ppen;
      return y - sub;
    };
    // Thread t owns positions t + SNT j of the counts (strided, so that a dense run of distinct tokens, as a
    // Zipf-like history puts at the low ids, spreads over every wave). It marks its non-zero ones in a bit mask and
    // visits only those, two per loop trip with both reads issued first: the loop runs as often as the busiest
    // lane of the wave has distinct tokens / 2, with no per-position branch.
    constexpr int NJ = EPT_MAX * SNT / SNT;  // the largest CH / SNT (CH <= EPT_MAX * SNT)
    static_assert(NJ <= 32, "one mask bit per owned position");
    // Reads are unconditional (a uniform guard would become a scalar branch per read); past CH they land in the
    // unused rest of the key area (NJ * SNT < 16384 words) and are masked out.
    uint32_t cv[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) cv[jj] = s.cnt[jj * SNT + t];
    __builtin_amdgcn_sched_barrier(0);  // all NJ reads in flight before the first test
    uint32_t mask = 0;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) mask |= (uint32_t)((cv[jj] != 0) & (jj * SNT < A.CH)) << jj;
    VS_TRX(34);
    while (mask) {
      const int ja = __builtin_ctz(mask);
      mask &= mask - 1;
      const bool two = mask != 0;
      const int jb = two ? __builtin_ctz(mask) : ja;
      mask &= mask - 1;
      const int ia = ja * SNT + t, ib = jb * SNT + t;
      const float ya = s.xv[ia], yb = s.xv[ib];
      const uint32_t ca = s.cnt[ia], cb = s.cnt[ib];
      const float za = penalised(ya, ca), zb = penalised(yb, cb);
      s.xv[ia] = za;
      if (two) s.xv[ib] = zb;
    }
    VS_TRX(35);
    __syncthreads();
    VS_TRX(36);
  }
  if (P.stop_end > P.stop_begin) {  // :123-126
    for (int p = P.stop_begin + t; p < P.stop_end; p += SNT) {
      const int id = A.mask_ids[p];
      if (id >= lo && id < hi) s.xv[id - lo] = -__builtin_inff();
    }
    __syncthreads();
  }
#define FOR_XV(BODY)                                              \
  _Pragma("unroll 4") for (int i_ = t; i_ < hi - lo; i_ += SNT) { \
    const int e = lo + i_;                                        \
    const float x = s.xv[i_];                                     \
    (void)e;                                                      \
    BODY                                                          \
  }
  // The chunk in LDS, four positions per lane at a time: the four reads are issued before any of them is used, so
  // branches in BODY do not serialise the LDS latency. Past the chunk's end a read lands on position 0 and is not
  // processed.
#define FOR_XV4(BODY)                                                                 \
  for (int i0_ = t; i0_ < hi - lo; i0_ += 4 * SNT) {                                 \
    float xq_[4];                                                                    \
    _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_) {                               \
      const int iq_ = i0_ + u_ * SNT;                                                \
      xq_[u_] = s.xv[iq_ < hi - lo ? iq_ : 0];                                       \
    }                                                                                \
    _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_) {                               \
      const int i_ = i0_ + u_ * SNT;                                                 \
      if (i_ < hi - lo) {                                                            \
        const int e = lo + i_;                                                       \
        const float x = xq_[u_];                                                     \
        BODY                                                                         \
      }                                                                              \
    }                                                                                \
  }
  // np.argmax key of the chunk; only needed when a whole row has no finite logit (sampler.py:131-132)
  auto chunk_amkey = [&]() -> u64 {
    u64 am = 0;
    FOR_XV({
      const u64 ka = amkey64(x, (uint32_t)e);
      am = ka > am ? ka : am;
    })
    return block_max<SNT>(am, s.red64);
  };
  VS_TR(A, 2);

  const int top_k = P.top_k;
  const int cls = (P.flags & VS_ROW_GREEDY) ? CLS_GREEDY : ((top_k >= 1 && top_k <= A.kmax) ? CLS_TOPK : CLS_FULL);
  int slot = 0;  // histogram slots used by this row (identical in all its workgroups)
  uint32_t nbar = 0;
  bool ok = true;

  // Arrive at the row's done counter; true in the last workgroup of the row.
  auto arrive_done = [&]() -> bool { return block_arrive(&ctl->done, (uint32_t*)&s.misc[8]) == (uint32_t)(G - 1); };
  // FULL rows: the arrival also reports whether this workgroup wrote the row's result and whether it timed out;
  // returns the counter before it
  auto arrive_full = [&](bool wrote, bool timed_out) -> uint32_t {
    return block_arrive(&ctl->done, (uint32_t*)&s.misc[8], 1u + (wrote ? 1u << 16 : 0u) + (timed_out ? 1u << 24 : 0u));
  };
  auto cleanup = [&](int nrounds) {
    // Only the last workgroup of the row gets here: restore the all-zero state of the row's workspace.
#pragma nounroll
    for (int r = 0; r < nrounds; ++r) {
      HistSlot* hs = hslots + r;
      if (t < NBIN) {
        st_dev(&hs->cnt[t], 0u);
        st_dev(&hs->fix[t], (u64)0);
        st_dev(&hs->f64[t], 0.0);
        st_dev(&hs->mk[t], (u64)0);
      }
    }
    constexpr int EPW = offsetof(RowCtl, epoch) / 4;
    if (t < (int)(sizeof(RowCtl) / 4)) st_dev(&((uint32_t*)ctl)[t], t == EPW ? epoch + 1u : 0u);
  };
  auto put_part = [&](u64 am, uint32_t nf, uint32_t kc, float mf, double se) {
    if (t == 0) {
      st_row<XL>(&parts[g].amkey, am);
      st_row<XL>(&parts[g].nfin, nf);
      st_row<XL>(&parts[g].kc, kc);
      st_row<XL>(&parts[g].mf, mf);
      st_row<XL>(&parts[g].se, se);
      if constexpr (XL) st_row<XL>(&parts[g].pad, xtag());
    }
  };
  // the timeout result of a row whose finishing workgroup found a partial from another XCD (or a stale one)
  auto split_final = [&]() {
    Final f;
    f.token = -1;
    f.lp = 0.0f;
    f.flags = VS_OUT_TIMEOUT;
    f.keep = 0;
    write_out(A, row, f, st, rng_next);
    __syncthreads();
    cleanup(0);
  };

  if (cls == CLS_GREEDY) {
    // ---- sampler.py:127-128: np.argmax(x), first maximum; logprob = log-softmax of the processed row ----
    // Every position of the lane read at once; a lane whose magnitudes stay below +inf's holds only finite logits:
    // its maximum by three-input instructions and the first position holding it by a backward sweep (positions
    // grow with u); a lane with a NaN or an infinity takes the exact loop (NaN ranks first, np.argmax).
    const int nel = hi - lo;
    const int t0 = t < nel ? t : 0;
    float xq[EPT_MAX];
#pragma unroll
    for (int u = 0; u < EPT_MAX; ++u) xq[u] = s.xv[t + u * SNT < nel ? t + u * SNT : t0];
    float best = -__builtin_inff();
    uint32_t mag = 0;
#pragma unroll
    for (int u = 0; u < EPT_MAX; u += 2) {
      best = max3f(best, xq[u], xq[u + 1]);
      mag = max3u(mag, __float_as_uint(xq[u]) & 0x7FFFFFFFu, __float_as_uint(xq[u + 1]) & 0x7FFFFFFFu);
    }
    u64 am = 0;
    float mf = -__builtin_inff();
    if (mag < 0x7F800000u) {
      if (t < nel) {
        int bu = 0;
#pragma unroll
        for (int u = EPT_MAX - 1; u >= 0; --u) bu = ((xq[u] == best) & (t + u * SNT < nel)) ? u : bu;
        am = amkey64(best, (uint32_t)(lo + t + bu * SNT));
        mf = best;
      }
    } else {
      FOR_XV({
        const u64 k = amkey64(x, (uint32_t)e);
        am = k > am ? k : am;
        if (is_finite(x)) mf = x > mf ? x : mf;
      })
    }
    {  // both maxima in one exchange
      am = wave_max(am);
      mf = wave_max(mf);
      const int w = t / WAVE;
      if (lane_id() == 0) {
        s.red64[w] = am;
        ((float*)s.redf)[w] = mf;
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < SNW; ++i) {
        const u64 ki = s.red64[i];
        const float mi = ((float*)s.redf)[i];
        am = ki > am ? ki : am;
        mf = mi > mf ? mi : mf;
      }
      __syncthreads();
    }
    // sum exp(x - mf) over the finite logits: exp2 of (x - mf) log2(e) per position, float sums per lane
    double se = 0.0;
    if (is_finite(mf)) {
      const float L2E = 1.44269504088896340736f;
      float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
      for (int u = 0; u < EPT_MAX; u += 2) {
        const float x0 = xq[u], x1 = xq[u + 1];
        s0 += __builtin_amdgcn_exp2f(((t + u * SNT < nel) & is_finite(x0)) ? (x0 - mf) * L2E : -__builtin_inff());
        s1 += __builtin_amdgcn_exp2f(((t + (u + 1) * SNT < nel) & is_finite(x1)) ? (x1 - mf) * L2E
                                                                                  : -__builtin_inff());
      }
      se = (double)s0 + (double)s1;
    }
    se = block_sum<SNT>(se, s.redf);
    put_part(am, 0, 0, mf, se);
    VS_TR(A, 3);
    if (arrive_done()) {
      VS_TR(A, 4);
      // last workgroup of the row: merge the G partials in one wave (G <= 64)
      if (t < WAVE) {
        u64 k = 0;
        float m = -__builtin_inff();
        double e = 0.0;
        bool bad = false;
        if (t < G) {
          k = ld_row<XL>(&parts[t].amkey);
          m = ld_row<XL>(&parts[t].mf);
          e = ld_row<XL>(&parts[t].se);
          if constexpr (XL) bad = ld_row<XL>(&parts[t].pad) != xtag();
        }
        const bool split = XL && __any(bad);  // a partial from another XCD (or a stale one): no result
        const u64 bam = wave_max(k);
        const float M = wave_max(m);
        const float L2E = 1.44269504088896340736f;
        const double S =
            wave_sum((e > 0.0 && is_finite(M)) ? e * (double)__builtin_amdgcn_exp2f((m - M) * L2E) : 0.0);
        if (split) {
          Final f;
          f.token = -1;
          f.lp = 0.0f;
          f.flags = VS_OUT_TIMEOUT;
          f.keep = 0;
          write_out(A, row, f, st, rng_next);
        } else if (t == 0) {
          const float xj = am_is_nan(bam) ? __builtin_nanf("") : key_value(bam);
          const int r = A.row0 + row;
          const uint32_t fl = commit_state(A, r, (int32_t)key_index(bam), VS_OUT_GREEDY, st, rng_next);
          A.out_ids[r] = (int32_t)key_index(bam);
          // log(S) = log1p(S - 1): S >= 1 holds the maximum's own term, so the float log1p keeps its relative
          // accuracy when one token dominates
          A.out_lp[r] = (is_finite(xj) && S > 0.0) ? (float)((double)xj - ((double)M + (double)log1pf((float)(S - 1.0))))
                                                   : 0.0f;
          if (A.out_flags) A.out_flags[r] = fl;
          if (A.out_keep) A.out_keep[r] = 0;
        }
      }
      cleanup(0);
    }
    VS_TR_FLUSH(A);
    return;
  }

  if (cls == CLS_TOPK) {
    // ---- local top-k by key among finite logits (sampler.py:133-136, ties toward the lower index) ----
    VS_TRX(17);
    const int k = top_k;
    if (t == 0) {
      s.misc[4] = 0;
      s.misc[9] = 0;
      s.misc[14] = 0;
    }
    // the lane's largest finite logit: a three-input maximum over every position read at once, unless the
    // magnitude bits show a NaN or an infinity (then the exact loop)
    float fmx = -__builtin_inff();
    bool hasf;
    float xq[EPT_MAX];  // the lane's positions t + SNT u (past the chunk: a repeat), kept for the candidate scan
    {
      const int nel = hi - lo;
      const int t0 = t < nel ? t : 0;
#pragma unroll
      for (int u = 0; u < EPT_MAX; ++u) xq[u] = s.xv[t + u * SNT < nel ? t + u * SNT : t0];  // no branch per read
      uint32_t mag = 0;
#pragma unroll
      for (int u = 0; u < EPT_MAX; u += 2) {
        fmx = max3f(fmx, xq[u], xq[u + 1]);
        mag = max3u(mag, __float_as_uint(xq[u]) & 0x7FFFFFFFu, __float_as_uint(xq[u + 1]) & 0x7FFFFFFFu);
      }
      hasf = t < nel;
      if (__builtin_expect(mag >= 0x7F800000u, 0)) {
        fmx = -__builtin_inff();
        hasf = false;
        FOR_XV({
          if (is_finite(x)) {
            hasf = true;
            fmx = fmaxf(fmx, x);
          }
        })
      }
    }
    const uint32_t tmax = hasf ? ord32(fmx) : 0u;  // ord32 of a finite value is never 0
    VS_TR(A, 10);
    // Only logits >= L can be in the local top-k (L = 0: no bound, every finite logit is a candidate).
    const LaneBound lb = lane_max_bound(tmax, k, s);
    VS_TR(A, 11);
    const u64 am = lb.nlanes ? (u64)0 : chunk_amkey();
    int kc = 0, C = 0;
    const int kr = pow2_ceil(k);  // sorted list length read by the merge (<= kcap)
    // Two list formats. Sorted: the local top-kc, zero padded to kr. Unsorted (when 8 G >= k, so that the row's
    // G * 8 heads can bound its k-th key): every candidate, zero padded to CP, and eight heads per workgroup (the
    // largest candidate of each wave), which spares the local rank sort; a workgroup with more than CP candidates
    // publishes its sorted top-kc instead (also a valid unsorted list, headed by its first eight keys).
    const bool ufmt = 8 * G >= k;
    const int CP = A.kcap < 4 * kr ? A.kcap : 4 * kr;  // a power of two
    bool listed = false;  // the candidates were published as they are
    if (lb.nlanes > 0) {
      const uint32_t L = lb.L;
      const float Lf = L ? inv_ord32(L) : -__builtin_inff();  // x >= Lf  <=>  ord32(x) >= L for finite x
      // Every candidate sits in a lane whose maximum reaches the bound (about k lanes), and each lane still holds
      // its positions in registers: a candidate mask per lane from compares alone, one wave scan for the offsets in
      // the wave's segment of the key area, then each lane stores its own candidates (a loop as long as the
      // busiest lane's count, usually one to three; no atomics, no block barrier).
      const int wv = t / WAVE, Ln = lane_id();
      const int nel = hi - lo;
      uint32_t cm = 0;
#pragma unroll
      for (int u = 0; u < EPT_MAX; ++u) {
        if (u % 4 == 0 && u * SNT >= nel) break;  // uniform: the chunk's positions end here
        cm |= (uint32_t)((xq[u] >= Lf) & (__builtin_fabsf(xq[u]) < __builtin_inff())) << u;
      }
      // positions past the chunk (repeats of the lane's first one) are not candidates
      const int npos = t < nel ? (nel - t + SNT - 1) / SNT : 0;
      cm &= npos >= 32 ? ~0u : (1u << npos) - 1u;
      const int nc = __builtin_popcount(cm);
      const int incl = wave_scan(nc);
      const int cw = __builtin_amdgcn_readlane(incl, WAVE - 1);
      int pos = incl - nc;
      u64* segw = s.keys + wv * SEGW;
      u64 lmx = 0;  // this lane's largest candidate key
      while (cm) {
        const int i = t + __builtin_ctz(cm) * SNT;
        cm &= cm - 1;
        const u64 kk = key64(s.xv[i], (uint32_t)(lo + i));
        if (pos < SEGW) segw[pos] = kk;
        lmx = kk > lmx ? kk : lmx;
        ++pos;
      }
      const u64 hwv = wave_max(lmx);  // the wave's head (0: no candidate)
      int* segc = s.misc + M_SEGC;  // [SNW] candidates per wave
      if (Ln == 0) {
        segc[wv] = cw;
        s.red64[8 + wv] = hwv;
      }
      __syncthreads();
      C = 0;
#pragma unroll
      for (int v = 0; v < SNW; ++v) C += segc[v];
      VS_TR(A, 12);
      VS_TRV(A, 19, C);
      kc = C < k ? C : k;
      if (ufmt && C <= CP) {
        // the unsorted list: each wave stores its segment at its offset (C <= CP <= kcap <= SEGW: none dropped)
        int off = 0;
#pragma unroll
        for (int v = 0; v < SNW; ++v) off += v < wv ? segc[v] : 0;
        for (int j = Ln; j < cw; j += WAVE) st_row<XL>(&cand[g * A.kcap + off + j], segw[j]);
        if (t < SNW) {  // the wave heads in descending order (equal ones, i.e. zeros, by wave): all 8 written
          const u64 hx = s.red64[8 + t];
          int rk = 0;
#pragma unroll
          for (int v = 0; v < SNW; ++v) {
            const u64 hy = s.red64[8 + v];
            rk += ((hy > hx) | ((hy == hx) & (v < t))) ? 1 : 0;
          }
          st_row<XL>(&parts[g].heads[rk], hx);
        }
        kc = C;
        listed = true;
      } else if (C <= RANK_MAX) {
        // the segments, made contiguous in the chunk area (no longer needed on this path), then ranked
        u64* ck = (u64*)s.xv;
        int off = 0;
#pragma unroll
        for (int v = 0; v < SNW; ++v) off += v < wv ? segc[v] : 0;
        for (int j = Ln; j < cw; j += WAVE) ck[off + j] = segw[j];
        __syncthreads();
        rank_sort(ck, C, s.tk, kc);  // the local top-k, sorted descending
      } else {
        // Many keys above the bound (few lanes hold finite values): radix select, then rank the k survivors.
        u64 T;
        {
          u64 prefix = 0;
          int shift = 56, krem = k;
          for (;;) {
            hist_clear(s);
            FOR_XV({
              if (is_finite(x)) {
                const u64 kk = key64(x, (uint32_t)e);
                if (prefix_match(kk, shift, prefix)) atomicAdd(&s.hc[(kk >> shift) & 0xFF], 1u);
              }
            })
            __syncthreads();
            const ScanOut o = hist_scan(s, true, (double)krem);
            const int need = krem - (int)o.cnt_before;
            const u64 np = (prefix << 8) | (u64)o.digit;
            if ((int)o.cnt == need || shift == 0) {
              T = np << shift;
              break;
            }
            krem = need;
            prefix = np;
            shift -= 8;
          }
        }
        if (t == 0) s.misc[5] = 0;
        __syncthreads();
        u64* sel = s.tk + KCAP;  // k <= KCAP survivors
        FOR_XV({
          if (is_finite(x)) {
            const u64 kk = key64(x, (uint32_t)e);
            if (kk >= T) {
              const int p = atomicAdd(&s.misc[5], 1);
              if (p < KCAP) sel[p] = kk;
            }
          }
        })
        __syncthreads();
        rank_sort(sel, kc, s.tk, kc);
      }
      VS_TR(A, 13);
    }
    if (listed) {
      for (int i = C + t; i < CP; i += SNT) st_row<XL>(&cand[g * A.kcap + i], (u64)0);
    } else {  // the sorted local top-kc, zero padded to kr (sorted format) or CP (unsorted format)
      const int plen = ufmt ? CP : kr;
      for (int i = t; i < plen; i += SNT) st_row<XL>(&cand[g * A.kcap + i], i < kc ? s.tk[i] : (u64)0);
      if (ufmt && t < 8) st_row<XL>(&parts[g].heads[t], t < kc ? s.tk[t] : (u64)0);
    }
    // C counts every finite logit when there is no bound, and is >= k otherwise: the row's sum decides
    // min(k, finite count) exactly.
    put_part(am, (uint32_t)C, (uint32_t)kc, 0.0f, 0.0);
    VS_TR(A, 3);
    if (arrive_done()) {
      VS_TR(A, 4);
      int n, keff;
      u64 bam;
      // ---- merge (last workgroup of the row). Each list holds its workgroup's candidates (unsorted format) or
      // sorted local top-kc, zero padded. A lower bound M of the row's keff-th key leaves few survivors >= M, which
      // are ranked; the bound, with r = ceil(k / G) heads per list (a sorted list's first r keys, or the first r of
      // an unsorted list's eight heads):
      //  * r <= 8: when >= keff heads are non-zero, M = the lowest key of the keff-th largest head value (>= keff
      //    heads, all keys of the row, are >= M, so its keff-th key is >= M), else 0;
      //  * otherwise (sorted lists): the smallest r-th key of the lists that hold >= r keys, valid when those
      //    lists number >= keff / r (they alone hold >= keff keys >= it), else 0.
      // Every wave loads the heads and list summaries and derives M itself (ballots over the heads), so the
      // survivors go straight from the registers to one LDS array: a single barrier before the rank. ----
      {
        const int plen = ufmt ? CP : kr;  // list stride read here (a power of two)
        const int lpl = __builtin_ctz((unsigned)plen);
        const int tot = G * plen;  // <= G * kcap <= KEYS_CAP
        const int r = (k + G - 1) / G;
        const int nh = G * r;  // heads: the first r keys (unsorted format: r <= 8 of its eight heads) of each list
        u64* sel = s.keys;  // survivors (<= tot)
        u64 r8[KEYS_CAP / SNT];  // all lists, loaded in one round trip
#pragma unroll
        for (int u = 0; u < KEYS_CAP / SNT; ++u) {
          const int idx = t + u * SNT;
          r8[u] = idx < tot ? ld_row<XL>(&cand[(idx >> lpl) * A.kcap + (idx & (plen - 1))]) : (u64)0;
        }
#ifdef VS_TRACE_WAITS
        publish_wait();
        VS_TRX(50);
#endif
        const int ln = lane_id();
        const bool hb8 = r <= 8;  // heads bound (else, sorted lists only, the smallest r-th key)
        int nf2 = 0, full = 0;
        u64 k2 = 0, h2 = ~(u64)0;
        const int hu = hb8 ? (nh + WAVE - 1) / WAVE : 0;  // head slots in use per lane (uniform)
        u64 hv[8];  // lane ln holds heads ln + 64 u (list h / r, place h % r)
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          hv[u] = 0;
          if (u < hu) {
            const int hx = ln + WAVE * u;
            const int hg = hx / r, hj = hx - hg * r;
            if (hx < nh) hv[u] = ld_row<XL>(ufmt ? &parts[hg].heads[hj] : &cand[hg * A.kcap + hj]);
          }
        }
        bool xbad = false;
        if (ln < G) {
          nf2 = (int)ld_row<XL>(&parts[ln].nfin);
          k2 = ld_row<XL>(&parts[ln].amkey);
          if constexpr (XL) xbad = ld_row<XL>(&parts[ln].pad) != xtag();
          if (!hb8) {
            full = (int)ld_row<XL>(&parts[ln].kc) >= r;
            const u64 h = ld_row<XL>(&cand[ln * A.kcap + r - 1]);
            h2 = full ? h : h2;
          }
        }
#ifdef VS_TRACE_WAITS
        publish_wait();
        VS_TRX(51);
#endif
        n = wave_sum(nf2);
        if constexpr (XL) {
          if (__any(xbad)) {  // every wave read the same tags: the whole workgroup takes this branch
            split_final();
            VS_TR_FLUSH(A);
            return;
          }
        }
        bam = wave_max(k2);
        keff = k < n ? k : n;  // sampler.py:133-134
        if (keff < 1) keff = 1;
        u64 M;
        if (hb8) {
          // th = the largest value with >= keff heads of value >= th (heads are keys of the row, so its keff-th
          // key is >= th's lowest key); bisection with ballots over the heads' value bits, most significant first
          uint32_t hh[8];
          int nzh = 0;
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            hh[u] = (uint32_t)(hv[u] >> 32);
            nzh += (int)__popcll(__ballot(hh[u] != 0));
          }
          uint32_t th = 0;  // the top BOUND_BITS bits: a lower bound just as valid (see lane_max_bound)
          if (hu == 1) {
#pragma unroll
            for (int b = 31; b >= 32 - BOUND_BITS; --b) {
              const uint32_t c = th | (1u << b);
              th = (int)__popcll(__ballot(hh[0] >= c)) >= keff ? c : th;
            }
          } else {
            for (int b = 31; b >= 32 - BOUND_BITS; --b) {
              const uint32_t c = th | (1u << b);
              int cnt = 0;
#pragma unroll
              for (int u = 0; u < 8; ++u) cnt += (int)__popcll(__ballot(hh[u] >= c));
              th = cnt >= keff ? c : th;
            }
          }
          M = nzh >= keff ? (u64)th << 32 : (u64)0;
        } else {
          const int nfull = wave_sum(full);
          const u64 mb = wave_min(h2);
          M = nfull * r >= keff ? mb : (u64)0;
        }
        VS_TRX(52);
        // a survivor is >= M and, in a sorted list, at a position below keff
        int cnt = 0;
#pragma unroll
        for (int u = 0; u < KEYS_CAP / SNT; ++u) {
          const u64 x = r8[u];
          cnt += ((x != 0) & (x >= M) & (ufmt | (((t + u * SNT) & (kr - 1)) < keff))) ? 1 : 0;
        }
        int p = wave_alloc(cnt, &s.misc[9]);
        if (cnt) {
#pragma unroll
          for (int u = 0; u < KEYS_CAP / SNT; ++u) {
            const u64 x = r8[u];
            if ((x != 0) & (x >= M) & (ufmt | (((t + u * SNT) & (kr - 1)) < keff))) sel[p++] = x;
          }
        }
        __syncthreads();
        const int Sv = s.misc[9];
        VS_TR(A, 14);
        if (n > 0) {
          if (Sv <= RANK_MAX) {
            rank_sort(sel, Sv, s.tk, keff);  // sampler.py:140 on the survivors
          } else {
            // many survivors (no useful bound): radix-select the keff-th key, then rank the keff keys above it
            if (t == 0) s.misc[10] = 0;
            __syncthreads();
            const u64 T = block_kth(s, sel, Sv, keff);
            u64* sel2 = (u64*)s.xv;
#pragma unroll
            for (int u = 0; u < KEYS_CAP / SNT; ++u)
              if (r8[u] != 0 && r8[u] >= T) sel2[atomicAdd(&s.misc[10], 1)] = r8[u];
            __syncthreads();
            rank_sort(sel2, keff, s.tk, keff);
          }
        }
        VS_TR(A, 6);
      }
      // top-list mode (vs_topk_batch): the sorted list, id -1 and value -inf past the row's finite logits
      auto write_list = [&](int have) {
        const int r = A.row0 + row;
        for (int i = t; i < A.list_k; i += SNT) {
          A.list_ids[(size_t)r * A.list_k + i] = i < have ? (int32_t)key_index(s.tk[i]) : -1;
          A.list_vals[(size_t)r * A.list_k + i] = i < have ? key_value(s.tk[i]) : -__builtin_inff();
        }
      };
      if (__builtin_expect(n == 0, 0)) {  // sampler.py:131-132
        if (A.list_k > 0) {
          write_list(0);
        } else {
          Final f;
          f.token = (int32_t)key_index(bam);
          f.lp = 0.0f;
          f.flags = VS_OUT_NOFINITE;
          f.keep = 0;
          write_out(A, row, f, st, rng_next);
        }
      } else if (A.list_k > 0) {
        write_list(keff);
      } else {
        const Final f = wave_sample(s, s.tk, keff, P);
        VS_TR(A, 7);
        write_out(A, row, f, st, rng_next);
      }
      cleanup(0);
    }
    VS_TR_FLUSH(A);
    return;
  }

  // =================================== FULL class ===================================
  // A workgroup that gives up at a row barrier skips everything after it. Work done after a barrier that every
  // workgroup contributes to (the gathers resolved by the row's last workgroup) is then incomplete, so the last
  // workgroup reports the row as timed out instead of resolving it (the host repeats the call cooperatively).
  // polls allowed at the row's nb-th barrier (the testing flag exempts the first)
  auto bar_limit = [&](uint32_t nb) -> uint32_t {
    return ((A.debug & VS_DEBUG_SPIN_LATER_BARRIERS) && nb < 2) ? 0xFFFFFFFFu : A.spin_limit;
  };
  // the testing flag VS_DEBUG_WAIT_CLOCK makes every row barrier unreachable, so each wait ends at the time bound
  auto bar_target = [&](uint32_t target) -> uint32_t { return (A.debug & VS_DEBUG_WAIT_CLOCK) ? 0xFFFFFFFFu : target; };
  // the row's next barrier: flag words in its XCD's L2 (XL) or the device-scope arrival counter
  auto rbar = [&]() -> bool {
    ++nbar;
    if constexpr (XL)
      return flag_barrier(bflags, g, G, ((u64)epoch << 32) | nbar, (A.debug & VS_DEBUG_WAIT_CLOCK) != 0, bar_limit(nbar),
                          A.spin_ticks, &s.misc[11]);
    else
      return row_barrier(&ctl->bar, bar_target(nbar * G), bar_limit(nbar), A.spin_ticks, &s.misc[11]);
  };
  auto timed_out_final = [&]() {
    Final f;
    f.token = -1;
    f.lp = 0.0f;
    f.flags = VS_OUT_TIMEOUT;
    f.keep = 0;
    write_out(A, row, f, st, rng_next);
    __syncthreads();
    cleanup(MAX_ROUNDS);
  };
  // ---- row statistics: finite count, largest and smallest finite logit, np.argmax key ----
  uint32_t lane_mk = 0;  // ord32 of this lane's largest finite logit, 0 when it has none
  {
    // Raw maximum and minimum by three-input instructions (reads past the chunk repeat the lane's first
    // position, which changes neither) and the largest magnitude bits: a lane whose magnitudes stay
    // below +inf's holds only finite logits, and its finite count is its position count. A lane with a NaN or an
    // infinity takes the exact loop.
    const int nel = hi - lo;
    const int t0 = t < nel ? t : 0;
    float fmx = -__builtin_inff(), fmn = __builtin_inff();
    uint32_t mag = 0;
    {
      static_assert(EPT_MAX % 2 == 0, "positions are taken in pairs");
      float xq[EPT_MAX];  // every read in flight at once (CH <= EPT_MAX * SNT)
#pragma unroll
      for (int u = 0; u < EPT_MAX; ++u) xq[u] = s.xv[t + u * SNT < nel ? t + u * SNT : t0];  // no branch per read
#pragma unroll
      for (int u = 0; u < EPT_MAX; u += 2) {
        fmx = max3f(fmx, xq[u], xq[u + 1]);
        fmn = min3f(fmn, xq[u], xq[u + 1]);
        mag = max3u(mag, __float_as_uint(xq[u]) & 0x7FFFFFFFu, __float_as_uint(xq[u + 1]) & 0x7FFFFFFFu);
      }
    }
    int nf = t < nel ? (nel - t + SNT - 1) / SNT : 0;
    if (__builtin_expect(mag >= 0x7F800000u, 0)) {
      nf = 0;
      fmx = -__builtin_inff();
      fmn = __builtin_inff();
      FOR_XV({
        if (is_finite(x)) {
          ++nf;
          fmx = x > fmx ? x : fmx;
          fmn = x < fmn ? x : fmn;
        }
      })
    }
    const uint32_t mk = nf ? ord32(fmx) : 0u, nmk = nf ? ~ord32(fmn) : 0u;
    lane_mk = mk;
    VS_TR(A, 20);
    Stats st = block_stats(nf, mk, nmk, s);
    if (__builtin_expect(st.n == 0, 0)) st.am = chunk_amkey();
    VS_TR(A, 21);
    if (t == 0) {
      if constexpr (XL) {  // each workgroup of the row reduces the G partials itself after the barrier
        st_row<XL>(&parts[g].amkey, st.am);
        st_row<XL>(&parts[g].nfin, (uint32_t)st.n);
        st_row<XL>(&parts[g].heads[0], st.n ? ((u64)st.mx1 << 32) | st.mx2 : (u64)0);
        st_row<XL>(&parts[g].pad, xtag());
      } else {
        if (st.n) {
          atomicAdd(&ctl->nfin, (uint32_t)st.n);
          atomicMax(&ctl->mkey, st.mx1);
          atomicMax(&ctl->nminkey, st.mx2);
        }
        atomicMax(&ctl->amkey, st.am);
      }
    }
  }
#ifdef VS_TRACE
  publish_wait();
  __syncthreads();
  VS_TR(A, 22);
#endif
  ok = rbar();
  VS_TR(A, 3);
  VS_TRC(A, 31);
  Final fin;
  fin.token = -1;
  fin.lp = 0.0f;
  fin.flags = VS_OUT_TIMEOUT;
  fin.keep = 0;
  bool g0_writes = true;  // false when the last workgroup of the row writes the result itself
  // the row statistics: reduced from the G partials (XL; a failed barrier leaves them unused), or the atomics' sums
  int n = 0;
  uint32_t mkey = 0, minkey = 0;
  u64 amk = 0;
  if constexpr (XL) {
    if (t < WAVE) {
      int nf = 0;
      u64 mm = 0, ak = 0;
      bool bad = false;
      if (t < G) {
        nf = (int)ld_row<XL>(&parts[t].nfin);
        mm = ld_row<XL>(&parts[t].heads[0]);
        ak = ld_row<XL>(&parts[t].amkey);
        bad = ld_row<XL>(&parts[t].pad) != xtag();
      }
      const bool anybad = __any(bad);
      nf = wave_sum(nf);
      const uint32_t m1 = wave_max((uint32_t)(mm >> 32)), m2 = wave_max((uint32_t)mm);
      ak = wave_max(ak);
      if (t == 0) {
        s.red64[0] = ak;
        s.red64[1] = ((u64)m1 << 32) | m2;
        s.red64[2] = (u64)nf;
        s.red64[3] = anybad ? 1u : 0u;
      }
    }
    __syncthreads();
    amk = s.red64[0];
    mkey = (uint32_t)(s.red64[1] >> 32);
    minkey = ~(uint32_t)s.red64[1];
    n = (int)s.red64[2];
    if (s.red64[3] != 0) ok = false;  // a partial from another XCD (or a stale one): the row reports VS_OUT_TIMEOUT
    __syncthreads();
  } else if (ok) {
    n = (int)ld_relaxed(&ctl->nfin);
    mkey = ld_relaxed(&ctl->mkey);
    minkey = ~ld_relaxed(&ctl->nminkey);
    amk = ld_relaxed64(&ctl->amkey);
  }
  if (ok) {
    if (__builtin_expect(n == 0, 0)) {  // sampler.py:131-132
      fin.token = (int32_t)key_index(amk);
      fin.flags = VS_OUT_NOFINITE;
    } else {
      int k = top_k > 0 ? (top_k < n ? top_k : n) : n;  // sampler.py:133-134
      if (k < 1) k = 1;
      const float tt = P.temperature;
      const float xs0 = inv_ord32(mkey) / tt;  // xs[0]: the maximum always survives
      int mode = 0;                            // 0 all finite, 1 key >= Tk, 2 exp(-40) filter
      u64 Tk = 0;
      float thr = 0.0f;
      float xs_lo = inv_ord32(minkey) / tt;  // smallest x/t of the kept set (a lower bound for mode 1)
      if (k < n) {
        // top-k with k beyond the TOPK class: cooperative count-weighted radix select (sampler.py:135-136)
        mode = 1;
        u64 prefix = 0;
        int shift = 56;
        int krem = k;
        for (;;) {
          hist_clear(s);
          FOR_XV({
            if (is_finite(x)) {
              const u64 kk = key64(x, (uint32_t)e);
              if (prefix_match(kk, shift, prefix)) atomicAdd(&s.hc[(kk >> shift) & 0xFF], 1u);
            }
          })
          __syncthreads();
          HistSlot* hs = hslots + slot;
          if (t < NBIN && s.hc[t]) atomicAdd(&hs->cnt[t], s.hc[t]);
          ok = rbar();
          if (!ok) break;
          if (t < NBIN) {
            s.hc[t] = ld_relaxed(&hs->cnt[t]);
            s.hfix[t] = 0;
            s.hf64[t] = 0.0;
            s.hmk[t] = 0;
          }
          __syncthreads();
          ++slot;
          const ScanOut o = hist_scan(s, true, (double)krem);
          const int need = krem - (int)o.cnt_before;
          const u64 np = (prefix << 8) | (u64)o.digit;
          if ((int)o.cnt == need || shift == 0) {
            Tk = np << shift;
            break;
          }
          krem = need;
          prefix = np;
          shift -= 8;
        }
        xs_lo = key_value(Tk) / tt;
      } else if (n > 4096) {
        mode = 2;  // sampler.py:137-139: keep x/t >= m/t - 40 (float32)
        thr = xs0 - 40.0f;
        xs_lo = xs_lo > thr ? xs_lo : thr;
      }
      // Every kept logit is >= xlb (mode 1: its key's value part; mode 2: a bound on x with fl(x/t) >= thr, from a
      // float64 product with a relative slack far above the rounding of the division). Lanes whose maximum is below
      // xlb hold no kept logit; when few lanes qualify, the passes below visit only their elements.
      // In mode 2 every x >= xhi passes as well, so the division only decides the few logits in [xlb, xhi).
      float xlb = -__builtin_inff(), xhi = __builtin_inff();
      if (mode == 1) {
        xlb = inv_ord32((uint32_t)(Tk >> 32));
      } else if (mode == 2 && tt > 0.0f) {
        const double d = (double)thr * (double)tt;  // exact: a product of two floats
        const double slack = fabs(d) * 0x1p-20 + (double)tt * 1e-44 + 1e-38;
        const float f = (float)(d - slack), f2 = (float)(d + slack);
        if (is_finite(f)) xlb = inv_ord32(ord32(f) - 1u);  // one more step covers the conversion's rounding
        if (is_finite(f2)) xhi = inv_ord32(ord32(f2) + 1u);
      }
      int* ql = (int*)(s.tk + KCAP);  // qualifying lanes (<= SNT)
      int nq = 0;
      if (ok) {
        if (t == 0) s.misc[14] = 0;
        __syncthreads();
        const bool qual = lane_mk != 0 && lane_mk >= ord32(xlb);
        const int pq = wave_append(qual, &s.misc[14]);
        if (qual) ql[pq] = t;
        __syncthreads();
        nq = s.misc[14];
      }
      // BODY runs for the chunk's logits x >= xlb (e = vocabulary index); it must not use wave-wide operations.
#define FOR_KEPT(BODY)                                                        \
  if (nq * 4 <= SNT) {                                                        \
    const int nel_ = hi - lo, M_ = (nel_ + SNT - 1) / SNT, tot_ = nq * M_;    \
    for (int w_ = t; w_ < tot_; w_ += SNT) {                                  \
      const int q_ = w_ / M_, m_ = w_ - q_ * M_;                              \
      const int i_ = ql[q_] + SNT * m_;                                       \
      if (i_ < nel_) {                                                        \
        const int e = lo + i_;                                                \
        const float x = s.xv[i_];                                             \
        if (x >= xlb) {                                                       \
          BODY                                                                \
        }                                                                     \
      }                                                                       \
    }                                                                         \
  } else {                                                                    \
    FOR_XV4({                                                                 \
      if (x >= xlb) {                                                         \
        BODY                                                                  \
      }                                                                       \
    })                                                                        \
  }
      if (ok) {
        // The per-element test of every pass: xs = x / t (float32, sampler.py:141, computed once and reused for
        // the bin and the mass), the key, and whether x is in the kept set; mode is uniform, combined with bit
        // operations so that no pass branches on it.
        auto keep_xs = [&](float x, int e, u64& kk, float& xs, auto unit_t) -> bool {
          xs = decltype(unit_t)::value ? x : x / tt;  // x / 1 == x exactly (signed zeros, infinities, NaN)
          kk = key64(x, (uint32_t)e);
          const bool m1 = (mode == 1) & (kk >= Tk);
          const bool m2 = (mode == 2) & ((x >= xhi) | (xs >= thr));
          return is_finite(x) & ((mode == 0) | m1 | m2);
        };
        // Value bins: u = xs0 - x/t >= 0 is monotone in the logit, so the fine index f = u * 65536 / span splits
        // the kept set, in sampler.py:140 order, into contiguous ranges. Bins are stored by digit 255 - c (coarse
        // c = f >> 8) and 255 - (f & 255) (fine), so that the 256-bin scan walks them in descending-logit order.
        const float span = xs0 - xs_lo;
        const float fscale = span > 0.0f ? 65536.0f / span : 0.0f;
        // The logprob's normaliser z (the kept mass, sampler.py:153) comes from the exact fixed-point sums when
        // every kept mass is >= exp(-span) >= 1e6 / scale: each mass then carries a relative rounding error
        // <= 5e-7, and so does every partial sum of them, far inside the logprob tolerance. Otherwise (masses down
        // to exp(-40)) the passes also keep float64 sums per bin.
        // Narrow rows (unit temperature, no top-k cut, span <= 4: near-flat rows such as
        // whole-vocabulary nucleus sampling) take a shorter value-bin pass: masses 2^(d log2 e) from the hardware
        // exponential without the product's correction term, in fixed point at 2^31, one LDS atomic per logit that
        // carries the count in bits 45 and up (a workgroup's count <= 12288 < 2^14 and mass sum < 12288 * 2^31 <
        // 2^45). Every mass is >= e^-4, so its relative error (the exponent's rounding, <= 2^-24 |d| log2 e, the
        // constant's tail and the instruction's own ulp, ~4e-7 together; the fixed point's half unit, 1.3e-8) stays
        // within the 5e-7 the fixed-point normaliser allows (below), and cumulative masses inherit that bound.
        const bool narrow = tt == 1.0f && mode != 1 && span <= 4.0f;  // row-uniform: every workgroup agrees
        const int fshift = narrow ? 31 : A.fix_shift;
        const double scale = __builtin_ldexp(1.0, fshift);
        const bool zfix_only = narrow || (double)span <= A.zspan_max;
        const double inv_scale = 1.0 / scale;  // a power of two: exact
        const float fsc = __builtin_amdgcn_ldexpf(1.0f, fshift), fsh = __builtin_amdgcn_ldexpf(1.0f, fshift - 32);
        constexpr float L2E_F = 1.44269502162933349609375f;  // log2(e) rounded to float
        auto fine_of = [&](float xs) -> int {  // xs = x / t
          const float u = xs0 - xs;
          int f = (int)(u * fscale);
          f = f < 1 ? 1 : (f > 65535 ? 65535 : f);
          return 65535 - f;  // (coarse digit << 8) | fine digit, at most 0xFFFE
        };
        // exp_nonpos's correction weight: 0 in narrow rows, whose masses are then the narrow pass's bit for bit
        // (fma(e, 0, e) == e, and fixed_mass at 2^31 is rint(e * 2^31))
        const float corr = narrow ? 0.0f : 0.693147180559945309f;
        auto mass = [&](float xs, u64* fx) -> double {  // pr = exp(float32(x/t - xs0)) (sampler.py:141-142)
          const float d = xs - xs0;
          const float e = exp_nonpos(d, corr);
          *fx = fixed_mass(e, fsh, fsc);  // == rint((double)e * scale)
          return (double)e;
        };
        VS_TR(A, 4);
        // ---- value-bin pass 1: coarse mass histogram of the kept set + its size + a bounded gather ----
        if (t == 0) s.misc[15] = 0;
        // every position's fine-bin id (0xFFFF = not kept), so that the later passes test a u16 per position
        uint16_t* fid = (uint16_t*)(s.keys + FID_OFF);
        // Visit the chunk positions whose fine-bin id satisfies PRED (a test on `id` alone, false for 0xFFFF): the
        // ids are read eight at a time (16-byte LDS reads, four in flight per lane) and tested without branches;
        // BODY runs for the (few) positions that pass, with i = the position in the chunk. The id array is
        // initialised to 0xFFFF over the whole chunk area, so the last group's tail never passes.
#define FOR_FID(PRED, BODY)                                                        \
  {                                                                                \
    const int n8_ = (hi - lo + 7) / 8;                                             \
    const uint4* f4_ = (const uint4*)fid;                                          \
    for (int w0_ = t; w0_ < n8_; w0_ += 4 * SNT) {                                 \
      uint4 q_[4];                                                                 \
      _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_) {                           \
        const int w_ = w0_ + u_ * SNT;                                             \
        q_[u_] = f4_[w_ < n8_ ? w_ : 0];                                           \
      }                                                                            \
      _Pragma("unroll") for (int u_ = 0; u_ < 4; ++u_) {                           \
        const int w_ = w0_ + u_ * SNT;                                             \
        const uint32_t wd_[4] = {q_[u_].x, q_[u_].y, q_[u_].z, q_[u_].w};          \
        uint32_t hm_ = 0;                                                          \
        _Pragma("unroll") for (int h_ = 0; h_ < 8; ++h_) {                         \
          const uint32_t id = (wd_[h_ >> 1] >> (16 * (h_ & 1))) & 0xFFFFu;         \
          hm_ |= (PRED) ? (1u << h_) : 0u;                                         \
        }                                                                          \
        hm_ = w_ < n8_ ? hm_ : 0u;                                                 \
        while (hm_) {                                                              \
          const int h_ = __builtin_ctz(hm_);                                       \
          hm_ &= hm_ - 1;                                                          \
          const int i = 8 * w_ + h_;                                               \
          const uint32_t id = (wd_[h_ >> 1] >> (16 * (h_ & 1))) & 0xFFFFu;         \
          (void)id;                                                                \
          BODY                                                                     \
        }                                                                          \
      }                                                                            \
    }                                                                              \
  }
        for (int v = t; v < A.CH / 8; v += SNT) ((uint4*)fid)[v] = make_uint4(~0u, ~0u, ~0u, ~0u);
        hist_clear(s);
        __syncthreads();
        // With few qualifying lanes the kept logits are also listed in LDS for the gather below; otherwise the
        // kept count exceeds GSMALL and no gather happens.
        const bool few = nq * 4 <= SNT && !narrow;  // narrow rows take the dense pass in every workgroup
        // one instance of the loop per zfix_only value, so that the float64 atomic is not a branch in it, and a
        // third for the dense case at unit temperature without float64 sums and without a top-k cut: no division,
        // and the kept set is x >= xkeep (finite), since x / 1 == x
        const float xkeep = mode == 2 ? fmaxf(xlb, fminf(xhi, thr)) : fmaxf(xlb, -__FLT_MAX__);
        auto pass1 = [&](auto with_f64, auto unit_t) -> int {
          int cnt = 0;
          if (!few) {
            // Dense case (many qualifying lanes): every position of the chunk, four LDS reads in flight per lane,
            // and no branch per logit: a logit outside the kept set adds nothing (a zero increment to a bin of
            // its own, so that it does not contend with the kept ones) and gets the id 0xFFFF.
            const int nel = hi - lo;
            for (int i0 = t; i0 < nel; i0 += 4 * SNT) {
              float xq[4];
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                const int iq = i0 + u * SNT;
                xq[u] = s.xv[iq < nel ? iq : 0];
              }
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * SNT;
                const float x = xq[u];
                u64 kk;
                float xs;
                bool keep;
                if constexpr (decltype(unit_t)::value) {  // mode 0 or 2 at unit temperature: one bound, finite
                  xs = x;
                  keep = (i < nel) & (x >= xkeep) & (x < __builtin_inff());
                } else {
                  keep = (i < nel) & (x >= xlb) & keep_xs(x, lo + i, kk, xs, unit_t);
                }
                u64 fx;
                const double pr = mass(xs, &fx);
                const int fo = fine_of(xs);
                if (i < nel) fid[i] = keep ? (uint16_t)fo : (uint16_t)0xFFFFu;
                const int c = fo >> 8;
                const int dmy = t & (NBIN - 1);
                atomicAdd(keep ? &s.hc[c] : &s.rc[dmy], keep ? 1u : 0u);
                atomicAdd(keep ? &s.hfix[c] : &s.rfix[dmy], keep ? fx : (u64)0);
                if constexpr (decltype(with_f64)::value) unsafeAtomicAdd(keep ? &s.hf64[c] : &s.rf64[dmy], keep ? pr : 0.0);
                cnt += keep ? 1 : 0;
              }
            }
            return cnt;
          }
          if constexpr (decltype(unit_t)::value) return cnt;  // only called dense
          FOR_KEPT({
            u64 kk;
            float xs;
            if (keep_xs(x, e, kk, xs, unit_t)) {
              ++cnt;
              u64 fx;
              const double pr = mass(xs, &fx);
              const int fo = fine_of(xs);
              fid[e - lo] = (uint16_t)fo;
              const int c = fo >> 8;
              atomicAdd(&s.hc[c], 1u);
              atomicAdd(&s.hfix[c], fx);
              if constexpr (decltype(with_f64)::value) unsafeAtomicAdd(&s.hf64[c], pr);
              if (few) {
                const int p = atomicAdd(&s.misc[15], 1);
                if (p < FID_OFF) s.keys[p] = kk;
              }
            }
          })
          return cnt;
        };
        // the narrow pass (see above): x / 1 == x, kept iff finite and x >= xkeep, bins and masses from d = x - xs0
        // (xs0 - x == -d exactly, so the fine bin equals fine_of's)
        auto pass1n = [&]() -> int {
          int cnt = 0;
          const int nel = hi - lo;
          const float nfs = -fscale;
          for (int i0 = t; i0 < nel; i0 += 4 * SNT) {
            float xq[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int iq = i0 + u * SNT;
              xq[u] = s.xv[iq < nel ? iq : 0];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const int i = i0 + u * SNT;
              const float x = xq[u];
              const bool keep = (i < nel) & (x >= xkeep) & (x < __builtin_inff());
              const float d = x - xs0;
              const uint32_t m = (uint32_t)__builtin_rintf(__builtin_amdgcn_exp2f(d * L2E_F) * 2147483648.0f);
              int f = (int)(d * nfs);
              f = f < 1 ? 1 : (f > 65535 ? 65535 : f);
              const int fo = 65535 - f;
              if (i < nel) fid[i] = keep ? (uint16_t)fo : (uint16_t)0xFFFFu;
              const int dmy = t & (NBIN - 1);
              atomicAdd(keep ? &s.hfix[fo >> 8] : &s.rfix[dmy], keep ? ((u64)1 << 45) | m : (u64)0);
              cnt += keep ? 1 : 0;
            }
          }
          return cnt;
        };
        const int cbr = narrow ? pass1n()
                        : !zfix_only ? pass1(std::true_type{}, std::false_type{})
                        : (!few && tt == 1.0f && mode != 1) ? pass1(std::false_type{}, std::true_type{})
                                                            : pass1(std::false_type{}, std::false_type{});
        int cb;
        if (few) {
          __syncthreads();
          cb = s.misc[15];
        } else {
          cb = block_sum<SNT>(cbr, s.redi);  // its barriers also order the pass's atomics before the unpacking
          if (narrow && t < NBIN) {  // count in bits 45 and up, mass below
            const u64 v = s.hfix[t];
            s.hc[t] = (uint32_t)(v >> 45);
            s.hfix[t] = v & (((u64)1 << 45) - 1);
          }
          if (narrow) __syncthreads();
        }
        VS_TR(A, 25);
        // each workgroup gathers into its own region of GB keys when its kept count fits
        const int GB = 1 << (31 - __builtin_clz(GCAP / G));  // power of two <= GCAP / G
        if (t == 0) {
          if constexpr (!XL) {
            atomicAdd(&ctl->gcount, (uint32_t)cb);
            atomicMax(&ctl->gmax, (uint32_t)cb);
          }
          st_row<XL>(&parts[g].kc, (uint32_t)cb);
        }
        if (cb <= GB && cb <= GSMALL) {
          if (!few) {  // rare: many lane maxima near the bound but few kept logits
            if (t == 0) s.misc[15] = 0;
            __syncthreads();
            FOR_KEPT({
              u64 kk;
              float xs;
              if (keep_xs(x, e, kk, xs, std::false_type{})) s.keys[atomicAdd(&s.misc[15], 1)] = kk;
            })
            __syncthreads();
          }
          for (int i = t; i < cb; i += SNT) st_row<XL>(&gather[g * GB + i], s.keys[i]);
        }
        VS_TR(A, 26);
        HistSlot* h1 = hslots + slot++;
        // XL rows with fixed-point sums only: each workgroup stores its whole coarse histogram in its own slot of
        // the row's list area (unused by this class), and every workgroup sums the G slots in workgroup order after
        // the barrier (integer sums: the same bits as the atomics). Otherwise the histograms meet in h1 by atomics.
        constexpr int PSLOT_G = (KEYS_CAP * 8) / (NBIN * 12);
        const bool pslot = XL && zfix_only && G <= PSLOT_G;
        u64* pfix = cand;                           // [G][NBIN]
        uint32_t* pcnt = (uint32_t*)(cand + G * NBIN);  // [G][NBIN]
        if (pslot) {
          if (t < NBIN) {
            st_row<XL>(&pfix[g * NBIN + t], s.hfix[t]);
            st_row<XL>(&pcnt[g * NBIN + t], s.hc[t]);
          }
        } else if (t < NBIN && s.hc[t]) {
          atomicAdd(&h1->cnt[t], s.hc[t]);
          atomicAdd(&h1->fix[t], s.hfix[t]);
          if (!zfix_only) unsafeAtomicAdd(&h1->f64[t], s.hf64[t]);
        }
        ok = rbar();
        if (ok) {
          int total, gmax;
          if constexpr (XL) {
            if (t < WAVE) {
              const int c = t < G ? (int)ld_row<XL>(&parts[t].kc) : 0;
              const int tot = wave_sum(c), mx = wave_max(c);
              if (t == 0) {
                s.redi[0] = tot;
                s.redi[1] = mx;
              }
            }
            __syncthreads();
            total = s.redi[0];
            gmax = s.redi[1];
            __syncthreads();
          } else {
            total = (int)ld_relaxed(&ctl->gcount);
            gmax = (int)ld_relaxed(&ctl->gmax);
          }
          VS_TR(A, 5);
          bool radix = false;
          if (total <= GSMALL && gmax <= GB) {
            // ---- small kept set: one workgroup ranks it and finishes as for TOPK ----
            if (g == 0) {
              int* offs = s.misc + M_OFFS;  // [G]
              int* cnts = s.misc + M_CNTS;  // [G]
              if (t < WAVE) {
                const int c = t < G ? (int)ld_row<XL>(&parts[t].kc) : 0;
                const int incl = wave_scan(c);
                if (t < G) {
                  offs[t] = incl - c;
                  cnts[t] = c;
                }
              }
              __syncthreads();
              {  // GCAP / SNT independent loads per lane, one round trip
                const int sh = __builtin_ctz(GB);  // GB is a power of two
                u64 r[GCAP / SNT];
#pragma unroll
                for (int u = 0; u < GCAP / SNT; ++u) {
                  const int idx = t + u * SNT;
                  r[u] = (idx < G * GB && (idx & (GB - 1)) < cnts[idx >> sh]) ? ld_row<XL>(&gather[idx]) : (u64)0;
                }
#pragma unroll
                for (int u = 0; u < GCAP / SNT; ++u) {
                  const int idx = t + u * SNT;
                  if (idx < G * GB && (idx & (GB - 1)) < cnts[idx >> sh]) s.keys[offs[idx >> sh] + (idx & (GB - 1))] = r[u];
                }
              }
              __syncthreads();
              VS_TR(A, 27);
              small_sort(s.keys, total, s.tk, total);
              VS_TR(A, 28);
              fin = wave_sample(s, s.tk, total, P);
              fin.flags |= VS_OUT_GATHER;
            }
          } else if (P.min_p > 0.0 || (A.debug & VS_DEBUG_FORCE_RADIX)) {
            radix = true;  // min-p on a large kept set: the radix path below handles it
          } else {
            // ---- large kept set: locate the top-p and draw positions by value bins ----
            if (pslot) {
              if (t < NBIN) {  // every slot's loads in flight at once (slots past G read slot 0 and are dropped)
                uint32_t cv[PSLOT_G];
                u64 fv[PSLOT_G];
#pragma unroll
                for (int q = 0; q < PSLOT_G; ++q) {
                  const int qq = q < G ? q : 0;
                  cv[q] = ld_row<XL>(&pcnt[qq * NBIN + t]);
                  fv[q] = ld_row<XL>(&pfix[qq * NBIN + t]);
                }
                uint32_t c = 0;
                u64 f = 0;
#pragma unroll
                for (int q = 0; q < PSLOT_G; ++q) {
                  c += q < G ? cv[q] : 0u;
                  f += q < G ? fv[q] : (u64)0;
                }
                s.hc[t] = c;
                s.hfix[t] = f;
                s.hf64[t] = 0.0;
              }
            } else if (t < NBIN) {
              s.hc[t] = ld_relaxed(&h1->cnt[t]);
              s.hfix[t] = ld_relaxed64(&h1->fix[t]);
              s.hf64[t] = zfix_only ? 0.0 : ld_relaxed_f64(&h1->f64[t]);
            }
            __syncthreads();
            // prefix sums of the coarse histogram (kept in the key area for every later lookup of this row)
            u64* cpc = s.keys + PFX_OFF;
            u64* cpw = cpc + NBIN;
            double* cpf = (double*)(cpw + NBIN);
            if (t < WAVE) hist_prefix(s.hc, s.hfix, s.hf64, cpc, cpw, cpf);
            __syncthreads();
            auto cfind = [&](double target) -> ScanOut {
              return hist_find(s.hc, s.hfix, s.hf64, cpc, cpw, cpf, target);
            };
            const u64 Sfix = cpw[0];
            const double Sf = zfix_only ? (double)Sfix * inv_scale : cpf[0] + s.hf64[0];
            VS_TRX(44);
            const bool has_tp = P.top_p < 1.0;
            const double tgt_p = P.top_p * (double)Sfix;
            ScanOut cpo;
            cpo.digit = -1;
            u64 zlo = Sfix, zhi = Sfix;
            if (has_tp) {
              cpo = cfind(tgt_p);
              zlo = cpo.fix_before;
              zhi = cpo.fix_before + cpo.fix;
            }
            const int dlo = cfind(P.u * (double)zlo).digit;
            const int dhi = cfind(P.u * (double)zhi).digit;
            // coarse digits to refine: the top-p bin and the draw's range dlo >= d >= dhi
            int set[NSET];
            int ns = 0;
            if (has_tp) set[ns++] = cpo.digit;
            for (int d = dlo; d >= dhi; --d) {
              if (has_tp && d == cpo.digit) continue;
              if (ns < NSET) set[ns] = d;
              ++ns;
            }
            VS_TRX(45);
            // kept logits of the row in the selected coarse bins (global counts)
            int ncand = 0;
#pragma unroll
            for (int q = 0; q < NSET; ++q) ncand += q < ns ? (int)s.hc[set[q]] : 0;
            const int bigcap = BIGCAP < A.lds_ch / 2 ? BIGCAP : A.lds_ch / 2;  // they must fit the chunk area
            if (__builtin_expect(ns > NSET, 0)) {
              radix = true;
            } else if (ncand <= bigcap) {
              // ---- the selected coarse bins hold few enough logits: gather them all, and let the row's last
              // workgroup resolve the top-p cut and the draw on its own (a fine histogram of the gathered keys, then
              // the exact key order inside the located fine bins), with no further row barrier ----
              static_assert(NSET == 4, "the coarse-bin test below names four set slots");
              int sd4[NSET];
#pragma unroll
              for (int q = 0; q < NSET; ++q) sd4[q] = q < ns ? set[q] : -1;
              u64* big = (u64*)(rws + OFF_BIG);
              if (t == 0) s.misc[16] = 0;
              __syncthreads();
              {
                // The selected coarse bins are the draw's digits dhi..dlo and the top-p digit: two ranges of fine-bin
                // ids [a, a + n), tested on two ids at once with 16-bit vector arithmetic (the difference wraps, so
                // an id below a is out of range too). n excludes 0xFFFF, the id of a logit outside the kept set.
                typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
                auto pk = [](uint32_t v) -> u16x2 { return __builtin_bit_cast(u16x2, v); };
                auto up = [](u16x2 v) -> uint32_t { return __builtin_bit_cast(uint32_t, v); };
                auto rng = [](int d0, int d1) -> uint32_t {  // (n << 16) | a for the digits d0..d1
                  return ((uint32_t)(((d1 - d0 + 1) << 8) - (d1 == 255 ? 1 : 0)) << 16) | ((uint32_t)d0 << 8);
                };
                const uint32_t r1 = rng(dhi, dlo);
                const uint32_t r2 = (has_tp && (cpo.digit < dhi || cpo.digit > dlo)) ? rng(cpo.digit, cpo.digit) : 0u;
                const u16x2 a1 = pk((r1 & 0xFFFFu) * 0x10001u), n1 = pk((r1 >> 16) * 0x10001u);
                const u16x2 a2 = pk((r2 & 0xFFFFu) * 0x10001u), n2 = pk((r2 >> 16) * 0x10001u);
                const u16x2 one = pk(0x10001u);
                static_assert(EPT_MAX * SNT / 8 <= 4 * SNT, "four 16-byte id words per lane cover the chunk");
                const int n8 = (hi - lo + 7) / 8;
                const uint4* f4 = (const uint4*)fid;
                uint4 q[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  const int w = t + u * SNT;
                  q[u] = f4[w < n8 ? w : 0];
                }
                // bit k (k < 16) / 16 + k: the low / high id of dword k = 4u + j of the lane's words; a half of
                // x1 | x2 is non-zero for an id in a range, and the saturating 1 - x marks the others
                uint32_t miss = 0;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  const uint32_t wd[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
                  for (int j = 0; j < 4; ++j) {
                    const u16x2 v = pk(wd[j]);
                    const uint32_t x1 = up(__builtin_elementwise_min((u16x2)(v - a1), n1)) ^ up(n1);
                    const uint32_t x2 = up(__builtin_elementwise_min((u16x2)(v - a2), n2)) ^ up(n2);
                    miss |= up(__builtin_elementwise_sub_sat(one, pk(x1 | x2))) << (4 * u + j);
                  }
                  if (t + u * SNT >= n8) miss |= 0x000F000Fu << (4 * u);
                }
                uint32_t hm = ~miss;
                const int nm = __builtin_popcount(hm);
                const int incl = wave_scan(nm);
                const int wtot = lane_bcast(incl, WAVE - 1);
                int wb = 0;
                if (lane_id() == 0 && wtot) wb = atomicAdd(&s.misc[16], wtot);
                wb = lane_bcast(wb, 0);
                __syncthreads();
                const int nloc = s.misc[16];
                if (t == 0 && nloc) s.misc[17] = (int)atomicAdd(&ctl->g2count, (uint32_t)nloc);
                __syncthreads();
                int p = (nloc ? s.misc[17] : 0) + wb + incl - nm;
                while (hm) {
                  const int bt = __builtin_ctz(hm);
                  hm &= hm - 1;
                  const int k = bt & 15;
                  const int i = 8 * (t + (k >> 2) * SNT) + 2 * (k & 3) + (bt >> 4);
                  st_row<XL>(&big[p++], key64(s.xv[i], (uint32_t)(lo + i)));
                }
              }
              g0_writes = false;
              VS_TR(A, 6);
              {
                const uint32_t old = arrive_full(false, false);
                if ((old & 0xFFFFu) != (uint32_t)(G - 1)) {
                  VS_TR_FLUSH(A);
                  return;
                }
                if (__builtin_expect((old >> 24) != 0, 0)) {  // a workgroup timed out and gathered nothing
                  timed_out_final();
                  VS_TR_FLUSH(A);
                  return;
                }
              }
              VS_TR(A, 7);
              // ---- final (last workgroup of the row): the gathered keys go to the chunk area, are histogrammed by
              // fine bin and placed in fine-bin order (an index array), so that each pick reads its bin's members
              // directly ----
              int m = (int)ld_relaxed(&ctl->g2count);
              m = m < bigcap ? m : bigcap;  // == ncand
              u64* bk = (u64*)s.xv;
              uint16_t* ord = (uint16_t*)s.keys;           // [BIGCAP] gathered positions in fine-bin order
              uint32_t* cur = (uint32_t*)(s.keys + 2048);  // [NSET * NBIN] per-bin placement cursors
              static_assert(BIGCAP * 2 <= 2048 * 8, "the order array stays below the cursors");
              static_assert(2048 + NSET * NBIN / 2 <= PFX_OFF, "the cursors stay below the prefix sums");
              for (int i = t; i < NSET * NBIN; i += SNT) {
                s.fc[i] = 0;
                s.ffix[i] = 0;
                s.ff64[i] = 0.0;
                cur[i] = 0;
              }
              constexpr int NL = (BIGCAP + SNT - 1) / SNT;
              int bb[NL];  // each held key's fine bin (set * NBIN + fine digit)
              {
                u64 r[NL];
#pragma unroll
                for (int u = 0; u < NL; ++u) {  // every load in flight at once
                  const int i = t + u * SNT;
                  r[u] = i < m ? ld_row<XL>(&big[i]) : (u64)0;
                }
                __syncthreads();  // the fine bins are clear
                VS_TRX(53);
                auto set_of = [&](int c) -> int { return sd4[1] == c ? 1 : (sd4[2] == c ? 2 : (sd4[3] == c ? 3 : 0)); };
#pragma unroll
                for (int u = 0; u < NL; ++u) {
                  const int i = t + u * SNT;
                  bb[u] = 0;
                  if (i < m) {
                    bk[i] = r[u];
                    const float xs = key_value(r[u]) / tt;
                    const int fo = fine_of(xs);
                    u64 fx;
                    const double pr = mass(xs, &fx);
                    const int b2 = set_of(fo >> 8) * NBIN + (fo & 0xFF);
                    bb[u] = b2;
                    atomicAdd(&s.fc[b2], 1u);
                    atomicAdd(&s.ffix[b2], fx);
                    if (!zfix_only) unsafeAtomicAdd(&s.ff64[b2], pr);
                  }
                }
              }
              __syncthreads();
              u64* fpc = cpc + 3 * NBIN;  // [NSET][NBIN] each
              VS_TRX(54);
              u64* fpw = fpc + NSET * NBIN;
              double* fpf = (double*)(fpw + NSET * NBIN);
              {
                const int j = t / WAVE;
                if (j < ns)
                  hist_prefix(s.fc + j * NBIN, s.ffix + j * NBIN, s.ff64 + j * NBIN, fpc + j * NBIN, fpw + j * NBIN,
                              fpf + j * NBIN);
              }
              __syncthreads();
              VS_TRX(55);
              // first position of fine bin b2 in the order array: the sets one after another, each in scan order
              auto bin_start = [&](int b2) -> int {
                const int j = b2 / NBIN;
                int base = 0;
#pragma unroll
                for (int q = 0; q < NSET; ++q) base += q < j ? (int)fpc[q * NBIN] : 0;
                return base + (int)(fpc[b2] - (u64)s.fc[b2]);
              };
#pragma unroll
              for (int u = 0; u < NL; ++u) {
                const int i = t + u * SNT;
                if (i < m) ord[bin_start(bb[u]) + (int)atomicAdd(&cur[bb[u]], 1u)] = (uint16_t)i;
              }
              __syncthreads();
              VS_TR(A, 27);
              struct BLoc {
                int id, set_j;
                u64 cnt_before, fix_before;
                double f64_before;
              };
              auto blocate = [&](double target) -> BLoc {
                BLoc r;
                const ScanOut co = cfind(target);
                int j = -1;
#pragma unroll
                for (int q = 0; q < NSET; ++q)
                  if (q < ns && sd4[q] == co.digit) j = q;
                r.set_j = j;
                r.cnt_before = co.cnt_before;
                r.fix_before = co.fix_before;
                r.f64_before = co.f64_before;
                r.id = co.digit << 8;
                if (j >= 0) {
                  const ScanOut fo = hist_find(s.fc + j * NBIN, s.ffix + j * NBIN, s.ff64 + j * NBIN, fpc + j * NBIN,
                                               fpw + j * NBIN, fpf + j * NBIN, target - (double)co.fix_before);
                  r.id |= fo.digit;
                  r.cnt_before += fo.cnt_before;
                  r.fix_before += fo.fix_before;
                  r.f64_before += fo.f64_before;
                }
                return r;
              };
              struct BPick {
                u64 key, cnt_in, fix_in, fix;
                double f64_in, f64;
              };
              // The first member (descending key) of the located fine bin whose cumulative mass inside the bin
              // reaches `tgt` (the bin's last member if none does, which only rounding can cause).
              // Up to 64 members: every wave computes it on its own, so no barrier is needed: lane L holds member L
              // and sums the masses of the members with larger keys (its rank in the bin; keys are distinct), one
              // member per trip read with readlane; the pick is the member whose mass crosses tgt, found by a
              // ballot. More: the whole workgroup, by a mass-weighted radix select.
              auto bpick = [&](const BLoc& lc, double tgt) -> BPick {
                BPick pk;
                pk.key = 0;
                pk.cnt_in = pk.fix_in = pk.fix = 0;
                pk.f64_in = pk.f64 = 0.0;
                if (lc.set_j < 0) return pk;
                const int b2 = lc.set_j * NBIN + (lc.id & 0xFF);
                const int nb = (int)s.fc[b2];
                const int st0 = bin_start(b2);
                if (nb <= WAVE) {
                  if (nb == 0) return pk;
                  const int L = lane_id();
                  const bool mem = L < nb;
                  const u64 kk = mem ? bk[ord[st0 + L]] : (u64)0;
                  u64 fx = 0;
                  double pr = 0.0;
                  if (mem) pr = mass(key_value(kk) / tt, &fx);
                  u64 ex = 0;  // mass of the larger keys
                  double exf = 0.0;
                  int rk = 0;  // their number
                  if (zfix_only) {
                    for (int j = 0; j < nb; ++j) {
                      const bool gt = lane_bcast(kk, j) > kk;
                      const u64 fj = lane_bcast(fx, j);
                      ex += gt ? fj : (u64)0;
                      rk += gt ? 1 : 0;
                    }
                  } else {
                    for (int j = 0; j < nb; ++j) {
                      const bool gt = lane_bcast(kk, j) > kk;
                      const u64 fj = lane_bcast(fx, j);
                      const double pj = lane_bcast(pr, j);
                      ex += gt ? fj : (u64)0;
                      exf += gt ? pj : 0.0;
                      rk += gt ? 1 : 0;
                    }
                  }
                  // in descending key order the inclusive sum first reaches tgt at one member: the first one, or
                  // the one whose exclusive sum is still below it (the last member, rank nb - 1, when none does)
                  const u64 tg = ceil_u64(tgt);
                  const unsigned long long hb = __ballot(mem & (ex + fx >= tg) & ((ex < tg) | (rk == 0)));
                  const unsigned long long lb = __ballot(mem & (rk == nb - 1));
                  const int ln = hb ? __ffsll((long long)hb) - 1 : __ffsll((long long)lb) - 1;
                  pk.key = lane_bcast(kk, ln);
                  pk.fix = lane_bcast(fx, ln);
                  pk.fix_in = lane_bcast(ex, ln);
                  pk.f64 = lane_bcast(pr, ln);
                  pk.f64_in = lane_bcast(exf, ln);
                  pk.cnt_in = (u64)lane_bcast(rk, ln);
                  return pk;
                }
                // many members (long runs of tied values): mass-weighted radix select on the 64-bit keys
                u64 prefix = 0;
                int shift = 56;
                for (;;) {
                  if (t < NBIN) {
                    s.rc[t] = 0;
                    s.rfix[t] = 0;
                    s.rf64[t] = 0.0;
                    s.rmk[t] = 0;
                  }
                  __syncthreads();
                  for (int q = t; q < nb; q += SNT) {
                    const u64 kk = bk[ord[st0 + q]];
                    if (prefix_match(kk, shift, prefix)) {
                      u64 fx;
                      const double pr = mass(key_value(kk) / tt, &fx);
                      const int d = (int)((kk >> shift) & 0xFF);
                      atomicAdd(&s.rc[d], 1u);
                      atomicAdd(&s.rfix[d], fx);
                      unsafeAtomicAdd(&s.rf64[d], pr);
                      atomicMax(&s.rmk[d], kk);
                    }
                  }
                  __syncthreads();
                  const ScanOut o = scan256(s, s.rc, s.rfix, s.rf64, s.rmk, false, tgt - (double)pk.fix_in);
                  pk.cnt_in += o.cnt_before;
                  pk.fix_in += o.fix_before;
                  pk.f64_in += o.f64_before;
                  if (o.cnt <= 1 || shift == 0) {
                    pk.key = o.mk;
                    pk.fix = o.fix;
                    pk.f64 = o.f64;
                    break;
                  }
                  prefix = (prefix << 8) | (u64)o.digit;
                  shift -= 8;
                }
                return pk;
              };
              uint32_t flags = VS_OUT_COOP | VS_OUT_GATHER;
              int keep = total;
              u64 zfix = Sfix;
              double zf = Sf;
              bool good = true;
              if (has_tp) {  // sampler.py:145-148
                const BLoc lp_ = blocate(tgt_p);
                VS_TRX(56);
                good = lp_.set_j >= 0;
                const BPick pp = bpick(lp_, tgt_p - (double)lp_.fix_before);
                VS_TRX(57);
                keep = (int)(lp_.cnt_before + pp.cnt_in) + 1;
                zfix = lp_.fix_before + pp.fix_in + pp.fix;
                zf = zfix_only ? (double)zfix * inv_scale : lp_.f64_before + pp.f64_in + pp.f64;
                const double tol = 1e-6 * (double)Sfix;
                if (fabs((double)(zfix - pp.fix) - tgt_p) < tol || fabs((double)zfix - tgt_p) < tol)
                  flags |= VS_OUT_TOPP_BOUNDARY;
              }
              // sampler.py:153-156
              const double tgt_d = P.u * (double)zfix;
              const BLoc ld = blocate(tgt_d);
              VS_TRX(58);
              good = good && ld.set_j >= 0;
              const BPick pd = bpick(ld, tgt_d - (double)ld.fix_before);
              VS_TRX(59);
              const float d = key_value(pd.key) / tt - xs0;
              const double before = (double)(ld.fix_before + pd.fix_in);
              const double tol = 1e-6 * (double)zfix;
              if (fabs(before - tgt_d) < tol || fabs(before + (double)pd.fix - tgt_d) < tol)
                flags |= VS_OUT_DRAW_BOUNDARY;
              // The draw range and the top-p bin are in the gathered set by construction (their coarse bins were
              // selected from bounds on z); a miss would be a defect, reported as an invalid row.
              fin.token = (int32_t)key_index(pd.key);
              fin.lp = (float)((double)d - log_ge1(zf));
              fin.keep = keep;
              fin.flags = good && pd.key != 0 ? flags : VS_OUT_TIMEOUT;
              VS_TR(A, 8);
              if (t < WAVE) write_out(A, row, fin, st, rng_next);  // every wave holds the same answer
              __syncthreads();
              cleanup(slot);
              VS_TR_FLUSH(A);
              return;
            } else {
              // ---- value-bin pass 2: fine histograms of the selected coarse bins ----
              for (int i = t; i < NSET * NBIN; i += SNT) {
                s.fc[i] = 0;
                s.ffix[i] = 0;
                s.ff64[i] = 0.0;
              }
              __syncthreads();
              VS_TRX(46);
              // the selected coarse digits, -1 for unused set slots (a valid id never has digit -1)
              static_assert(NSET == 4, "the fine-bin test below names four set slots");
              int sd4[NSET];
#pragma unroll
              for (int q = 0; q < NSET; ++q) sd4[q] = q < ns ? set[q] : -1;
              FOR_FID((id != 0xFFFFu) & (((int)(id >> 8) == sd4[0]) | ((int)(id >> 8) == sd4[1]) |
                                          ((int)(id >> 8) == sd4[2]) | ((int)(id >> 8) == sd4[3])),
                      {
                        const int c = (int)(id >> 8);
                        const int j = sd4[1] == c ? 1 : (sd4[2] == c ? 2 : (sd4[3] == c ? 3 : 0));
                        u64 fx;
                        const double pr = mass(s.xv[i] / tt, &fx);
                        const int b2 = j * NBIN + (int)(id & 0xFF);
                        atomicAdd(&s.fc[b2], 1u);
                        atomicAdd(&s.ffix[b2], fx);
                        if (!zfix_only) unsafeAtomicAdd(&s.ff64[b2], pr);
                      })
              __syncthreads();
              VS_TR(A, 15);
              HistSlot* h2 = hslots + slot;
              slot += ns;
              for (int i = t; i < ns * NBIN; i += SNT) {
                if (s.fc[i]) {
                  HistSlot* hs = h2 + i / NBIN;
                  const int b2 = i % NBIN;
                  atomicAdd(&hs->cnt[b2], s.fc[i]);
                  atomicAdd(&hs->fix[b2], s.ffix[i]);
                  if (!zfix_only) unsafeAtomicAdd(&hs->f64[b2], s.ff64[i]);
                }
              }
              VS_TR(A, 16);
              ok = rbar();
              VS_TR(A, 18);
              if (ok) {
                for (int i = t; i < ns * NBIN; i += SNT) {
                  const HistSlot* hs = h2 + i / NBIN;
                  const int b2 = i % NBIN;
                  s.fc[i] = ld_relaxed(&hs->cnt[b2]);
                  s.ffix[i] = ld_relaxed64(&hs->fix[b2]);
                  s.ff64[i] = zfix_only ? 0.0 : ld_relaxed_f64(&hs->f64[b2]);
                }
                __syncthreads();
                // prefix sums of each fine set, one wave per set
                u64* fpc = cpc + 3 * NBIN;  // [NSET][NBIN] each
                u64* fpw = fpc + NSET * NBIN;
                double* fpf = (double*)(fpw + NSET * NBIN);
                {
                  const int j = t / WAVE;
                  if (j < ns)
                    hist_prefix(s.fc + j * NBIN, s.ffix + j * NBIN, s.ff64 + j * NBIN, fpc + j * NBIN,
                                fpw + j * NBIN, fpf + j * NBIN);
                }
                __syncthreads();
                // Locate a target in the two-level histogram: the fine bin id and the sums before it.
                struct Loc {
                  int id, set_j;
                  u64 cnt_before, fix_before;
                  double f64_before;
                };
                auto locate = [&](double target) -> Loc {
                  Loc r;
                  const ScanOut co = cfind(target);
                  int j = -1;
#pragma unroll
                  for (int q = 0; q < NSET; ++q)
                    if (q < ns && set[q] == co.digit) j = q;
                  r.set_j = j;
                  r.cnt_before = co.cnt_before;
                  r.fix_before = co.fix_before;
                  r.f64_before = co.f64_before;
                  r.id = co.digit << 8;
                  if (j >= 0) {
                    const ScanOut fo = hist_find(s.fc + j * NBIN, s.ffix + j * NBIN, s.ff64 + j * NBIN,
                                                 fpc + j * NBIN, fpw + j * NBIN, fpf + j * NBIN,
                                                 target - (double)co.fix_before);
                    r.id |= fo.digit;
                    r.cnt_before += fo.cnt_before;
                    r.fix_before += fo.fix_before;
                    r.f64_before += fo.f64_before;
                  }
                  return r;
                };
                Loc lp_ = {-1, -1, 0, 0, 0.0};
                u64 z2lo = Sfix, z2hi = Sfix;
                if (has_tp) {
                  lp_ = locate(tgt_p);
                  z2lo = lp_.fix_before;
                  z2hi = lp_.fix_before + (lp_.set_j >= 0 ? (u64)s.ffix[lp_.set_j * NBIN + (lp_.id & 0xFF)] : (u64)0);
                }
                const Loc la = locate(P.u * (double)z2lo), lb = locate(P.u * (double)z2hi);
                // gather: the top-p fine bin and the fine bins la.id >= id >= lb.id
                int gcount = 0;
                bool located = la.set_j >= 0 && lb.set_j >= 0 && (!has_tp || lp_.set_j >= 0);
                if (located) {
                  for (int i = t; i < ns * NBIN; i += SNT) {
                    const int id = (set[i / NBIN] << 8) | (i % NBIN);
                    if ((has_tp && id == lp_.id) || (id <= la.id && id >= lb.id)) gcount += (int)s.fc[i];
                  }
                  gcount = block_sum<SNT>(gcount, s.redi);
                }
                if (!located || gcount > GCAP2) {
                  radix = true;
                } else {
                  if (t == 0) s.misc[16] = 0;
                  __syncthreads();
                  const int tpid = has_tp ? lp_.id : -1, laid = la.id, lbid = lb.id;
                  FOR_FID((id != 0xFFFFu) & (((int)id == tpid) | (((int)id <= laid) & ((int)id >= lbid))), {
                    const int p = atomicAdd(&s.misc[16], 1);
                    if (p < FID_OFF) s.keys[p] = key64(s.xv[i], (uint32_t)(lo + i));
                  })
                  __syncthreads();
                  const int nloc = s.misc[16];  // <= gcount <= GCAP2
                  if (t == 0 && nloc) s.misc[17] = (int)atomicAdd(&ctl->g2count, (uint32_t)nloc);
                  __syncthreads();
                  for (int i = t; i < nloc; i += SNT) st_row<XL>(&gather[s.misc[17] + i], s.keys[i]);
                  g0_writes = false;
                  VS_TR(A, 6);
                  {  // the last workgroup of the row resolves the exact positions
                    const uint32_t old = arrive_full(false, false);
                    if ((old & 0xFFFFu) != (uint32_t)(G - 1)) {
                      VS_TR_FLUSH(A);
                      return;
                    }
                    if (__builtin_expect((old >> 24) != 0, 0)) {  // a workgroup timed out and gathered nothing
                      timed_out_final();
                      VS_TR_FLUSH(A);
                      return;
                    }
                  }
                  VS_TR(A, 7);
                  // ---- final: exact key order inside the located fine bins ----
                  const int m = (int)ld_relaxed(&ctl->g2count);
                  if (m <= WAVE) {
                    // Few gathered keys (the usual case): one wave sorts them (descending key) and answers both
                    // picks with scans and ballots, no barrier. A fine bin's members are contiguous in key order,
                    // so the in-bin cumulative masses are masked scans of the sorted keys.
                    if (t < WAVE) {
                      u64 e1[1] = {t < m ? ld_row<XL>(&gather[t]) : (u64)0};
                      wave_sort_desc<1>(e1);
                      const u64 kk = e1[0];
                      const float xs = key_value(kk) / tt;
                      const int fi = kk != 0 ? fine_of(xs) : -1;
                      u64 fx = 0;
                      const double pr = kk != 0 ? mass(xs, &fx) : 0.0;
                      struct WPick {
                        u64 key, cnt_in, fix_in, fix;
                        double f64_in, f64;
                      };
                      // first member (descending key) of fine bin `id` whose in-bin cumulative mass reaches
                      // `tgt`, else the bin's last member
                      auto wpick = [&](int id, double tgt) -> WPick {
                        const bool mem = fi == id;
                        const u64 w = mem ? fx : (u64)0;
                        const double wf = mem ? pr : 0.0;
                        const u64 inc = wave_scan(w);
                        const double incf = wave_scan(wf);
                        const unsigned long long mm = __ballot(mem);
                        const unsigned long long hb = __ballot(mem & ((double)inc >= tgt));
                        const int ln = hb ? __ffsll((long long)hb) - 1 : (mm ? 63 - __clzll((long long)mm) : 0);
                        WPick pk;
                        pk.key = mm ? lane_bcast(kk, ln) : (u64)0;
                        pk.fix = mm ? lane_bcast(w, ln) : (u64)0;
                        pk.fix_in = mm ? lane_bcast(inc - w, ln) : (u64)0;
                        pk.f64 = mm ? lane_bcast(wf, ln) : 0.0;
                        pk.f64_in = mm ? lane_bcast(incf - wf, ln) : 0.0;
                        pk.cnt_in = (u64)__popcll(mm & ((1ull << ln) - 1ull));
                        return pk;
                      };
                      uint32_t flags = VS_OUT_COOP;
                      int keep = total;
                      u64 zfix = Sfix;
                      double zf = Sf;
                      if (has_tp) {  // sampler.py:145-148
                        const WPick pp = wpick(lp_.id, tgt_p - (double)lp_.fix_before);
                        keep = (int)(lp_.cnt_before + pp.cnt_in) + 1;
                        zfix = lp_.fix_before + pp.fix_in + pp.fix;
                        zf = zfix_only ? (double)zfix * inv_scale : lp_.f64_before + pp.f64_in + pp.f64;
                        const double tol = 1e-6 * (double)Sfix;
                        if (fabs((double)(zfix - pp.fix) - tgt_p) < tol || fabs((double)zfix - tgt_p) < tol)
                          flags |= VS_OUT_TOPP_BOUNDARY;
                      }
                      // sampler.py:153-156
                      const double tgt_d = P.u * (double)zfix;
                      const Loc ld = locate(tgt_d);
                      const WPick pd = wpick(ld.id, tgt_d - (double)ld.fix_before);
                      const float d = key_value(pd.key) / tt - xs0;
                      const double before = (double)(ld.fix_before + pd.fix_in);
                      const double tol = 1e-6 * (double)zfix;
                      if (fabs(before - tgt_d) < tol || fabs(before + (double)pd.fix - tgt_d) < tol)
                        flags |= VS_OUT_DRAW_BOUNDARY;
                      fin.token = (int32_t)key_index(pd.key);
                      fin.lp = (float)((double)d - log_ge1(zf));
                      fin.keep = keep;
                      fin.flags = flags;
                      VS_TR(A, 8);
                      write_out(A, row, fin, st, rng_next);
                    }
                    __syncthreads();
                    cleanup(slot);
                    VS_TR_FLUSH(A);
                    return;
                  }
                  u64* fk = s.keys;
                  int* fi = (int*)(s.keys + GCAP2);
                  u64* fxs = s.keys + GCAP2 + GCAP2 / 2;
                  double* fds = (double*)(s.keys + 2 * GCAP2 + GCAP2 / 2);
                  u64* xch = (u64*)(s.misc + M_XCH);  // two 8-byte exchange slots
                  for (int i = t; i < m; i += SNT) {
                    const u64 kk = ld_row<XL>(&gather[i]);
                    const float x = key_value(kk);
                    fk[i] = kk;
                    const float xs = x / tt;
                    fi[i] = fine_of(xs);
                    fds[i] = mass(xs, &fxs[i]);
                  }
                  __syncthreads();
                  // First element (descending key) of fine bin `id` whose cumulative mass inside the bin reaches
                  // `tgt` (the last element of the bin if none does, which only rounding can cause).
                  struct Pick {
                    u64 key, cnt_in, fix_in, fix;
                    double f64_in, f64;
                  };
                  auto pick = [&](int id, double tgt) -> Pick {
                    // the bin's members, ranked by key (descending) with their masses, then prefix sums
                    int* mem = (int*)(s.keys + 2048);      // [GCAP2] member positions
                    u64* mkey = s.keys + 2304;             // [GCAP2] member keys (dense)
                    u64* sk = mkey + GCAP2;                // [GCAP2] sorted keys
                    u64* sf = sk + GCAP2;                  // [GCAP2] their fixed-point masses
                    double* sd = (double*)(sf + GCAP2);    // [GCAP2] their float64 masses
                    if (t == 0) s.misc[18] = 0;
                    __syncthreads();
                    for (int i0 = 0; i0 < m; i0 += SNT) {  // uniform trip count
                      const int i = i0 + t;
                      const bool in = i < m && fi[i] == id;
                      const int p = wave_append(in, &s.misc[18]);
                      if (in) {
                        mem[p] = i;
                        mkey[p] = fk[i];
                      }
                    }
                    __syncthreads();
                    const int nb = s.misc[18];
                    {  // rank of each member among the members: T lanes per member, 8 reads in flight per lane
                      const int lg = nb > 1 ? 32 - __builtin_clz((unsigned)(nb - 1)) : 0;
                      int T = lg >= 9 ? 1 : (SNT >> lg);
                      T = T > 64 ? 64 : T;
                      const int sub = t & (T - 1);
                      for (int q0 = 0; q0 < nb; q0 += SNT / T) {
                        const int q = q0 + t / T;
                        const u64 kq = mkey[q < nb ? q : 0];
                        int r = 0;
                        for (int j0 = 0; j0 < nb; j0 += 8 * T) {
                          u64 v[8];
#pragma unroll
                          for (int u = 0; u < 8; ++u) {
                            const int j = j0 + u * T + sub;
                            v[u] = mkey[j < nb ? j : 0];
                          }
#pragma unroll
                          for (int u = 0; u < 8; ++u) r += (j0 + u * T + sub < nb && v[u] > kq) ? 1 : 0;
                        }
                        if (T > 1) r += lane_xor<1>(r);
                        if (T > 2) r += lane_xor<2>(r);
                        if (T > 4) r += lane_xor<4>(r);
                        if (T > 8) r += lane_xor<8>(r);
                        if (T > 16) r += lane_xor<16>(r);
                        if (T > 32) r += lane_xor<32>(r);
                        if (sub == 0 && q < nb) {
                          const int i = mem[q];
                          sk[r] = kq;
                          sf[r] = fxs[i];
                          sd[r] = fds[i];
                        }
                      }
                    }
                    __syncthreads();
                    // inclusive prefix sums in key order (nb <= GCAP2 <= SNT: one position per thread)
                    const u64 myf = t < nb ? sf[t] : (u64)0;
                    const double myd = t < nb ? sd[t] : 0.0;
                    u64 totf;
                    double totd;
                    const u64 incf = block_scan<SNT>(myf, s.red64, &totf);
                    const double incd = block_scan<SNT>(myd, s.redf, &totd);
                    // the first position whose cumulative mass reaches tgt, else the last one
                    const int cand = (t < nb && (double)incf >= tgt) ? t : 0x7FFFFFFF;
                    int rs = block_min<SNT>(cand, s.redi);
                    if (rs == 0x7FFFFFFF) rs = nb - 1;
                    if (t == rs) {
                      xch[0] = incf - myf;
                      ((double*)xch)[1] = incd - myd;
                    }
                    __syncthreads();
                    Pick pk;
                    pk.key = nb ? sk[rs] : (u64)0;
                    pk.cnt_in = (u64)(rs > 0 ? rs : 0);
                    pk.fix_in = nb ? xch[0] : (u64)0;
                    pk.f64_in = nb ? ((double*)xch)[1] : 0.0;
                    pk.fix = nb ? sf[rs] : (u64)0;
                    pk.f64 = nb ? sd[rs] : 0.0;
                    __syncthreads();
                    return pk;
                  };
                  uint32_t flags = VS_OUT_COOP;
                  int keep = total;
                  u64 zfix = Sfix;
                  double zf = Sf;
                  if (has_tp) {  // sampler.py:145-148
                    const Pick pp = pick(lp_.id, tgt_p - (double)lp_.fix_before);
                    keep = (int)(lp_.cnt_before + pp.cnt_in) + 1;
                    zfix = lp_.fix_before + pp.fix_in + pp.fix;
                    zf = zfix_only ? (double)zfix * inv_scale : lp_.f64_before + pp.f64_in + pp.f64;
                    const double tol = 1e-6 * (double)Sfix;
                    if (fabs((double)(zfix - pp.fix) - tgt_p) < tol || fabs((double)zfix - tgt_p) < tol)
                      flags |= VS_OUT_TOPP_BOUNDARY;
                  }
                  // sampler.py:153-156
                  const double tgt_d = P.u * (double)zfix;
                  const Loc ld = locate(tgt_d);
                  const Pick pd = pick(ld.id, tgt_d - (double)ld.fix_before);
                  const float d = key_value(pd.key) / tt - xs0;
                  const double before = (double)(ld.fix_before + pd.fix_in);
                  const double tol = 1e-6 * (double)zfix;
                  if (fabs(before - tgt_d) < tol || fabs(before + (double)pd.fix - tgt_d) < tol)
                    flags |= VS_OUT_DRAW_BOUNDARY;
                  fin.token = (int32_t)key_index(pd.key);
                  fin.lp = (float)((double)d - log_ge1(zf));
                  fin.keep = keep;
                  fin.flags = flags;
                  VS_TR(A, 8);
                  write_out(A, row, fin, st, rng_next);
                  cleanup(slot);
                  VS_TR_FLUSH(A);
                  return;
                }
              }
            }
          }
          if (__builtin_expect(ok && radix, 0)) {
            // ---- radix fallback: cooperative mass-weighted radix select on the 64-bit keys ----
            hist_clear(s);
            FOR_KEPT({
              u64 kk;
              float xs;
              if (keep_xs(x, e, kk, xs, std::false_type{})) {
                u64 fx;
                const double pr = mass(xs, &fx);
                hist_add(s, kk, 56, fx, pr);
              }
            })
            __syncthreads();
            HistSlot* hr = hslots + slot++;
            if (t < NBIN && s.hc[t]) {
              atomicAdd(&hr->cnt[t], s.hc[t]);
              atomicAdd(&hr->fix[t], s.hfix[t]);
              unsafeAtomicAdd(&hr->f64[t], s.hf64[t]);
              atomicMax(&hr->mk[t], s.hmk[t]);
            }
            ok = rbar();
            if (ok) {
              auto load_slot = [&](HistSlot* hs) {
                if (t < NBIN) {
                  s.hc[t] = ld_relaxed(&hs->cnt[t]);
                  s.hfix[t] = ld_relaxed64(&hs->fix[t]);
                  s.hf64[t] = ld_relaxed_f64(&hs->f64[t]);
                  s.hmk[t] = ld_relaxed64(&hs->mk[t]);
                }
                __syncthreads();
              };
              load_slot(hr);
              const u64 Sfix = block_sum<SNT>(t < NBIN ? s.hfix[t] : (u64)0, s.red64);
              const double Sf = block_sum<SNT>(t < NBIN ? s.hf64[t] : 0.0, s.redf);
              // the first key (descending) whose inclusive cumulative mass reaches target
              struct Sel {
                u64 key, cnt_before, fix_before, fix;
                double f64_before, f64;
              };
              auto select = [&](double target) -> Sel {
                Sel r;
                r.key = 0;
                r.cnt_before = r.fix_before = r.fix = 0;
                r.f64_before = r.f64 = 0.0;
                load_slot(hr);
                u64 prefix = 0;
                int shift = 56;
                for (;;) {
                  const ScanOut o = hist_scan(s, false, target - (double)r.fix_before);
                  r.cnt_before += o.cnt_before;
                  r.fix_before += o.fix_before;
                  r.f64_before += o.f64_before;
                  if (o.cnt <= 1 || shift == 0) {
                    r.key = o.mk;
                    r.fix = o.fix;
                    r.f64 = o.f64;
                    return r;
                  }
                  prefix = (prefix << 8) | (u64)o.digit;
                  shift -= 8;
                  hist_clear(s);
                  FOR_KEPT({
                    u64 kk;
                    float xs;
                    if (keep_xs(x, e, kk, xs, std::false_type{}) && (kk >> (shift + 8)) == prefix) {
                      u64 fx;
                      const double pr = mass(xs, &fx);
                      hist_add(s, kk, shift, fx, pr);
                    }
                  })
                  __syncthreads();
                  HistSlot* hs = hslots + slot;
                  ++slot;
                  if (t < NBIN && s.hc[t]) {
                    atomicAdd(&hs->cnt[t], s.hc[t]);
                    atomicAdd(&hs->fix[t], s.hfix[t]);
                    unsafeAtomicAdd(&hs->f64[t], s.hf64[t]);
                    atomicMax(&hs->mk[t], s.hmk[t]);
                  }
                  ok = rbar();
                  if (!ok) return r;
                  load_slot(hs);
                }
              };
              int keep = total;
              u64 zfix = Sfix;
              double zf = Sf;
              uint32_t flags = VS_OUT_COOP;
              if (P.top_p < 1.0) {  // sampler.py:145-148
                const double tgt = P.top_p * (double)Sfix;
                const Sel a = select(tgt);
                if (ok) {
                  keep = (int)a.cnt_before + 1;
                  zfix = a.fix_before + a.fix;
                  zf = a.f64_before + a.f64;
                  const double tol = 1e-6 * (double)Sfix;
                  if (fabs((double)a.fix_before - tgt) < tol || fabs((double)zfix - tgt) < tol)
                    flags |= VS_OUT_TOPP_BOUNDARY;
                }
              }
              if (ok && P.min_p > 0.0) {  // sampler.py:149-152
                const double pthr = (1.0 / Sf) * P.min_p;
                int mc = 0;
                u64 mfx = 0;
                double mff = 0.0;
                FOR_KEPT({
                  u64 kk;
                  float xs;
                  if (keep_xs(x, e, kk, xs, std::false_type{})) {
                    u64 fx;
                    const double pr = mass(xs, &fx);
                    if (!(pr / Sf < pthr)) {
                      ++mc;
                      mfx += fx;
                      mff += pr;
                    }
                  }
                })
                mc = block_sum<SNT>(mc, s.redi);
                mfx = block_sum<SNT>(mfx, s.red64);
                mff = block_sum<SNT>(mff, s.redf);
                if (t == 0) {
                  atomicAdd(&ctl->mcnt, (uint32_t)mc);
                  atomicAdd(&ctl->mfix, mfx);
                  unsafeAtomicAdd(&ctl->mf64, mff);
                }
                ok = rbar();
                if (ok) {
                  const int cm = (int)ld_relaxed(&ctl->mcnt);
                  const int km = cm > 1 ? cm : 1;
                  if (km < keep) {
                    keep = km;
                    if (cm >= 1) {
                      zfix = ld_relaxed64(&ctl->mfix);
                      zf = ld_relaxed_f64(&ctl->mf64);
                    } else {
                      zfix = (u64)(scale + 0.5);
                      zf = 1.0;
                    }
                  }
                }
              }
              if (ok) {  // sampler.py:153-156
                const double tgt = P.u * (double)zfix;
                const Sel bsel = select(tgt);
                if (ok) {
                  const float d = key_value(bsel.key) / tt - xs0;
                  fin.token = (int32_t)key_index(bsel.key);
                  fin.lp = (float)((double)d - log_ge1(zf));
                  fin.keep = keep;
                  const double tol = 1e-6 * (double)zfix;
                  if (fabs((double)bsel.fix_before - tgt) < tol ||
                      fabs((double)(bsel.fix_before + bsel.fix) - tgt) < tol)
                    flags |= VS_OUT_DRAW_BOUNDARY;
                  fin.flags = flags;
                }
              }
            }
          }
        }
#undef FOR_KEPT
      }
    }
  }
#undef FOR_XV
#undef FOR_XV4
  VS_TR(A, 9);
  // In the small-gather case only workgroup 0 computed `fin`; in the radix and no-finite cases all agree. Its
  // result is complete even when another workgroup timed out at the last barrier (everything it reads was
  // published before that barrier).
  const bool wrote = g == 0 && g0_writes;
  if (wrote) write_out(A, row, fin, st, rng_next);
  const uint32_t old = arrive_full(wrote, !ok);
  if ((old & 0xFFFFu) == (uint32_t)(G - 1)) {
    const bool any_timeout = !ok || (old >> 24) != 0;
    if (any_timeout && !wrote && ((old >> 16) & 0xFFu) == 0) {
      // a workgroup timed out and nobody wrote the row's result: the others took a gather path and left its
      // resolution to the last workgroup, which is this timed-out one
      timed_out_final();
    } else {
      cleanup(any_timeout ? MAX_ROUNDS : slot);  // a timed-out row clears every histogram slot
    }
  }
  VS_TR_FLUSH(A);
#undef FOR_ELEMS
#undef ELEM
}

// =================================================================================================================
// Merge of the fused head-and-sample kernel (vs_lmhead.hip): one workgroup per row reads the head workgroups'
// partials and candidate lists (LSParts) and finishes Sampler.sample (sampler.py:127-156) as the TOPK and GREEDY
// classes of vs_sample_kernel do.
// =================================================================================================================
constexpr int LSM_SEL = LS_KMAX * LS_KMAX;  // survivors at most: the keff lists whose heads reach the bound

struct LSMArgs {
  const vs_row_params* params;
  int R, N, P;
  char* ws;
  int32_t* out_ids;
  float* out_lp;
  uint32_t* out_flags;
  int32_t* out_keep;
  unsigned long long* trace;  // development builds only (VS_TRACE); null otherwise
};

__global__ __launch_bounds__(SNT) void vs_lmhead_sample_merge_kernel(LSMArgs A) {
  __shared__ u64 sel[LSM_SEL];
  __shared__ u64 tk[LS_KMAX];
  __shared__ u64 red64[NRED];
  __shared__ double redf[NRED];
  __shared__ int misc[NMISC];
  __shared__ u64 bound;
  __shared__ int qlist[LS_KMAX + 1];  // the qualifying lists, then their number
  __shared__ float exf[SNW];
  __shared__ int exn[SNW], exz[SNW];
  __shared__ uint32_t hist1[256], hist2[256];  // list heads by the first / second byte of their value
  __shared__ int rsel[4];
  __shared__ int redi[NRED];
  const int pos = blockIdx.x, t = threadIdx.x, w = t / WAVE, ln = lane_id();
  VS_TR_DECL(A);
  VS_TR(A, 0);
  // Every load of the row at once, before its class is known: the parameters and, one per thread, the workgroups'
  // partials and list heads (the heads are used only by a top-k row).
  const vs_row_params P = A.params[pos];
  const LSParts q = ls_parts(A.ws, A.R);
  const size_t base = (size_t)pos * LS_PMAX;
  static_assert(LS_PMAX <= SNT, "one partial per thread");
  const bool in = t < A.P;
  const int ti = in ? t : 0;
  u64 hd = q.heads[base + ti];
  const u64 k0 = q.amkey[base + ti];
  const float m0 = q.mf[base + ti];
  const double s0 = q.se[base + ti];
  const uint32_t n0 = q.nfin[base + ti];
  hd = in ? hd : (u64)0;
  if (t < 256) {
    hist1[t] = 0;
    hist2[t] = 0;
  }
  int vlim;
  const int cls = ls_class(P, A.N, &vlim);
  auto out = [&](int32_t tok, float lp, uint32_t fl, int32_t keep) {
    VS_TR(A, 6);
    VS_TR_FLUSH(A);
    if (t == 0) {
      A.out_ids[pos] = tok;
      A.out_lp[pos] = lp;
      if (A.out_flags) A.out_flags[pos] = fl;
      if (A.out_keep) A.out_keep[pos] = keep;
    }
  };
  if (cls == LS_UNSUPPORTED) {
    out(-1, 0.0f, VS_OUT_UNSUPPORTED, 0);
    return;
  }
  // one exchange for the row's argmax key, maximum, finite count and non-empty lists
  {
    const u64 wa = wave_max(in ? k0 : (u64)0);
    const float wm = wave_max(in ? m0 : -__builtin_inff());
    const int wn = wave_sum(in ? (int)n0 : 0);
    const int wz = (int)__popcll(__ballot(hd != 0));
    if (ln == 0) {
      red64[w] = wa;
      exf[w] = wm;
      exn[w] = wn;
      exz[w] = wz;
    }
  }
  __syncthreads();
  u64 am = 0;
  float M = -__builtin_inff();
  int n = 0, nzh = 0;
#pragma unroll
  for (int i = 0; i < SNW; ++i) {
    am = red64[i] > am ? red64[i] : am;
    M = exf[i] > M ? exf[i] : M;
    n += exn[i];
    nzh += exz[i];
  }
  VS_TR(A, 1);
  if (cls == LS_GREEDY) {  // sampler.py:127-128 (or :95-96 over [0, vv)): first maximum, log-softmax there
    const float L2E = 1.44269504088896340736f;
    const double S = block_sum<SNT>(
        (in && s0 > 0.0 && is_finite(M)) ? s0 * (double)__builtin_amdgcn_exp2f((m0 - M) * L2E) : 0.0, redf);
    const float xj = am_is_nan(am) ? __builtin_nanf("") : key_value(am);
    out((int32_t)key_index(am),
        (is_finite(xj) && S > 0.0) ? (float)((double)xj - ((double)M + (double)log1pf((float)(S - 1.0)))) : 0.0f,
        VS_OUT_GREEDY, 0);
    return;
  }
  if (n == 0) {  // sampler.py:131-132: np.argmax of a row without finite logits
    out((int32_t)key_index(am), 0.0f, VS_OUT_NOFINITE, 0);
    return;
  }
  const int keff = cls < n ? cls : n;  // sampler.py:133-134
  // The bound T: the keff-th largest list head (heads are keys of the row, so its keff-th largest key reaches it),
  // to its 16-bit value prefix, found by a two-round radix select over the heads (one byte per round, every thread
  // holding one head); exact only when more than LS_KMAX heads share that prefix. Only the lists whose heads reach T
  // can hold keys >= T (<= LS_KMAX lists of LS_KMAX keys); their indices go to LDS.
  // Wave 0: the bin of a 256-bin histogram (bins visited from the top) where the count from the top first reaches
  // `need`, and the count above it.
  auto find_desc = [&](const uint32_t* h, int need) {
    if (t < WAVE) {
      uint32_t c[4];
      int tot = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c[j] = h[255 - 4 * ln - j];
        tot += (int)c[j];
      }
      const int incl = wave_scan(tot);
      int run = incl - tot, hit = -1, before = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (hit < 0 && run + (int)c[j] >= need) {
          hit = j;
          before = run;
        }
        run += (int)c[j];
      }
      const unsigned long long hb = __ballot(hit >= 0);
      const int L = hb ? __ffsll((long long)hb) - 1 : WAVE - 1;
      if (ln == L) {
        const int bin = hit >= 0 ? 255 - 4 * ln - hit : 0;
        rsel[0] = bin;
        rsel[1] = hit >= 0 ? before : 0;
        rsel[2] = (int)h[bin];
      }
    }
  };
  u64 T = 1;
  if (nzh >= keff) {
    if (hd) atomicAdd(&hist1[hd >> 56], 1u);
    __syncthreads();
    find_desc(hist1, keff);
    __syncthreads();
    const int b1 = rsel[0], above1 = rsel[1];
    if (hd && (int)(hd >> 56) == b1) atomicAdd(&hist2[(hd >> 48) & 0xFF], 1u);
    __syncthreads();
    find_desc(hist2, keff - above1);
    __syncthreads();
    const int b2 = rsel[0];
    T = ((u64)b1 << 56) | ((u64)b2 << 48);
    if (above1 + rsel[1] + rsel[2] > LS_KMAX) {
      // more than LS_KMAX heads share the prefix: the exact keff-th head, bit by bit below it (rare: long runs of
      // equal logits)
      for (int b = 47; b >= 0; --b) {
        const u64 c = T | ((u64)1 << b);
        T = block_sum<SNT>(hd >= c ? 1 : 0, redi) >= keff ? c : T;
      }
    }
  }
  if (t == 0) misc[1] = 0;
  __syncthreads();
  {
    const int p = wave_append(hd != 0 && hd >= T, &misc[1]);
    if (p >= 0 && p < LS_KMAX) qlist[p] = t;
  }
  __syncthreads();
  if (t == 0) {
    bound = T;
    qlist[LS_KMAX] = misc[1] < LS_KMAX ? misc[1] : LS_KMAX;
    misc[0] = 0;
  }
  __syncthreads();
  VS_TR(A, 2);
  const u64 Mb = bound;
  const int nq = qlist[LS_KMAX];
  // the qualifying lists' slots, all loaded at once (LS_KMAX * LS_KMAX / SNT per thread)
  constexpr int QPT = LS_KMAX * LS_KMAX / SNT;
  u64 lv[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int i = u * SNT + t;
    const int li = i / LS_KMAX < nq ? i / LS_KMAX : 0;
    lv[u] = q.lists[(base + qlist[li]) * LS_KMAX + (i % LS_KMAX)];
    lv[u] = i / LS_KMAX < nq ? lv[u] : (u64)0;
  }
  int c = 0;
#pragma unroll
  for (int u = 0; u < QPT; ++u) c += (lv[u] != 0 && lv[u] >= Mb) ? 1 : 0;
  int p = wave_alloc(c, &misc[0]);
#pragma unroll
  for (int u = 0; u < QPT; ++u)
    if (lv[u] != 0 && lv[u] >= Mb) sel[p++] = lv[u];
  __syncthreads();
  int Sv = misc[0];
  Sv = Sv < LSM_SEL ? Sv : LSM_SEL;
  VS_TR(A, 3);
  VS_TRV(A, 10, Sv);
  rank_sort(sel, Sv, tk, keff);  // sampler.py:140 on the survivors
  VS_TR(A, 4);
  Smem s = {};
  s.misc = misc;
  s.redf = redf;
  const Final f = wave_sample(s, tk, keff, P);
  out(f.token, f.lp, f.flags, f.keep);
}

int ls_merge_launch(const vs_row_params* params, int R, int N, int P, char* ws, int32_t* out_ids, float* out_lp,
                    uint32_t* out_flags, int32_t* out_keep, hipStream_t stream) {
  LSMArgs a;
  a.params = params;
  a.R = R;
  a.N = N;
  a.P = P;
  a.ws = ws;
  a.out_ids = out_ids;
  a.out_lp = out_lp;
  a.out_flags = out_flags;
  a.out_keep = out_keep;
  a.trace = g_trace;
  hipLaunchKernelGGL(vs_lmhead_sample_merge_kernel, dim3(R), dim3(SNT), 0, stream, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VS_OK : hip_fail(e, "vs_lmhead_sample: merge launch");
}

}  // namespace vs

// =================================================================================================================
// Host entry points
// =================================================================================================================
using namespace vs;

// Workgroups of the sampling kernel per CU for a dynamic LDS size, cached per (device, dtype): the query costs more
// than the rest of a launch's host work, and a serving loop launches one shape over and over.
static hipError_t occupancy(int dev, int dtype, bool xl, const void* kfn, size_t lds, int* per_cu) {
  struct Entry {
    size_t lds;
    int per_cu;
  };
  static std::mutex mu;
  static Entry cache[64][3][2];  // zero lds: not yet queried (every launch has LDS)
  if (dev < 0 || dev >= 64 || dtype < 0 || dtype > 2)
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, kfn, SNT, lds);
  std::lock_guard<std::mutex> lk(mu);
  Entry& c = cache[dev][dtype][xl ? 1 : 0];
  if (c.lds != lds) {
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&c.per_cu, kfn, SNT, lds);
    if (e != hipSuccess) {
      c.lds = 0;
      return e;
    }
    c.lds = lds;
  }
  *per_cu = c.per_cu;
  return hipSuccess;
}

static bool use_cooperative() {
  static const bool coop = [] {
    const char* v = getenv("VS_COOPERATIVE");
    return v && v[0] == '1';
  }();
  return coop || g_cooperative != 0;
}

extern "C" size_t vs_sample_workspace_bytes(int B, int V) {
  (void)V;
  const int rows = B < 1 ? 1 : (B > RPL_MAX ? RPL_MAX : B);
  return (size_t)rows * ROW_WS;
}

static int sample_launch(const void* logits, int dtype, int B, int V, int64_t ld, const vs_row_params* params,
                         vs_row_state* state, int32_t* pool, const int32_t* hist, const int32_t* bias_ids,
                         const float* bias_vals, const int32_t* mask_ids, int32_t* out_ids, float* out_logprob,
                         uint32_t* out_flags, int32_t* out_keep, void* ws, size_t ws_bytes, vs_stream_t stream,
                         int list_k = 0, int32_t* list_ids = nullptr, float* list_vals = nullptr,
                         int rows_cap = RPL_MAX, const int32_t* slots = nullptr, const int32_t* tabs = nullptr) {
  if (B < 0) return fail(VS_EINVAL, "vs_sample_batch: B < 0");
  if (B == 0) return VS_OK;
  if (V < 1) return fail(VS_EINVAL, "vs_sample_batch: V < 1");
  if (ld < V) return fail(VS_EINVAL, "vs_sample_batch: ld < V");
  if (dtype != VS_F32 && dtype != VS_BF16 && dtype != VS_F16) return fail(VS_EINVAL, "vs_sample_batch: bad dtype");
  if (list_k > 0) {
    if (!logits || !list_ids || !list_vals || !ws) return fail(VS_EINVAL, "vs_topk_batch: null pointer argument");
  } else if (!logits || !params || !out_ids || !out_logprob || !ws) {
    return fail(VS_EINVAL, "vs_sample_batch: null logits/params/out_ids/out_logprob/ws");
  }
  const DevInfo* dv = dev_info();
  if (!dv) return fail(VS_EHIP, "vs_sample_batch: no HIP device");
  const int VEC = dtype == VS_F32 ? 4 : 8;
  const int unit = SNT * VEC;
  const int chmax = (EPT_MAX / VEC) * unit;
  const int rows_target = B < rows_cap ? B : rows_cap;
  const int gmin = (V + chmax - 1) / chmax;
  if (gmin > GMAX) return fail(VS_EINVAL, "vs_sample_batch: V too large for one launch row");
  int G = dv->cus / rows_target;
  if (G < 1) G = 1;
  if (G > GMAX) G = GMAX;
  if (G < gmin) G = gmin;
  int CH = (V + G - 1) / G;
  CH = (CH + unit - 1) / unit * unit;
  G = (V + CH - 1) / CH;
  const int NV = CH / unit;
  if (state && !pool) return fail(VS_EINVAL, "vs_sample_batch_state: null state pool");
  const int has_hist = state ? 1 : (hist != nullptr);
  const int lds_ch = CH;
  const size_t lds = smem_bytes(lds_ch);
  if (lds > dv->lds_per_block) return fail(VS_EINVAL, "vs_sample_batch: LDS need exceeds the device limit");
  // Two instances per dtype: XL exchanges a row's data through its XCD's L2 (every workgroup of each row on one XCD),
  // the other through the device-coherent level.
  auto kernel_fn = [dtype](bool xl) -> const void* {
    if (xl)
      return dtype == VS_F32    ? (const void*)vs_sample_kernel<VS_F32, true>
             : dtype == VS_BF16 ? (const void*)vs_sample_kernel<VS_BF16, true>
                                : (const void*)vs_sample_kernel<VS_F16, true>;
    return dtype == VS_F32    ? (const void*)vs_sample_kernel<VS_F32, false>
           : dtype == VS_BF16 ? (const void*)vs_sample_kernel<VS_BF16, false>
                              : (const void*)vs_sample_kernel<VS_F16, false>;
  };
  int per_cu = 0, per_cu_xl = 0;
  hipError_t e = occupancy(dv->device, dtype, false, kernel_fn(false), lds, &per_cu);
  if (e == hipSuccess) e = occupancy(dv->device, dtype, true, kernel_fn(true), lds, &per_cu_xl);
  if (e != hipSuccess) return hip_fail(e, "vs_sample_batch: occupancy query");
  if (per_cu_xl < per_cu) per_cu = per_cu_xl;
  const int maxres = per_cu * dv->cus;
  int RB = maxres / G;
  if (RB > rows_target) RB = rows_target;
  if (RB < 1) return fail(VS_EINVAL, "vs_sample_batch: a row does not fit on the device at once");
  if (ws_bytes < (size_t)RB * ROW_WS) return fail(VS_EWORKSPACE, "vs_sample_batch: workspace too small");
  int kcap = 1;  // list capacity per workgroup: a power of two <= KEYS_CAP / G
  while (kcap * 2 <= KEYS_CAP / G && kcap * 2 <= 1024) kcap *= 2;
  const int kmax = kcap < KCAP ? kcap : KCAP;
  if (list_k > kmax) return fail(VS_EINVAL, "vs_topk_batch: k above the largest list this shape supports");
  int bits = 0;
  while ((1ll << bits) < (long long)V) ++bits;
  SampleArgs a;
  a.logits = logits;
  a.ld = ld;
  a.V = V;
  a.G = G;
  a.CH = CH;
  a.NV = NV;
  a.vec_ok = ((uintptr_t)logits % 16 == 0) && (ld % VEC == 0);
  a.has_hist = has_hist;
  a.lds_ch = lds_ch;
  a.kcap = kcap;
  a.kmax = kmax;
  // The testing spin limit applies to plain launches only: a cooperative launch guarantees that every workgroup of
  // a row is resident, so its waits keep the default bound.
  const bool coop = use_cooperative();
  a.spin_limit = (g_spin_limit && !coop) ? g_spin_limit : 0xFFFFFFFFu;
  a.spin_ticks = coop ? WAIT_TICKS_COOP : WAIT_TICKS;
  a.debug = g_debug;
  a.fix_scale = ldexp(1.0, 63 - bits);
  a.fix_shift = 63 - bits;
  a.zspan_max = (63 - bits) * 0.6931471805599453 - 13.815510557964274;  // ln(fix_scale) - ln(1e6)
  a.params = list_k > 0 ? nullptr : params;
  a.list_k = list_k;
  a.list_ids = list_ids;
  a.list_vals = list_vals;
  a.state = state;
  a.pool = pool;
  a.slots = slots;
  a.tabs = tabs;
  a.hist = state ? pool : hist;
  a.bias_ids = bias_ids;
  a.bias_vals = bias_vals;
  a.mask_ids = mask_ids;
  a.out_ids = out_ids;
  a.out_lp = out_logprob;
  a.out_flags = out_flags;
  a.out_keep = out_keep;
  a.ws = (char*)ws;
  a.trace = g_trace;
  for (int r0 = 0; r0 < B; r0 += RB) {
    a.row0 = r0;
    a.B = (B - r0) < RB ? (B - r0) : RB;
    void* kargs[] = {&a};
    // Workgroup b runs on XCD b % 8 (the dispatcher deals a grid's workgroups to the 8 XCDs in turn; a rotation of
    // that order keeps equal b % 8 together, which is all this needs), and the kernel gives row r the workgroups
    // b with (b % 8) * nb / 8 + b / 8 in [r G, r G + G). A row lies on one XCD exactly when nb is a multiple of 8
    // and each XCD's nb / 8 workgroups hold whole rows.
    const int nbl = a.B * G;
    const bool xl = !(g_debug & VS_DEBUG_NO_XCD_EXCHANGE) && nbl % 8 == 0 && (nbl / 8) % G == 0;
    const void* kfn = kernel_fn(xl);
    // The grid never exceeds what the device holds at once (RB above), so on an otherwise idle device every
    // workgroup of a row is resident and the row barriers complete; a plain launch is ~18 us cheaper than a
    // cooperative one on MI355X. VS_COOPERATIVE=1 requests the residency guarantee of a cooperative launch; without
    // it, a barrier that cannot complete ends with VS_OUT_TIMEOUT on that row instead of hanging.
    if (coop)
      e = hipLaunchCooperativeKernel(kfn, dim3(a.B * G), dim3(SNT), kargs, (unsigned)lds, (hipStream_t)stream);
    else
      e = hipLaunchKernel(kfn, dim3(a.B * G), dim3(SNT), kargs, (unsigned)lds, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "vs_sample_batch: launch");
  }
  return VS_OK;
}

extern "C" int vs_sample_batch(const void* logits, int dtype, int B, int V, int64_t ld, const vs_row_params* params,
                               const int32_t* hist, const int32_t* bias_ids, const float* bias_vals,
                               const int32_t* mask_ids, int32_t* out_ids, float* out_logprob, uint32_t* out_flags,
                               int32_t* out_keep, void* ws, size_t ws_bytes, vs_stream_t stream) {
  return sample_launch(logits, dtype, B, V, ld, params, nullptr, nullptr, hist, bias_ids, bias_vals, mask_ids, out_ids,
                       out_logprob, out_flags, out_keep, ws, ws_bytes, stream);
}

extern "C" int vs_topk_batch(const void* logits, int dtype, int B, int V, int64_t ld, int k, int32_t* out_ids,
                             float* out_vals, void* ws, size_t ws_bytes, vs_stream_t stream) {
  if (k < 1) return fail(VS_EINVAL, "vs_topk_batch: k < 1");
  return sample_launch(logits, dtype, B, V, ld, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                       nullptr, nullptr, nullptr, ws, ws_bytes, stream, k, out_ids, out_vals);
}

extern "C" int vs_sample_batch_state(const void* logits, int dtype, int B, int V, int64_t ld,
                                     const vs_row_params* params, vs_row_state* state, int32_t* pool,
                                     const int32_t* tabs, const int32_t* slots, const int32_t* bias_ids,
                                     const float* bias_vals, const int32_t* mask_ids, int32_t* out_ids,
                                     float* out_logprob, uint32_t* out_flags, int32_t* out_keep, void* ws,
                                     size_t ws_bytes, vs_stream_t stream) {
  if (!state) return fail(VS_EINVAL, "vs_sample_batch_state: null state");
  return sample_launch(logits, dtype, B, V, ld, params, state, pool, nullptr, bias_ids, bias_vals, mask_ids, out_ids,
                       out_logprob, out_flags, out_keep, ws, ws_bytes, stream, 0, nullptr, nullptr, RPL_MAX, slots,
                       tabs);
}

// ---------------------------------------------------------------------------------------------------------------
// vs_state_fold: one 512-thread workgroup per listed request merges its recent history tokens (<= FOLD_MAX) into
// its (id, count) table, writing the merged table to the other half of its table region.
// ---------------------------------------------------------------------------------------------------------------
constexpr int FOLD_MAX = 512;
__global__ __launch_bounds__(SNT) void vs_state_fold_kernel(vs_row_state* state, const int32_t* pool, int32_t* tabs,
                                                            int64_t tab_cap, const int32_t* slots) {
  __shared__ u64 raw[FOLD_MAX];    // the recent tokens as (id << 32 | position), then sorted
  __shared__ u64 srt[FOLD_MAX];
  __shared__ int32_t uid[FOLD_MAX];  // distinct recent ids, ascending
  __shared__ int32_t ucnt[FOLD_MAX];
  __shared__ int32_t ulb[FOLD_MAX];  // each one's lower bound in the table
  __shared__ int32_t ufound[FOLD_MAX];
  __shared__ int32_t newpre[FOLD_MAX + 1];  // new ids (not in the table) before index j
  __shared__ int red[NRED];
  const int t = threadIdx.x;
  const int q = slots ? slots[blockIdx.x] : blockIdx.x;
  vs_row_state* S = state + q;
  const vs_row_state st = *S;
  const int nr = st.hist_len - st.hist_base;
  if (nr <= 0) return;
  const int n = nr < FOLD_MAX ? nr : FOLD_MAX;  // the host folds before FOLD_MAX tokens accumulate
  // the merged table must fit half of the slot's region (tab_cap pairs); a slot laid out otherwise keeps its tokens
  // counted from the history (every later step stays exact)
  if ((int64_t)st.tab_len + n > tab_cap) return;
  for (int i = t; i < n; i += SNT) raw[i] = ((u64)(uint32_t)pool[st.hist_off + st.hist_base + i] << 32) | (u64)i;
  __syncthreads();
  // ascending by (id, position): the rank of each key (keys are unique)
  for (int i = t; i < n; i += SNT) {
    const u64 k = raw[i];
    int r = 0;
    for (int j = 0; j < n; ++j) r += raw[j] < k ? 1 : 0;
    srt[r] = k;
  }
  __syncthreads();
  // distinct ids and their counts: a run head starts each id
  int nu;
  {
    int heads = 0;
    for (int i = t; i < n; i += SNT) heads += (i == 0 || (srt[i] >> 32) != (srt[i - 1] >> 32)) ? 1 : 0;
    nu = block_sum<SNT>(heads, red);
    __syncthreads();
    for (int i = t; i < n; i += SNT) {
      if (i == 0 || (srt[i] >> 32) != (srt[i - 1] >> 32)) {
        int u = 0;  // the run's index: heads before it
        for (int j = 1; j <= i; ++j) u += ((srt[j] >> 32) != (srt[j - 1] >> 32)) ? 1 : 0;
        int e = i + 1;
        while (e < n && (srt[e] >> 32) == (srt[i] >> 32)) ++e;
        uid[u] = (int32_t)(srt[i] >> 32);
        ucnt[u] = e - i;
      }
    }
  }
  __syncthreads();
  const int2* tab = (const int2*)(tabs + st.tab_off);
  const int64_t tl = st.tab_len;
  // each distinct recent id: its lower bound in the table and whether it is there
  for (int j = t; j < nu; j += SNT) {
    int64_t b = 0, e = tl;
    while (b < e) {
      const int64_t m = (b + e) >> 1;
      if (tab[m].x < uid[j]) b = m + 1;
      else e = m;
    }
    ulb[j] = (int32_t)b;
    ufound[j] = (b < tl && tab[b].x == uid[j]) ? 1 : 0;
  }
  __syncthreads();
  if (t == 0) {
    int c = 0;
    for (int j = 0; j < nu; ++j) {
      newpre[j] = c;
      c += ufound[j] ? 0 : 1;
    }
    newpre[nu] = c;
  }
  __syncthreads();
  const int64_t region = (int64_t)4 * tab_cap;
  const int64_t base = st.tab_off - st.tab_off % region;
  const int64_t alt = st.tab_off == base ? base + 2 * tab_cap : base;
  int2* out = (int2*)(tabs + alt);
  // table entries, shifted past the new ids that go before them, with the recent counts added
  for (int64_t i = t; i < tl; i += SNT) {
    const int2 e = tab[i];
    int lo = 0, hi = nu;  // the first distinct recent id >= e.x
    while (lo < hi) {
      const int m = (lo + hi) >> 1;
      if (uid[m] < e.x) lo = m + 1;
      else hi = m;
    }
    const int add = (lo < nu && uid[lo] == e.x) ? ucnt[lo] : 0;
    out[i + newpre[lo]] = make_int2(e.x, e.y + add);
  }
  // new ids: before table entry ulb[j], after the new ids before them
  for (int j = t; j < nu; j += SNT)
    if (!ufound[j]) out[ulb[j] + newpre[j]] = make_int2(uid[j], ucnt[j]);
  __syncthreads();
  if (t == 0) {
    S->tab_off = alt;
    S->tab_len = (int32_t)(tl + newpre[nu]);
    S->hist_base = st.hist_base + n;
  }
}

extern "C" int vs_state_fold(vs_row_state* state, const int32_t* pool, int32_t* tabs, int64_t tab_cap,
                             const int32_t* slots, int n, vs_stream_t stream) {
  if (n < 0) return fail(VS_EINVAL, "vs_state_fold: n < 0");
  if (n == 0) return VS_OK;
  if (!state || !pool || !tabs || tab_cap < 1) return fail(VS_EINVAL, "vs_state_fold: null pointer or tab_cap < 1");
  hipLaunchKernelGGL(vs_state_fold_kernel, dim3(n), dim3(SNT), 0, (hipStream_t)stream, state, pool, tabs, tab_cap,
                     slots);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? VS_OK : hip_fail(e, "vs_state_fold: launch");
}

// =================================================================================================================
// Allocation-free entry point: the workspace is a file-scope device array instead of a caller buffer
// =================================================================================================================
// The launches of this entry point hold at most NOALLOC_ROWS rows (larger batches run as consecutive launches that
// reuse the array; 16 rows is the batch that fills the 256 CUs at the vocabulary sizes of the path), so the array has
// a fixed size of NOALLOC_ROWS * ROW_WS bytes (about 5.6 MB) per device, held until the process ends. It is
// zero-initialised when the code object is loaded (static storage), and every call leaves it zeroed, so no call
// clears it (a clear on the first call would be stream work that a call from another stream could overtake).
namespace {
constexpr int NOALLOC_ROWS = 16;
constexpr size_t SCRATCH_BYTES = (size_t)NOALLOC_ROWS * ROW_WS;
static __device__ __align__(256) char scratch[SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64];  // device address of `scratch` per device (the host symbol is only a stand-in)

// The current device's address of `scratch`, looked up once per device.
int scratch_ptr(void** out) {
  int d = 0;
  hipError_t e = hipGetDevice(&d);
  if (e != hipSuccess) return hip_fail(e, "vs_sample_batch_noalloc: hipGetDevice");
  if (d < 0 || d >= 64) return fail(VS_EINVAL, "vs_sample_batch_noalloc: device index above 63");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[d]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e, "vs_sample_batch_noalloc: hipGetSymbolAddress(scratch)");
    g_scratch_ptr[d] = p;
  }
  *out = g_scratch_ptr[d];
  return VS_OK;
}
}  // namespace

extern "C" size_t vs_sample_noalloc_scratch_bytes(void) { return SCRATCH_BYTES; }

extern "C" int vs_sample_batch_noalloc(const void* logits, int dtype, int B, int V, int64_t ld,
                                       const vs_row_params* params, const int32_t* hist, const int32_t* bias_ids,
                                       const float* bias_vals, const int32_t* mask_ids, int32_t* out_ids,
                                       float* out_logprob, uint32_t* out_flags, int32_t* out_keep,
                                       vs_stream_t stream) {
  if (B < 0) return fail(VS_EINVAL, "vs_sample_batch_noalloc: B < 0");
  if (B == 0) return VS_OK;
  void* ws = nullptr;
  const int rc = scratch_ptr(&ws);
  if (rc != VS_OK) return rc;
  return sample_launch(logits, dtype, B, V, ld, params, nullptr, nullptr, hist, bias_ids, bias_vals, mask_ids, out_ids,
                       out_logprob, out_flags, out_keep, ws, SCRATCH_BYTES, stream, 0, nullptr, nullptr,
                       NOALLOC_ROWS);
}
