// vs_draft.hip - the DFlash2 drafter's candidate walk for gfx950: for each block, 7 sequential slots pick one of the
// slot's top-16 vocabulary candidates by logit + low-rank bigram score, first maximum.
//
// Reference: volundr-mlx/spec/dflash.py:50-60 (_walk) fed by dflash.py:228-240 (propose: top-16 of each row's
// logits, value descending, then the walk from the anchor token).
//   for e in 0..S-1:  a = float32(A[pred]) * hp[e];  s[c] = uval[e][c] + float32(B[cid[e][c]]) . a;
//                     pred = cid[e][first argmax of s]
//
// One 256-thread workgroup per block: thread t owns candidate c = t / 16 and the contiguous part p = t % 16 of the
// rank axis (R / 16 entries). Everything the walk can touch is independent of the path it takes, so it is fetched
// before the first slot: the successor rows B[cid[e][c]] stay in VGPRs as packed bf16 (thread's part, every slot);
// the predecessor rows A[anchor] and A[cid[e][c]] (any of them can become `pred`) go to LDS, each multiplied by the
// hp of the one slot that can use it. Every global load is issued before the first is consumed, so the fetch costs
// two memory latencies (ids, then the rows they name). The slots then run from registers and LDS only: 16 products,
// a 16-lane sum, one LDS exchange of the 16 scores and a barrier, and a 16-lane first-max reduction.
#include "vs_common.h"
#include "vs_host.h"

#pragma clang fp contract(off)

namespace vs {

constexpr int DNT = 256;
constexpr int DK = 16;          // candidates per slot (dflash.py TOPK)
constexpr int DPARTS = DNT / DK;  // threads per candidate
constexpr int DSMAX = 8;        // slots per block (dflash.py BLOCK - 1 = 7)
constexpr int DRMAX = 256;      // rank (dflash.py RANK)
constexpr int DM = DRMAX / DPARTS;  // rank entries per thread at most
constexpr int DROWS = 1 + (DSMAX - 1) * DK;  // predecessor rows: the anchor and every non-final slot's 16 positions
static_assert((DROWS + DSMAX) * DRMAX * 4 <= 160 * 1024 - 1024, "predecessor rows and hp fit the LDS");

struct WalkArgs {
  const float* uval;     // [n, S, ldk] candidate logits, value descending
  const int32_t* cid;    // [n, S, ldk] candidate ids
  int ldk;               // row stride of uval / cid (>= K)
  const float* hp;       // [n, S, R]
  const uint16_t* A;     // [vocab, R] bf16 predecessor codebook
  const uint16_t* Bc;    // [vocab, R] bf16 successor codebook
  const int32_t* anchor; // [n]
  int32_t* out;          // [n, S]
  int n, S, K, R, vocab;
  unsigned long long* trace;  // development builds only (VS_TRACE); null otherwise
};

// Raw bf16 part of a row (thread part p: M entries from p*M on), packed two per 32-bit word. M == 0: run-time m
// (any R % 16 == 0), element loads; M = 8 or 16: 16-byte loads.
template <int M>
struct Part16 {
  uint32_t w[DM / 2];
};

template <int M>
__device__ __forceinline__ void load_part(const uint16_t* row, int m, Part16<M>& d) {
  if constexpr (M == 0) {
#pragma unroll
    for (int i = 0; i < DM / 2; ++i) {
      const uint32_t lo = 2 * i < m ? row[2 * i] : 0u, hi = 2 * i + 1 < m ? row[2 * i + 1] : 0u;
      d.w[i] = lo | (hi << 16);
    }
  } else {
#pragma unroll
    for (int q = 0; q < M / 8; ++q) {
      const uint4 r = ((const uint4*)row)[q];
      d.w[4 * q] = r.x;
      d.w[4 * q + 1] = r.y;
      d.w[4 * q + 2] = r.z;
      d.w[4 * q + 3] = r.w;
    }
#pragma unroll
    for (int i = M / 2; i < DM / 2; ++i) d.w[i] = 0u;
  }
}

template <int M>
__device__ __forceinline__ float part_get(const Part16<M>& d, int i) {
  const uint32_t w = d.w[i >> 1];
  return __uint_as_float((i & 1) ? (w & 0xFFFF0000u) : (w << 16));
}

template <int M>
__global__ __launch_bounds__(DNT) void vs_draft_walk_kernel(WalkArgs W) {
  // sA row 0 = A[anchor] * hp[0]; row 1 + e*DK + c = A[cid[e][c]] * hp[e + 1]: a predecessor row is only ever
  // used by the slot after its own, so it is stored already multiplied by that slot's hp (rounded to fp32 as in
  // a = float32(A[pred]) * hp[e]).
  __shared__ float sA[DROWS][DRMAX];
  __shared__ float sH[DSMAX][DRMAX];  // hp of the block
  __shared__ float sS[2][DK];         // the current slot's scores (double-buffered across slots)
  __shared__ int sId[DSMAX][DK];      // candidate ids, -1 where invalid
  const int blk = blockIdx.x, t = threadIdx.x;
  const int c = t / DPARTS, p = t % DPARTS;
  const int S = W.S, K = W.K, R = W.R, m = M ? M : R / DPARTS;
  const float* uv = W.uval + (size_t)blk * S * W.ldk;
  const int32_t* cd = W.cid + (size_t)blk * S * W.ldk;
  const float* hpb = W.hp + (size_t)blk * S * R;
  VS_TR_DECL(W);
  VS_TR(W, 0);

  // ---- path-independent operands. Every load is unconditional (indices clamped into the arrays, results masked
  // afterwards) and issued before any is consumed, so the fetch costs two memory latencies: the candidate ids and
  // the anchor, then the rows they name.
  const int a0 = W.anchor[blk];
  const int cc0 = c < K ? c : K - 1;
  int id[DSMAX];
  float u[DSMAX];
#pragma unroll
  for (int e = 0; e < DSMAX; ++e) {
    const int ee = e < S ? e : S - 1;
    id[e] = cd[ee * W.ldk + cc0];
    u[e] = uv[ee * W.ldk + cc0];
  }
  constexpr int HPT = DSMAX * DRMAX / DNT;  // hp elements per thread (S * R <= DSMAX * DRMAX)
  float hq[HPT];
#pragma unroll
  for (int j = 0; j < HPT; ++j) {
    const int i = j * DNT + t;
    hq[j] = hpb[i < S * R ? i : 0];
  }
  // keep the scheduler from interleaving each load with its use (it would wait on every load in turn)
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int e = 0; e < DSMAX; ++e) id[e] = (e < S && c < K && id[e] >= 0 && id[e] < W.vocab) ? id[e] : -1;
  const bool anchor_ok = a0 >= 0 && a0 < W.vocab;
  Part16<M> bq[DSMAX], aq[DSMAX];  // successor rows of every slot; predecessor rows (slots 0..S-2, then the anchor)
#pragma unroll
  for (int e = 0; e < DSMAX; ++e) load_part<M>(W.Bc + (size_t)(id[e] < 0 ? 0 : id[e]) * R + p * m, m, bq[e]);
#pragma unroll
  for (int e = 0; e < DSMAX - 1; ++e) load_part<M>(W.A + (size_t)(id[e] < 0 ? 0 : id[e]) * R + p * m, m, aq[e]);
  load_part<M>(W.A + (size_t)(anchor_ok ? a0 : 0) * R + p * m, m, aq[DSMAX - 1]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < HPT; ++j) {
    const int i = j * DNT + t;
    if (i < S * R) sH[i / R][i % R] = hq[j];
  }
  if (p == 0) {
#pragma unroll
    for (int e = 0; e < DSMAX; ++e) sId[e][c] = id[e];
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < DSMAX - 1; ++e) {
    if (e + 1 < S) {
#pragma unroll
      for (int i = 0; i < DM; ++i)
        if (i < m) sA[1 + e * DK + c][p * m + i] = part_get(aq[e], i) * sH[e + 1][p * m + i];
    }
  }
  if (c == 0) {
#pragma unroll
    for (int i = 0; i < DM; ++i)
      if (i < m) sA[0][p * m + i] = part_get(aq[DSMAX - 1], i) * sH[0][p * m + i];
  }
  __syncthreads();
  VS_TR(W, 1);

  // ---- the walk: registers and LDS only
  const int lc = lane_id() & (DK - 1);  // the candidate this lane reads back for the first-max reduction
  int slot = anchor_ok ? 0 : -1;       // LDS row of pred; -1 once no valid predecessor remains
#pragma unroll
  for (int e = 0; e < DSMAX; ++e) {
    if (e < S) {
      float acc = 0.0f;
      const float* arow = &sA[slot < 0 ? 0 : slot][p * m];
#pragma unroll
      for (int i = 0; i < DM; ++i)
        if (i < m) acc = acc + part_get(bq[e], i) * arow[i];
      acc = acc + lane_xor<1>(acc);
      acc = acc + lane_xor<2>(acc);
      acc = acc + lane_xor<4>(acc);
      acc = acc + lane_xor<8>(acc);
      if (p == 0) sS[e & 1][c] = u[e] + acc;
      __syncthreads();
      // first maximum over the valid candidates, in every 16-lane group: key = score order, then the lower
      // position; 0 = no valid candidate (a valid key is never 0: ord32 of a non-NaN float is non-zero)
      const float sc = sS[e & 1][lc];
      const int cid_l = sId[e][lc];
      const float scn = sc != sc ? -__builtin_inff() : sc;  // a NaN score ranks as -inf
      u64 key = (cid_l >= 0 && lc < K) ? ((u64)ord32(scn) << 32) | (u64)(DK - 1 - lc) : (u64)0;
      u64 o = lane_xor<1>(key);
      key = o > key ? o : key;
      o = lane_xor<2>(key);
      key = o > key ? o : key;
      o = lane_xor<4>(key);
      key = o > key ? o : key;
      o = lane_xor<8>(key);
      key = o > key ? o : key;
      const int best = (key == 0 || slot < 0) ? -1 : DK - 1 - (int)(key & (DK - 1));
      const int tok = best < 0 ? -1 : sId[e][best];
      if (t == 0) W.out[(size_t)blk * S + e] = tok;
      slot = best < 0 ? -1 : 1 + e * DK + best;
      VS_TR(W, 2 + e);
    }
  }
  VS_TR_FLUSH(W);
}

}  // namespace vs

using namespace vs;

extern "C" int vs_draft_walk(const float* uval, const int32_t* cid, int ldk, const float* hp, const void* A,
                             const void* B, int vocab, int R, const int32_t* anchor, int n, int S, int K,
                             int32_t* out, vs_stream_t stream) {
  if (n < 0 || S < 0) return fail(VS_EINVAL, "vs_draft_walk: negative n or slot count");
  if (n == 0 || S == 0) return VS_OK;
  if (!uval || !cid || !hp || !A || !B || !anchor || !out) return fail(VS_EINVAL, "vs_draft_walk: null pointer argument");
  if (S > DSMAX) return fail(VS_EINVAL, "vs_draft_walk: more than 8 slots per block");
  if (K < 1 || K > DK) return fail(VS_EINVAL, "vs_draft_walk: candidates per slot outside [1, 16]");
  if (ldk < K) return fail(VS_EINVAL, "vs_draft_walk: ldk < K");
  if (R < DPARTS || R > DRMAX || R % DPARTS != 0)
    return fail(VS_EINVAL, "vs_draft_walk: rank must be a multiple of 16 in [16, 256]");
  if (vocab < 1) return fail(VS_EINVAL, "vs_draft_walk: vocab < 1");
  WalkArgs w{uval, cid, ldk, hp, (const uint16_t*)A, (const uint16_t*)B, anchor, out, n, S, K, R, vocab, g_trace};
  // 16-byte loads where every part is 16-byte aligned: rank 128 or 256 with aligned codebooks
  const bool vec = ((uintptr_t)A % 16 == 0) && ((uintptr_t)B % 16 == 0);
  if (vec && R == 256)
    hipLaunchKernelGGL(vs_draft_walk_kernel<16>, dim3(n), dim3(DNT), 0, (hipStream_t)stream, w);
  else if (vec && R == 128)
    hipLaunchKernelGGL(vs_draft_walk_kernel<8>, dim3(n), dim3(DNT), 0, (hipStream_t)stream, w);
  else
    hipLaunchKernelGGL(vs_draft_walk_kernel<0>, dim3(n), dim3(DNT), 0, (hipStream_t)stream, w);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "vs_draft_walk: launch");
  return VS_OK;
}

extern "C" int vs_topk_batch(const void* logits, int dtype, int B, int V, int64_t ld, int k, int32_t* out_ids,
                             float* out_vals, void* ws, size_t ws_bytes, vs_stream_t stream);
extern "C" size_t vs_sample_workspace_bytes(int B, int V);

// Workspace: [sampler region, fixed size] [candidate lists]. The sampler region is zeroed once and left zeroed by
// every call; it must not move with the row count, or a later call would find an earlier call's lists where it
// expects zeroed counters. The lists are written in full by every call before the walk reads them.
static size_t sample_region() { return vs_sample_workspace_bytes(1 << 30, 1); }
static size_t list_bytes(int rows) { return (size_t)rows * DK * 8; }

extern "C" size_t vs_draft_workspace_bytes(int n, int S, int V) {
  (void)V;
  if (n < 1 || S < 1) return 0;
  return sample_region() + list_bytes(n * S);
}

extern "C" int vs_draft_propose(const void* logits, int dtype, int n, int S, int V, int64_t ld, const float* hp,
                                const void* A, const void* B, int vocab, int R, const int32_t* anchor, int32_t* out,
                                void* ws, size_t ws_bytes, vs_stream_t stream) {
  if (n < 0 || S < 0) return fail(VS_EINVAL, "vs_draft_propose: negative n or slot count");
  if (n == 0 || S == 0) return VS_OK;
  if (!ws) return fail(VS_EINVAL, "vs_draft_propose: null workspace");
  if ((long long)n * S > (1 << 24)) return fail(VS_EINVAL, "vs_draft_propose: too many rows");
  const int rows = n * S;
  const size_t sr = sample_region();
  if (ws_bytes < sr + list_bytes(rows)) return fail(VS_EWORKSPACE, "vs_draft_propose: workspace too small");
  int32_t* ids = (int32_t*)((char*)ws + sr);
  float* vals = (float*)((char*)ws + sr + (size_t)rows * DK * 4);
  int rc = vs_topk_batch(logits, dtype, rows, V, ld, DK, ids, vals, ws, sr, stream);
  if (rc != VS_OK) return rc;
  return vs_draft_walk(vals, ids, DK, hp, A, B, vocab, R, anchor, n, S, DK, out, stream);
}
