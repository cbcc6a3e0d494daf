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
// before the first slot: the successor rows B[cid[e][c]] and hp[e] go to VGPRs (thread's part, every slot), the
// predecessor rows A[anchor] and A[cid[e][c]] (any of them can become `pred`) go to LDS. The 7 slots then run from
// registers and LDS only: products, a 16-lane sum, one LDS exchange of the 16 scores per slot and a barrier. The
// walk is latency-bound: two dependent global loads (anchor, then its row) and ~7 LDS round trips.
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
constexpr int DROWS = 1 + (DSMAX - 1) * DK;  // predecessor rows: the anchor and every non-final slot's candidates

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
};

__global__ __launch_bounds__(DNT) void vs_draft_walk_kernel(WalkArgs W) {
  __shared__ uint16_t sA[DROWS * DRMAX];
  __shared__ float sS[2][DK];
  const int blk = blockIdx.x, t = threadIdx.x;
  const int c = t / DPARTS, p = t % DPARTS;
  const int S = W.S, K = W.K, R = W.R, m = R / DPARTS;
  const float* uv = W.uval + (size_t)blk * S * W.ldk;
  const int32_t* cd = W.cid + (size_t)blk * S * W.ldk;
  const float* hpb = W.hp + (size_t)blk * S * R;

  // ---- path-independent operands: this thread's candidate id, logit, successor part and hp part of every slot
  int id[DSMAX];
  float u[DSMAX];
  float hv[DSMAX][DM];
  float bv[DSMAX][DM];
#pragma unroll
  for (int e = 0; e < DSMAX; ++e) {
    id[e] = -1;
    u[e] = 0.0f;
    if (e < S && c < K) {
      const int x = cd[e * W.ldk + c];
      id[e] = (x >= 0 && x < W.vocab) ? x : -1;
      u[e] = uv[e * W.ldk + c];
    }
  }
#pragma unroll
  for (int e = 0; e < DSMAX; ++e) {
    const uint16_t* brow = W.Bc + (size_t)(id[e] < 0 ? 0 : id[e]) * R + p * m;
    const float* hrow = hpb + (size_t)(e < S ? e : 0) * R + p * m;
#pragma unroll
    for (int i = 0; i < DM; ++i) {
      bv[e][i] = (i < m) ? bf16_to_f32(brow[i]) : 0.0f;
      hv[e][i] = (i < m) ? hrow[i] : 0.0f;
    }
  }
  // ---- predecessor rows to LDS: slot 0 = the anchor, slot 1 + e*K + c = cid[e][c] (e < S - 1)
  const int a0 = W.anchor[blk];
  const bool anchor_ok = a0 >= 0 && a0 < W.vocab;
  const int nrows = 1 + (S - 1) * K;
  const int wpr = R / 2;  // 32-bit words per row (R is even)
  for (int i = t; i < nrows * wpr; i += DNT) {
    const int rr = i / wpr, wd = i - rr * wpr;
    int src = -1;
    if (rr == 0) {
      src = anchor_ok ? a0 : -1;
    } else {
      const int e = (rr - 1) / K, cc = (rr - 1) - e * K;
      const int x = cd[e * W.ldk + cc];
      src = (x >= 0 && x < W.vocab) ? x : -1;
    }
    const uint32_t v = src >= 0 ? ((const uint32_t*)(W.A + (size_t)src * R))[wd] : 0u;
    ((uint32_t*)(sA + rr * DRMAX))[wd] = v;
  }
  __syncthreads();

  // ---- the walk
  int slot = anchor_ok ? 0 : -1;  // LDS row of pred; -1 once no valid predecessor remains
#pragma unroll
  for (int e = 0; e < DSMAX; ++e) {
    if (e < S) {
      float acc = 0.0f;
      const uint16_t* arow = sA + (slot < 0 ? 0 : slot) * DRMAX + p * m;
#pragma unroll
      for (int i = 0; i < DM; ++i) {
        if (i < m) {
          const float a = bf16_to_f32(arow[i]) * hv[e][i];  // A[pred] * hp[e], rounded to fp32
          acc = acc + bv[e][i] * a;
        }
      }
      acc = acc + lane_xor<1>(acc);
      acc = acc + lane_xor<2>(acc);
      acc = acc + lane_xor<4>(acc);
      acc = acc + lane_xor<8>(acc);
      if (p == 0 && c < K) sS[e & 1][c] = id[e] >= 0 ? u[e] + acc : -__builtin_inff();
      __syncthreads();
      // every thread resolves the same first maximum over the valid candidates
      int best = -1;
      float bs = 0.0f;
      for (int cc = 0; cc < K; ++cc) {
        const int x = cd[e * W.ldk + cc];
        if (x < 0 || x >= W.vocab) continue;
        const float s = sS[e & 1][cc];
        if (best < 0 || s > bs) {
          best = cc;
          bs = s;
        }
      }
      if (slot < 0) best = -1;
      const int tok = best < 0 ? -1 : cd[e * W.ldk + best];
      if (t == 0) W.out[(size_t)blk * S + e] = tok;
      slot = best < 0 ? -1 : 1 + e * K + best;
    }
  }
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
  if ((uintptr_t)A % 4 != 0) return fail(VS_EINVAL, "vs_draft_walk: predecessor codebook not 4-byte aligned");
  WalkArgs w{uval, cid, ldk, hp, (const uint16_t*)A, (const uint16_t*)B, anchor, out, n, S, K, R, vocab};
  hipLaunchKernelGGL(vs_draft_walk_kernel, dim3(n), dim3(DNT), 0, (hipStream_t)stream, w);
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
