// vs_lmsample.h - what the fused head-and-sample kernel (vs_lmhead.hip) leaves for the per-row merge
// (vs_sample.hip): the workspace layout and the row classification both kernels share.
#pragma once
#include "vs_common.h"

namespace vs {

constexpr int LS_RMAX = 16;   // rows (decode positions) per call: one MFMA tile of 16 positions
constexpr int LS_KMAX = 64;   // largest top_k the fused epilogue serves (a workgroup keeps <= 64 keys per row)
constexpr int LS_PMAX = 512;  // head workgroups per launch at most

// Per (row, workgroup) results of the head kernel, row-major ([R][LS_PMAX] each; lists [R][LS_PMAX][LS_KMAX]).
struct LSParts {
  u64* heads;      // the largest key of each list (0: empty)
  u64* lists;      // the workgroup's largest keys of the row (key64: value descending, lower id first), unsorted,
                   // zero padded: every key whose bf16 value reaches that of its top_k-th largest (<= LS_KMAX)
  u64* amkey;      // np.argmax key of the workgroup's values (NaN first)
  double* se;      // sum exp(x - mf) over its finite values
  float* mf;       // their maximum
  uint32_t* nfin;  // their number
};
__host__ __device__ inline size_t ls_list_bytes(int R) { return (size_t)R * LS_PMAX * LS_KMAX * 8; }
__host__ __device__ inline size_t ls_workspace_bytes(int R) {
  return ls_list_bytes(R) + (size_t)R * LS_PMAX * (8 + 8 + 8 + 4 + 4);
}
__host__ __device__ inline LSParts ls_parts(char* ws, int R) {
  LSParts q;
  q.lists = (u64*)ws;
  q.heads = (u64*)(ws + ls_list_bytes(R));
  q.amkey = q.heads + (size_t)R * LS_PMAX;
  q.se = (double*)(q.amkey + (size_t)R * LS_PMAX);
  q.mf = (float*)(q.se + (size_t)R * LS_PMAX);
  q.nfin = (uint32_t*)(q.mf + (size_t)R * LS_PMAX);
  return q;
}

// How the fused path serves a row (Sampler.sample, sampler.py:100-156, on the head's output):
//   LS_GREEDY : np.argmax over [0, vlim) and the log-softmax there (Sampling.greedy, :127-128; with
//               VS_ROW_ARGMAX_VV, mx.argmax(logits[:vv]) of Sampler.choose, :95-96)
//   k >= 1    : top-k sampling (:129-156) from the workgroups' candidate lists
//   LS_UNSUPPORTED : logit edits (bias, suppressed ids, an active stop range, penalties over a history) or top_k
//               off / above LS_KMAX: the row needs the logits (the caller runs the head and vs_sample_batch)
constexpr int LS_GREEDY = 0;
constexpr int LS_UNSUPPORTED = -1;
__device__ __forceinline__ int ls_class(const vs_row_params& P, int N, int* vlim) {
  *vlim = N;
  const bool edits = P.bias_end > P.bias_begin || P.supp_end > P.supp_begin || P.stop_end > P.stop_begin ||
                     (P.hist_end > P.hist_begin &&
                      (P.repetition_penalty != 1.0f || P.frequency_penalty != 0.0f || P.presence_penalty != 0.0f));
  if (edits || (P.flags & VS_ROW_FORCE)) return LS_UNSUPPORTED;
  if (P.flags & VS_ROW_GREEDY) {
    if (P.flags & VS_ROW_ARGMAX_VV) *vlim = P.vocab_valid < N ? P.vocab_valid : N;
    return LS_GREEDY;
  }
  return (P.top_k >= 1 && P.top_k <= LS_KMAX) ? P.top_k : LS_UNSUPPORTED;
}

// Launches vs_lmhead_sample_merge_kernel (vs_sample.hip): one workgroup per row merges the P head workgroups'
// results and writes the token, logprob, flags and kept size.
int ls_merge_launch(const vs_row_params* params, int R, int N, int P, char* ws, int32_t* out_ids, float* out_lp,
                    uint32_t* out_flags, int32_t* out_keep, hipStream_t stream);

}  // namespace vs
