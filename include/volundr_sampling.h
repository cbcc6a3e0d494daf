/* volundr_sampling.h - C ABI of the MI355X token-selection library (libvolundr_sampling.so).
 *
 * The library replaces the token-selection hot path of volundr-mlx:
 *   - vs_sample_batch   : Sampler.sample for a batch of rows (volundr-mlx/sampler.py:100-156), called per row
 *                         by scheduler.py:424 / session.py:615 through Sampler.choose (sampler.py:83-98);
 *   - vs_sample_batch_state : the same with the per-request sampler state kept on the device (the xorshift64*
 *                         draw, Sampler.counts as a token history in a device pool, Sampler.produced), so that a
 *                         serving loop uploads nothing per step (sampler.py:58-81);
 *   - vs_verify_greedy  : the greedy verify step of speculative decoding: first-max argmax over the valid
 *                         vocabulary and the accept prefix (volundr-mlx/spec/specdec.py:326-336 for B=1,
 *                         volundr-mlx/scheduler.py:462-470 for B<=4), plus the chosen-token logprob.
 * The reference has no function boundary for these (NumPy and inline MLX ops); the Python host in
 * volundr-mlx_amd/volundr_amd keeps sampler.py's call surface on top of these entry points.
 *
 * Conventions: every pointer argument is a DEVICE pointer (ws included); all work is
 * stream-ordered on `stream` (a hipStream_t; 0 = the null stream); nothing is allocated inside the hot calls.
 * Return codes: 0 = OK; VS_EINVAL = bad argument; VS_EWORKSPACE = workspace too small; VS_EHIP = a HIP runtime
 * call failed. vs_last_error() describes the last failure of the calling thread.
 * Workspaces must be zeroed once (vs_workspace_init) before first use; every call leaves its workspace ready for
 * the next one, so no reset is needed.
 * Calls that share one workspace must be ordered on one stream.
 */
#ifndef VOLUNDR_SAMPLING_H
#define VOLUNDR_SAMPLING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* vs_stream_t; /* hipStream_t, declared without the HIP headers */

enum { VS_OK = 0, VS_EINVAL = -1, VS_EWORKSPACE = -2, VS_EHIP = -3 };

/* Logit element types. bf16 and f16 rows are widened to float32 exactly, as sampler.py:94 does with
 * logits.astype(mx.float32). */
enum { VS_F32 = 0, VS_BF16 = 1, VS_F16 = 2 };

/* vs_row_params.flags */
enum {
  VS_ROW_GREEDY = 1u, /* Sampling.greedy (session.py:466-467): top_k == 1 or temperature < 1e-6 -> np.argmax of the
                         processed row over the full vocabulary, first maximum (sampler.py:127-128) */
  VS_ROW_ARGMAX_VV = 2u, /* with VS_ROW_GREEDY: a request that needs no logits (Sampling.needs_logits is False,
                           session.py:469-474) takes the first-max argmax over [0, vocab_valid) with no edits
                           (sampler.py:96, mx.argmax(logits[:vv])). The host sets it only for rows with no bias,
                           neutral penalties and no suppressed id below vocab_valid; the one condition that can change
                           per step, an active stop mask (produced < min_new_tokens with stop ids), is decided by the
                           kernel: a row whose stop range applies takes the ordinary greedy path over the full row */
  VS_ROW_HIST_PAIRS = 8u, /* vs_sample_batch: the row's hist range holds the penalty counts as a table of (id, count)
                            int32 pairs, ids ascending and unique (Sampler.counts, sampler.py:77-78, as :113-122 reads
                            it), hist_begin even, instead of the raw token history; each workgroup then reads only
                            the entries of its vocabulary range. Ignored by vs_sample_batch_state (its pool holds
                            raw ids) */
  VS_ROW_FORCE = 4u /* the reasoning budget forces force_token (sampler.py:88-90, Sampler.choose returns it without
                       sampling): the row's logits are not read and no draw is consumed; the state entry point records
                       the token as Sampler.accept does */
};

/* out_flags bits */
enum {
  VS_OUT_DRAW_BOUNDARY = 1u << 0, /* the scaled draw u*z lies within 1e-6*z of a CDF boundary */
  VS_OUT_TOPP_BOUNDARY = 1u << 1, /* the top-p cut lies within 1e-6 of a cumulative boundary */
  VS_OUT_GREEDY = 1u << 3,        /* the row took the greedy argmax */
  VS_OUT_NOFINITE = 1u << 4,      /* no finite logit: np.argmax of the row (sampler.py:131-132) */
  VS_OUT_COOP = 1u << 5,          /* the distribution was resolved by the row-cooperative radix select */
  VS_OUT_GATHER = 1u << 6,        /* the distribution was resolved in one workgroup after a gather */
  VS_OUT_HIST_FULL = 1u << 7,     /* vs_sample_batch_state: the request's history slots were full, the token was
                                     not recorded (later penalties miss it) */
  VS_OUT_FORCED = 1u << 8,        /* the row returned its VS_ROW_FORCE token */
  VS_OUT_UNSUPPORTED = 1u << 9,   /* vs_lmhead_sample: the row needs its logits (edits, or top_k off or above 64);
                                     no result was computed */
  VS_OUT_TIMEOUT = 1u << 31       /* an inter-workgroup wait hit its spin limit: results of this row are invalid */
};

/* Per-row sampling parameters (the fields of session.py:439-456 that Sampler.sample reads, sampler.py:100-156).
 * 96 bytes, 8-byte aligned. Index ranges are [begin, end) into the shared arrays of vs_sample_batch.
 * top_p and min_p stay float64 because the reference compares them with float64 sums (sampler.py:146,150). */
typedef struct vs_row_params {
  float temperature;        /* sampler.py:129 t = float32(temperature) */
  float repetition_penalty; /* sampler.py:118-120 (float32); 1 disables */
  float frequency_penalty;  /* sampler.py:121 (float32) */
  float presence_penalty;   /* sampler.py:121 (float32) */
  int32_t top_k;            /* sampler.py:133-134; 0 = off (None and 0 both mean off); the host maps k < 0 to 1 */
  uint32_t flags;           /* VS_ROW_GREEDY */
  double top_p;             /* sampler.py:145; >= 1 disables */
  double min_p;             /* sampler.py:149; <= 0 disables */
  double u;                 /* the uniform draw in [0,1) (sampler.py:154 self.uniform()) */
  int64_t hist_begin, hist_end; /* token history (the multiset behind Sampler.counts, sampler.py:77-78) */
  int32_t bias_begin, bias_end; /* additive float32 biases, ids sorted ascending, equal ids in application order
                                   (budget extra then logit_bias, sampler.py:104-109) */
  int32_t supp_begin, supp_end; /* suppressed ids, sorted: -inf before the penalties (sampler.py:110-112) */
  int32_t stop_begin, stop_end; /* stop ids masked while produced < min_new_tokens, sorted: -inf after the
                                   penalties (sampler.py:123-126); the host passes an empty range otherwise */
  int32_t vocab_valid;          /* Sampler.vv (sampler.py:59), read only by VS_ROW_ARGMAX_VV rows; 1 <= vv */
  int32_t force_token;          /* the token of a VS_ROW_FORCE row (zero otherwise) */
} vs_row_params;

/* Sampler.sample for B rows of logits (row r starts at element r*ld; ld >= V).
 *   params     : device array [B] of vs_row_params
 *   hist       : device int32 token ids, indexed by params[r].hist_begin..hist_end (may be NULL if all empty);
 *                ids outside [0, V) are ignored
 *   bias_ids/bias_vals, mask_ids : device arrays indexed by the bias / supp / stop ranges (may be NULL if empty)
 *   out_ids    : int32 [B] token ids
 *   out_logprob: float32 [B] log(pr[j]/z) of the drawn token (greedy rows: log-softmax of the processed row)
 *   out_flags  : uint32 [B] VS_OUT_* bits (may be NULL)
 *   out_keep   : int32 [B] size of the distribution drawn from (may be NULL)
 *   ws         : device workspace of at least vs_sample_workspace_bytes(B, V) bytes, zeroed once beforehand
 * Replaces: volundr-mlx/sampler.py:100-156 (Sampler.sample), applied per row as scheduler.py:416-425 does. */
int vs_sample_batch(const void* logits, int dtype, int B, int V, int64_t ld, const vs_row_params* params,
                    const int32_t* hist, const int32_t* bias_ids, const float* bias_vals, const int32_t* mask_ids,
                    int32_t* out_ids, float* out_logprob, uint32_t* out_flags, int32_t* out_keep, void* ws,
                    size_t ws_bytes, vs_stream_t stream);

size_t vs_sample_workspace_bytes(int B, int V);

/* vs_sample_batch without a workspace argument and without any allocation: the kernels use a fixed device array
 * of vs_sample_noalloc_scratch_bytes() bytes (about 5.6 MB: 16 rows of the sampling workspace) in the library, one
 * per device, kept until the process ends. It covers every batch size and vocabulary the library accepts (batches
 * above 16 rows run as consecutive launches that reuse it). The array is zero when the library is loaded and every
 * call leaves it zeroed (rows that report VS_OUT_TIMEOUT included), so no call clears it and the first call does no
 * extra work. All calls on one device share the array: calls that overlap on one device (different streams, or
 * threads without ordering) race and give wrong results.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). */
int vs_sample_batch_noalloc(const void* logits, int dtype, int B, int V, int64_t ld, const vs_row_params* params,
                            const int32_t* hist, const int32_t* bias_ids, const float* bias_vals,
                            const int32_t* mask_ids, int32_t* out_ids, float* out_logprob, uint32_t* out_flags,
                            int32_t* out_keep, vs_stream_t stream);

size_t vs_sample_noalloc_scratch_bytes(void);

/* Per-request sampler state kept on the device (Sampler, sampler.py:58-81). 48 bytes, 8-byte aligned.
 * The penalty counts (Sampler.counts) are a table of (id, count) pairs sorted by id in a table pool, holding the
 * history up to hist_base, plus the history tokens recorded since (pool[hist_off + hist_base, hist_off + hist_len)),
 * which vs_state_fold merges into the table. */
typedef struct vs_row_state {
  uint64_t rng;           /* xorshift64* state (Sampler.rng); the host seeds it as Sampler.__init__ does */
  int64_t hist_off;       /* first slot of this request's token history in the pool */
  int32_t hist_len;       /* tokens recorded so far (the history, in order) */
  int32_t hist_cap;       /* slots reserved from hist_off */
  int32_t produced;       /* Sampler.produced */
  int32_t min_new_tokens; /* the stop range of the row's params applies while produced < min_new_tokens */
  int64_t tab_off;        /* first int32 of the (id, count) table in the table pool (even) */
  int32_t tab_len;        /* its entries: the counts of history tokens [0, hist_base) */
  int32_t hist_base;      /* history tokens already counted in the table */
} vs_row_state;

/* vs_sample_batch with the state on the device: row r of the logits belongs to request q = slots[r] (slots NULL:
 * q = r), whose parameters are params[q] and whose state is state[q]. The draw is Sampler.uniform() on
 * state[q].rng; the penalty counts are the table tabs[tab_off, tab_off + 2 tab_len) plus the history tokens
 * pool[hist_off + hist_base, hist_off + hist_len) (tabs may be NULL when every tab_len is 0); the stop mask applies
 * while produced < min_new_tokens (params[q].u, hist_begin/hist_end are ignored; the stop range gives the stop ids).
 * After the choice the request's state is advanced as Sampler.accept does (sampler.py:77-81): the token is appended
 * to the history (flag VS_OUT_HIST_FULL when hist_len == hist_cap), produced += 1, and the xorshift64* state moves on
 * when the row drew (not for greedy rows, rows with no finite logit, which return before self.uniform(),
 * sampler.py:127-133, or VS_ROW_FORCE rows). Outputs are indexed by r. Rows flagged VS_OUT_TIMEOUT leave their
 * state unchanged. Rows of one call must not share a request or history slots. The params and state tables may
 * hold more requests than the call has rows (a continuous-batching slot table: requests join and leave between
 * calls by changing their rows of the tables and the slots array).
 * Replaces: Sampler.choose (sampler.py:83-98) for a batch of requests (scheduler.py:402-425), with uniform() and
 * accept() on the device; the reasoning budget's force and bias arrive as VS_ROW_FORCE and bias entries. */
int vs_sample_batch_state(const void* logits, int dtype, int B, int V, int64_t ld, const vs_row_params* params,
                          vs_row_state* state, int32_t* pool, const int32_t* tabs, const int32_t* slots,
                          const int32_t* bias_ids, const float* bias_vals, const int32_t* mask_ids, int32_t* out_ids,
                          float* out_logprob, uint32_t* out_flags, int32_t* out_keep, void* ws, size_t ws_bytes,
                          vs_stream_t stream);

/* Merge the history tokens recorded since each listed request's last merge (pool[hist_off + hist_base, hist_off +
 * hist_len), at most 512 of them) into its (id, count) table: the merged table is written to the other half of the
 * request's table region (a region of 4 * tab_cap int32 at a multiple of 4 * tab_cap; tab_cap >= the number of
 * distinct ids the request can hold), tab_off / tab_len / hist_base are updated; a request whose table length plus
 * the tokens to merge exceeds tab_cap is left unchanged (its tokens stay counted from the history, every later step
 * exact). Stream-ordered with the sampling
 * calls that read the tables. No counterpart in the reference (Sampler.counts is a dict updated per token,
 * sampler.py:77-78). */
int vs_state_fold(vs_row_state* state, const int32_t* pool, int32_t* tabs, int64_t tab_cap, const int32_t* slots, int n,
                  vs_stream_t stream);

/* Greedy speculative verify over logits [B, T, V] (row (b,t) starts at element (b*T + t)*ld).
 *   drafts     : int32 [B, T-1], the draft tokens inp[:, 1:] of the verify input
 *   out_argmax : int32 [B, T], first-max argmax over [0, vocab_valid)
 *   out_accept : int32 [B], nacc = sum(cumprod(drafts == argmax[:, :-1]))
 *   out_logprob: float32 [B, T], x[argmax] - logsumexp(x[:vocab_valid]) (may be NULL)
 * Replaces: volundr-mlx/spec/specdec.py:326-327 and volundr-mlx/scheduler.py:462-463 (tok, nacc). */
int vs_verify_greedy(const void* logits, int dtype, int B, int T, int V, int64_t ld, int vocab_valid,
                     const int32_t* drafts, int32_t* out_argmax, int32_t* out_accept, float* out_logprob, void* ws,
                     size_t ws_bytes, vs_stream_t stream);

size_t vs_verify_workspace_bytes(int B, int T, int V);

/* The bf16 lm_head GEMM with greedy verify fused into its epilogue: logits = bf16(h @ W^T) (one rounding, nearest
 * even, of a float32 sum of products) are reduced in registers and never written unless out_logits is given.
 *   h          : bf16 [B*T, ldh] final hidden states (row b*T + t), 16-byte aligned, ldh % 8 == 0
 *   W          : bf16 [N, ldw] lm_head weight (vocab_size rows of K = hidden), 16-byte aligned, ldw % 8 == 0
 *   K          : hidden size, any multiple of 256;  B*T <= 80
 *   drafts, out_argmax, out_accept, out_logprob : as vs_verify_greedy (first-max argmax over [0, vocab_valid))
 *   out_logits : bf16 [B*T, ldo] or NULL (testing / callers that need the rows; costs the logits write)
 *   ws         : device workspace of at least vs_lmhead_workspace_bytes(B, T) bytes, zeroed once beforehand
 * Replaces: volundr-mlx/volundr.py:958-968 (lm_head, bf16) with spec/verify.py:223 feeding spec/specdec.py:326-327
 * (argmax + accept), in one launch. */
int vs_lmhead_verify_greedy(const void* h, int64_t ldh, const void* W, int64_t ldw, int N, int K, int vocab_valid,
                            int B, int T, const int32_t* drafts, int32_t* out_argmax, int32_t* out_accept,
                            float* out_logprob, void* out_logits, int64_t ldo, void* ws, size_t ws_bytes,
                            vs_stream_t stream);

size_t vs_lmhead_workspace_bytes(int B, int T);

/* The bf16 lm_head with Sampler.sample fused after it, for R <= 16 decode rows: logits = bf16(h @ W^T) are reduced
 * in the GEMM's epilogue (per workgroup: each top-k row's largest keys, the first-max key, max, sum-exp and finite
 * count) and never written; a second launch merges them per row and draws as vs_sample_batch does.
 *   h, ldh, W, ldw, N, K : as vs_lmhead_verify_greedy (h [R, ldh], W [N, ldw] bf16, K a multiple of 256)
 *   params : device array [R] of vs_row_params (u supplied). Served rows: greedy (VS_ROW_GREEDY, with
 *            VS_ROW_ARGMAX_VV the argmax over [0, vocab_valid)) and top-k rows with 1 <= top_k <= 64, temperature,
 *            top_p and min_p, with no logit edits. A row with bias or suppressed ids, an active stop range, penalties
 *            over a history, VS_ROW_FORCE or top_k off / above 64 is not computed: out_flags = VS_OUT_UNSUPPORTED
 *            (such a batch takes the head and vs_sample_batch).
 *   outputs: as vs_sample_batch (out_ids, out_logprob required; out_flags, out_keep may be NULL)
 *   ws     : device workspace of at least vs_lmhead_sample_workspace_bytes(R) bytes (no zeroing needed)
 * Replaces: volundr-mlx/volundr.py:958-968 (lm_head, bf16) feeding Sampler.sample (sampler.py:100-156) through the
 * decode step's per-row loop (scheduler.py:382-392, 416-425). */
int vs_lmhead_sample(const void* h, int64_t ldh, const void* W, int64_t ldw, int N, int K, int R,
                     const vs_row_params* params, int32_t* out_ids, float* out_logprob, uint32_t* out_flags,
                     int32_t* out_keep, void* ws, size_t ws_bytes, vs_stream_t stream);

size_t vs_lmhead_sample_workspace_bytes(int R);

/* The k largest logits of each of B rows, value descending, ties to the lower id (rows with fewer than k finite
 * logits pad with id -1 and value -inf). 1 <= k <= 256 (less when V needs many workgroups per row; the call fails
 * with VS_EINVAL above the shape's limit). Values are the logits widened to float32.
 *   out_ids : int32 [B, k];  out_vals : float32 [B, k]
 *   ws      : as for vs_sample_batch (vs_sample_workspace_bytes(B, V), zeroed once)
 * Replaces: volundr-mlx/spec/dflash.py:232-236 (argpartition + take_along_axis + argsort of the drafter logits). */
int vs_topk_batch(const void* logits, int dtype, int B, int V, int64_t ld, int k, int32_t* out_ids, float* out_vals,
                  void* ws, size_t ws_bytes, vs_stream_t stream);

/* The drafter's greedy candidate walk for n blocks of S <= 8 slots with K <= 16 candidates each:
 *   pred = anchor[b]; for e < S: s[c] = uval[b,e,c] + sum_r B[cid[b,e,c]][r] * float32(A[pred][r] * hp[b,e,r]);
 *   pred = cid[b,e, first argmax of s]; out[b,e] = pred.
 *   uval, cid : float32 / int32 [n, S, ldk] (ldk >= K);  hp : float32 [n, S, R];  anchor : int32 [n] (device)
 *   A, B      : bf16 [vocab, R] codebooks, R a multiple of 16 in [16, 256]
 * Candidates with ids outside [0, vocab) never win; a slot with no valid candidate, and every slot after it,
 * outputs -1 (as does every slot of a block whose anchor is outside [0, vocab)). Sums are fp32 in a fixed order
 * of this build (the reference's matmul order is its own): picks agree except between scores within rounding.
 * Replaces: volundr-mlx/spec/dflash.py:50-60 (_walk). */
int vs_draft_walk(const float* uval, const int32_t* cid, int ldk, const float* hp, const void* A, const void* B,
                  int vocab, int R, const int32_t* anchor, int n, int S, int K, int32_t* out, vs_stream_t stream);

/* DFlash2 propose for n blocks: the top-16 of each of the n*S logit rows (row (b,e) starts at element
 * (b*S + e)*ld, the first V entries are the valid vocabulary), then vs_draft_walk over them. out : int32 [n, S].
 *   ws : device workspace of at least vs_draft_workspace_bytes(n, S, V) bytes (about 20 MB + 128 B per row),
 *        zeroed once beforehand
 * Replaces: volundr-mlx/spec/dflash.py:228-240 (DFlash2Drafter.propose after the head: top-16, sort, _walk). */
int vs_draft_propose(const void* logits, int dtype, int n, int S, int V, int64_t ld, const float* hp, const void* A,
                     const void* B, int vocab, int R, const int32_t* anchor, int32_t* out, void* ws, size_t ws_bytes,
                     vs_stream_t stream);

size_t vs_draft_workspace_bytes(int n, int S, int V);

/* The inter-workgroup waits of vs_sample_batch / vs_sample_batch_state (row barriers of rows with top-k off or above
 * 256) give up after 200 us (5 ms under a cooperative launch), measured on the GPU's 100 MHz real-time counter, and
 * flag their row VS_OUT_TIMEOUT. A testing hook: a non-zero `polls` also bounds each wait of later plain launches of
 * the process by that many polls (0 restores the time bound alone), so a tiny limit forces the timeout path, whose
 * rows report VS_OUT_TIMEOUT, commit no request state and leave the workspace zeroed. No counterpart in the
 * reference (its sampler is single-threaded host code). */
int vs_set_spin_limit(unsigned polls);

/* Testing flags for later calls of the process (0 restores the default behaviour). VS_DEBUG_FORCE_RADIX: rows of
 * the FULL class (top-k off or above 256) with large kept sets resolve top-p and the draw with the cooperative radix
 * select, the fallback otherwise reached only with min-p or with value bins too full to refine.
 * VS_DEBUG_SPIN_LATER_BARRIERS: the spin limit of vs_set_spin_limit applies only from a row's second barrier on, so
 * that every workgroup passes the first and some give up at a later one while others pass it.
 * VS_DEBUG_WAIT_CLOCK: every row barrier is treated as unreachable, so each wait ends at its time bound (measures
 * the bound; every such row reports VS_OUT_TIMEOUT). VS_DEBUG_NO_XCD_EXCHANGE: the workgroups of a row exchange their
 * data through the device-coherent level even when they all run on one XCD (the default then uses that XCD's L2;
 * results are identical either way). VS_DEBUG_FAKE_XCD_SPLIT: in launches that use the XCD's L2, every row's last
 * workgroup reports a neighbouring XCD, so the placement guard flags each such row VS_OUT_TIMEOUT (the path taken
 * if the dispatcher ever split a row across XCDs). No counterpart in the reference. */
enum {
  VS_DEBUG_FORCE_RADIX = 1u,
  VS_DEBUG_SPIN_LATER_BARRIERS = 2u,
  VS_DEBUG_WAIT_CLOCK = 4u,
  VS_DEBUG_NO_XCD_EXCHANGE = 8u,
  VS_DEBUG_FAKE_XCD_SPLIT = 16u
};
int vs_set_debug(unsigned flags);

/* on != 0: the calling thread's later sampling calls launch cooperatively (every workgroup of the grid resident at
 * once, so a row barrier cannot starve when other streams hold CUs; ~18 us more per call); 0: plain launches (the
 * default, unless the environment sets VS_COOPERATIVE=1, which makes every call of the process cooperative). The
 * setting is per thread. Returns the calling thread's previous setting (0 or 1), so a caller can restore it. The
 * Python layer uses it to retry a call whose rows reported VS_OUT_TIMEOUT. No counterpart in the reference. */
int vs_set_cooperative(int on);

/* Launch `reps` empty kernels of `blocks` workgroups of `threads` threads with `lds_bytes` of dynamic LDS back to
 * back on `stream` from one host call: a measurement hook (the launch floor a kernel of that shape pays; reps > 1
 * takes the caller's per-call host overhead out of the figure). No counterpart in the reference. */
int vs_launch_floor(int blocks, int threads, size_t lds_bytes, int reps, vs_stream_t stream);

/* Read `bytes` (a multiple of 16, 16-byte aligned) once with `blocks` 512-thread workgroups, each over a contiguous
 * share, eight 16-byte loads per lane in flight: a measurement hook (the streaming rate a kernel that reads its
 * bytes once, such as the lm_head weight stream, can reach). `out` (device, >= blocks words) is written only on an
 * impossible value. No counterpart in the reference. */
int vs_stream_read(const void* p, size_t bytes, int blocks, uint32_t* out, vs_stream_t stream);

/* Write, for each of `blocks` workgroups of `threads` threads, the id of the XCD it runs on (out: device, >= blocks
 * words): a placement check. The sampling kernel lets the workgroups of a row exchange data through their XCD's L2
 * when the grid puts each row on one XCD, which holds when workgroups b and b + 8 always share an XCD. No
 * counterpart in the reference. */
int vs_xcd_ids(uint32_t* out, int blocks, int threads, vs_stream_t stream);

/* Zero a workspace (stream-ordered). */
int vs_workspace_init(void* ws, size_t bytes, vs_stream_t stream);

/* Text of the calling thread's last error ("" if none). */
const char* vs_last_error(void);

/* Library ABI version (increments on any signature or struct change): 10. */
int vs_version(void);

#ifdef __cplusplus
}
#endif

#endif /* VOLUNDR_SAMPLING_H */
