"""NumPy restatement of the reference sampler. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Follows volundr-mlx/sampler.py line by line; each step cites the reference line it restates. The one change of
interface: the uniform draw `u` in [0, 1) is an argument instead of `self.uniform()` (sampler.py:154), so the GPU
path and this oracle can be fed the same draw.

Build-defined outputs that the reference does not compute (sampler.py never returns a logprob):
  * sampled rows: logprob = log(pr[j] / z), the probability of the drawn token under the distribution actually
    drawn from (pr normalised at sampler.py:143, z = pr[:keep].sum() at :153);
  * greedy rows (sampler.py:127-128) and rows with no finite logit (:131-132): logprob = x[j] - logsumexp(x[finite])
    in float64 when x[j] is finite, else 0.0.
Diagnostics (also build-defined): whether the draw lies within 1e-6 of a CDF boundary (the north-star exemption),
whether the top-p cut lies within 1e-6 of a boundary, and whether the top-k cut splits a run of tied logits.

Pinning. tests/test_oracle.py checks this module against (a) hand-computed fp32 penalty values, (b) a pure-Python
brute force that sorts with `sorted()` and accumulates with `math.fsum`/`math.exp` on small vocabularies,
(c) special cases fixed by the definition (u=0 -> top token, u->1 -> last kept token, top_k=1 -> argmax, tiny top_p
-> top token, all -inf -> argmax 0), (d) the reference's own tie-order hand case (volundr-mlx/tests/test_volundr.py:
159-161: [1,3,3,2,3,-inf,3,-1], k=3 -> {1,2,4}), and (e) the published xorshift64* recurrence (Vigna 2016).
Parity unpinned: NumPy's argpartition choice among values tied at the k-th position (implementation-defined; this
oracle and the GPU both take the lower index, as the task mandates) and the exact float64 summation order of
np.sum / np.cumsum (covered by the 1e-5 / 1e-6 tolerances).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

MASK = (1 << 64) - 1
XS_MULT = 0x2545F4914F6CDD1D


@dataclass
class Params:
    """The sampling fields the sampler reads (volundr-mlx/session.py:439-456)."""
    temperature: float = 1.0
    top_p: float = 1.0
    top_k: Optional[int] = None
    min_p: float = 0.0
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    repetition_penalty: float = 1.0
    min_new_tokens: int = 0
    logit_bias: list = field(default_factory=list)
    suppress_tokens: list = field(default_factory=list)
    stop_token_ids: list = field(default_factory=list)

    @property
    def greedy(self):  # session.py:466-467
        return self.top_k == 1 or self.temperature < 1e-6


def xorshift64s_next(state: int):
    """One xorshift64* step (sampler.py:69-75): returns (new_state, uniform in [0,1))."""
    r = state
    r ^= r >> 12
    r ^= (r << 25) & MASK
    r ^= r >> 27
    return r, (((r * XS_MULT) & MASK) >> 11) / float(1 << 53)


def seed_state(seed: int) -> int:
    """sampler.py:62: rng = (seed | 1) & MASK."""
    return (int(seed) | 1) & MASK


def counts_from_history(hist) -> dict:
    """The `counts` dict that Sampler.accept builds (sampler.py:77-78) from a token history, in first-seen order."""
    c: dict = {}
    for t in (() if hist is None else hist):
        t = int(t)
        c[t] = c.get(t, 0) + 1
    return c


@dataclass
class Result:
    token: int
    logprob: float
    keep: int = 0             # tokens in the distribution drawn from (0 for greedy / no-finite rows)
    draw_boundary: bool = False
    topp_boundary: bool = False
    topk_tie: bool = False
    kind: str = "sample"      # "sample" | "greedy" | "nofinite"


def _logsoftmax_at(x: np.ndarray, j: int) -> float:
    xj = float(x[j])
    if not math.isfinite(xj):
        return 0.0
    f = x[np.isfinite(x)].astype(np.float64)
    m = f.max()
    return xj - (m + math.log(np.exp(f - m).sum()))


def preprocess(x, sp, counts: dict, produced: int = 0, extra=()):
    """sampler.py:102-126: logit edits and penalties, all in float32 (NumPy 2 / NEP 50 promotion)."""
    x = np.array(x, dtype=np.float32, copy=True)                     # :102
    V = x.shape[0]                                                    # :103
    for t, d in extra:                                                # :104-106
        if t < V:
            x[t] += np.float32(d)
    for t, b in sp.logit_bias:                                        # :107-109
        if t < V:
            x[t] += np.float32(b)
    sup = [t for t in sp.suppress_tokens if t < V]                    # :110-112
    if sup:
        x[np.asarray(sup)] = -np.inf
    if counts:                                                        # :113-122
        ids = np.fromiter(counts.keys(), dtype=np.int64)
        ids = ids[ids < V]
        c = np.asarray([counts[int(i)] for i in ids], dtype=np.float32)
        v = x[ids]
        if sp.repetition_penalty != 1.0:
            r = np.float32(sp.repetition_penalty)
            v = np.where(v > 0, v / r, v * r)
        v = v - (np.float32(sp.frequency_penalty) * c + np.where(c > 0, np.float32(sp.presence_penalty), 0))
        x[ids] = v.astype(np.float32)
    if produced < sp.min_new_tokens and sp.stop_token_ids:            # :123-126
        st = [t for t in sp.stop_token_ids if t < V]
        if st:
            x[np.asarray(st)] = -np.inf
    return x


def sample(x, sp, u: float, counts: Optional[dict] = None, produced: int = 0, extra=()) -> Result:
    """Sampler.sample (sampler.py:100-156) with the uniform draw `u` supplied."""
    x = preprocess(x, sp, counts or {}, produced, extra)
    if sp.greedy:                                                     # :127-128
        j = int(np.argmax(x))
        return Result(j, _logsoftmax_at(x, j), kind="greedy")
    t = np.float32(sp.temperature)                                    # :129
    idx = np.nonzero(np.isfinite(x))[0]                               # :130
    if idx.size == 0:                                                 # :131-132
        j = int(np.argmax(x))
        return Result(j, _logsoftmax_at(x, j), kind="nofinite")
    k = min(sp.top_k if sp.top_k else idx.size, idx.size)            # :133
    k = max(k, 1)                                                     # :134
    tie = False
    if k < idx.size:                                                  # :135-136
        # np.argpartition picks among values tied at the k-th position in an implementation-defined way; the
        # task's contract is "ties toward the lower index", which a stable argsort of -x gives exactly.
        order = np.argsort(-x[idx], kind="stable")
        tie = bool(x[idx][order[k - 1]] == x[idx][order[k]])
        idx = idx[order[:k]]
    elif idx.size > 4096:                                             # :137-139
        m = x[idx].max()
        idx = idx[x[idx] / t >= m / t - 40.0]
    idx = idx[np.lexsort((idx, -x[idx]))]                             # :140
    xs = (x[idx] / t).astype(np.float32)                              # :141
    pr = np.exp((xs - xs[0]).astype(np.float64))                      # :142
    pr /= pr.sum()                                                    # :143
    keep = pr.size                                                    # :144
    cs = np.cumsum(pr)
    topp_b = False
    if sp.top_p < 1.0:                                                # :145-148
        hit = np.nonzero(cs >= sp.top_p)[0]
        if hit.size:
            keep = int(hit[0]) + 1
            lo = cs[keep - 2] if keep >= 2 else 0.0
            topp_b = abs(cs[keep - 1] - sp.top_p) < 1e-6 or abs(lo - sp.top_p) < 1e-6
    if sp.min_p > 0.0:                                                # :149-152
        below = np.nonzero(pr < pr[0] * sp.min_p)[0]
        cnt = int(below[0]) if below.size else pr.size
        keep = min(keep, max(cnt, 1))
    z = pr[:keep].sum()                                               # :153
    uz = u * z                                                        # :154
    ck = np.cumsum(pr[:keep])
    j = int(np.searchsorted(ck, uz, side="left"))                     # :155
    j = min(j, keep - 1)                                              # :156
    lo = ck[j - 1] if j >= 1 else 0.0
    draw_b = abs(ck[j] - uz) < 1e-6 * z or (j >= 1 and abs(lo - uz) < 1e-6 * z)
    lp = math.log(pr[j] / z)
    return Result(int(idx[j]), lp, keep, draw_b, topp_b, tie)


def sample_plain(x, sp, u: float, counts: Optional[dict] = None, produced: int = 0, extra=()) -> int:
    """Sampler.sample (sampler.py:100-156) as the reference computes it, for timing only (bench.py's CPU baseline):
    np.argpartition for the top-k cut (:136) instead of the stable sort of `sample`, and no boundary diagnostics.
    Returns the token; equals `sample(...).token` except where values tie at the k-th position
    (tests/test_oracle.py checks this)."""
    x = preprocess(x, sp, counts or {}, produced, extra)              # :102-126
    if sp.greedy:                                                     # :127-128
        return int(np.argmax(x))
    t = np.float32(sp.temperature)                                    # :129
    idx = np.nonzero(np.isfinite(x))[0]                               # :130
    if idx.size == 0:                                                 # :131-132
        return int(np.argmax(x))
    k = max(min(sp.top_k if sp.top_k else idx.size, idx.size), 1)   # :133-134
    if k < idx.size:                                                  # :135-136
        idx = idx[np.argpartition(-x[idx], k - 1)[:k]]
    elif idx.size > 4096:                                             # :137-139
        m = x[idx].max()
        idx = idx[x[idx] / t >= m / t - 40.0]
    idx = idx[np.lexsort((idx, -x[idx]))]                             # :140
    xs = (x[idx] / t).astype(np.float32)                              # :141
    pr = np.exp((xs - xs[0]).astype(np.float64))                      # :142
    pr /= pr.sum()                                                    # :143
    keep = pr.size                                                    # :144
    if sp.top_p < 1.0:                                                # :145-148
        hit = np.nonzero(np.cumsum(pr) >= sp.top_p)[0]
        if hit.size:
            keep = int(hit[0]) + 1
    if sp.min_p > 0.0:                                                # :149-152
        below = np.nonzero(pr < pr[0] * sp.min_p)[0]
        cnt = int(below[0]) if below.size else pr.size
        keep = min(keep, max(cnt, 1))
    z = pr[:keep].sum()                                               # :153
    j = int(np.searchsorted(np.cumsum(pr[:keep]), u * z, side="left"))  # :154-155
    return int(idx[min(j, keep - 1)])                                 # :156


def sample_batch(X, params, u, hists=None, produced=None):
    """Row-by-row application of `sample` (the way scheduler.py:416-425 calls the sampler per batch row)."""
    out = []
    for i in range(X.shape[0]):
        c = counts_from_history(hists[i]) if hists is not None else {}
        out.append(sample(X[i], params[i], float(u[i]), c, 0 if produced is None else produced[i]))
    return out


# ---------------------------------------------------------------- Sampler.choose (sampler.py:83-98)
def budget_action(prompt, generated, n, soft, start, end):
    """The reasoning budget's action before output token p = len(generated) (volundr-mlx/sampler.py:18-55, driven
    by Sampler.choose / accept, sampler.py:77-92), derived from the whole token record instead of a state machine:

      * the span is open from the prompt when the last `start` among the prompt's final 16 tokens has no `end`
        after it (sampler.py:25-31); its origin is output position 0, and j0 = -1;
      * otherwise the first generated `start` (at j0) opens it with origin j0 + 1 (sampler.py:34-36);
      * the span is forced shut at position pf = origin + n (sampler.py:47-50): the forced token is `end`;
      * it closes by itself if an `end` is generated at some j with j0 < j < min(p, pf) (sampler.py:37-39).

    Returns ("none", None), ("force", end) or ("bias", [(id, value)]) as Budget.act does."""
    tail = list(prompt)[-16:]
    j0, origin = None, None
    if start in tail:
        last = len(tail) - 1 - tail[::-1].index(start)
        if end not in tail[last + 1:]:
            j0, origin = -1, 0
    if origin is None:
        if start not in generated:
            return ("none", None)
        j0 = list(generated).index(start)
        origin = j0 + 1
    p = len(generated)
    pf = origin + int(n)
    if end in list(generated)[j0 + 1:min(p, pf)]:
        return ("none", None)
    if p > pf:
        return ("bias", [(start, -np.inf)])
    if p == pf:
        return ("force", end)
    if float(soft) != 0.0 and p - origin >= 0.8 * int(n):
        return ("bias", [(end, float(soft))])
    return ("none", None)


def needs_logits(sp, vocab_valid: int, produced: int) -> bool:
    """Sampling.needs_logits (volundr-mlx/session.py:469-474)."""
    return (not sp.greedy or bool(sp.logit_bias) or sp.repetition_penalty != 1.0
            or sp.frequency_penalty != 0.0 or sp.presence_penalty != 0.0
            or (produced < sp.min_new_tokens and bool(sp.stop_token_ids))
            or any(t < vocab_valid for t in sp.suppress_tokens))


def choose(x, sp, vocab_valid: int, u: float, generated, prompt=(), think_ids=(None, None)) -> Result:
    """Sampler.choose (sampler.py:83-98) for one row x (the full logits row, float32) given the tokens the request
    has produced so far (`generated`, forced tokens included). `u` is the draw the row would consume. Returns the
    Result with kind "force" (budget, no draw), "argmax" (mx.argmax(x[:vv]), first maximum, no draw; logprob =
    x[j] - logsumexp(x[:vv])) or what `sample` returns."""
    extra = []
    if sp.reasoning_budget and think_ids[0] is not None and think_ids[1] is not None:      # :85-92
        kind, v = budget_action(prompt, generated, sp.reasoning_budget, sp.reasoning_budget_soft_bias, *think_ids)
        if kind == "force":
            return Result(int(v), 0.0, kind="force")
        if kind == "bias":
            extra = v
    produced = len(generated)
    if extra or needs_logits(sp, vocab_valid, produced):                                   # :93-94
        return sample(x, sp, u, counts_from_history(generated), produced, extra)
    xv = np.asarray(x, dtype=np.float32)[:vocab_valid]                                     # :95-96
    j = int(np.argmax(xv))
    return Result(j, _logsoftmax_at(xv, j), kind="argmax")
