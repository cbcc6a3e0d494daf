"""Token sampling with the call surface of volundr-mlx/sampler.py, computed by the HIP library.

`Sampler` keeps the reference's per-request state (the xorshift64* generator, the counts of generated tokens,
`produced`, the reasoning budget) on the host and runs Sampler.sample's arithmetic (sampler.py:100-156) on the GPU
through `ops.sample_batch`. Batched callers (the scheduler's per-row loop, scheduler.py:416-425) can instead call
`sample_rows_for` once for all rows that need the sampler.
"""
from __future__ import annotations

import time
from typing import Optional, Sequence

import numpy as np
import torch

from . import ops
from ._lib import OUT_NOFINITE, OUT_TIMEOUT, VsError

MASK = (1 << 64) - 1
SAMPLING_EPS = 1e-6


class Budget:
    """Reasoning budget (volundr-mlx/sampler.py:18-55): count tokens since `<|think|>` opened (in the prompt's last
    16 tokens, or generated); after n of them with no `<|/think|>`, force `<|/think|>` and mask `<|think|>` for the
    rest of the request; with a soft bias b, add b to the `<|/think|>` logit from 80% of the budget on."""

    def __init__(self, n, soft, prompt, start, end):
        self.start, self.end, self.n, self.soft = start, end, int(n), float(soft)
        tail = list(prompt[-16:])
        self.open = None
        # the last `start` in the tail opens the budget unless an `end` follows it
        for i in reversed(range(len(tail))):
            if tail[i] == start:
                if end not in tail[i + 1:]:
                    self.open = 0
                break
        self.closed = False
        self.forced = False

    def accept(self, j, t):
        if t == self.start:
            if self.open is None and not self.closed:
                self.open = j + 1
        elif t == self.end and self.open is not None:
            self.open = None
            self.closed = True

    def act(self, produced):
        """-> ("none" | "force" | "bias", payload) before sampling output token `produced`."""
        if self.closed:
            return ("bias", [(self.start, -np.inf)]) if self.forced else ("none", None)
        if self.open is None:
            return ("none", None)
        k = produced - self.open
        if k >= self.n:
            self.forced = self.closed = True
            self.open = None
            return ("force", self.end)
        if self.soft != 0.0 and k >= 0.8 * self.n:
            return ("bias", [(self.end, self.soft)])
        return ("none", None)


class Sampler:
    """Per-request sampler (volundr-mlx/sampler.py:58-156). Logits rows are GPU tensors; the arithmetic runs in
    vs_sample_batch. `last_logprob` holds log p of the last sampled token under the distribution drawn from."""

    def __init__(self, sp, prompt=(), think_ids=(None, None), vocab_valid=248077, request_id=0):
        self.sp, self.vv = sp, vocab_valid
        seed = sp.seed if sp.seed is not None else time.time_ns() ^ ((request_id * 0x9E3779B97F4A7C15) & MASK)
        self.rng = (int(seed) | 1) & MASK
        self.counts = {}
        self.history: list = []  # the accepted tokens, in order (the multiset behind `counts`)
        self.produced = 0
        self.budget = None
        self.last_logprob = None
        if sp.reasoning_budget and think_ids[0] is not None and think_ids[1] is not None:
            self.budget = Budget(sp.reasoning_budget, sp.reasoning_budget_soft_bias, prompt, *think_ids)

    def uniform(self) -> float:
        """xorshift64* (shifts 12, 25, 27; multiplier 0x2545F4914F6CDD1D), top 53 bits / 2^53 (sampler.py:69-75)."""
        r = self.rng
        r ^= r >> 12
        r ^= (r << 25) & MASK
        r ^= r >> 27
        self.rng = r
        return (((r * 0x2545F4914F6CDD1D) & MASK) >> 11) / float(1 << 53)

    def accept(self, tok):
        tok = int(tok)
        self.counts[tok] = self.counts.get(tok, 0) + 1
        self.history.append(tok)
        if self.budget is not None:
            self.budget.accept(self.produced, tok)
        self.produced += 1

    def _extra(self):
        """Budget action before sampling (sampler.py:85-92): ("force", tok) or the extra biases."""
        if self.budget is None:
            return None, []
        kind, v = self.budget.act(self.produced)
        if kind == "force":
            return v, []
        return None, (v if kind == "bias" else [])

    def choose(self, logits) -> int:
        """The next token from a logits row (GPU tensor [vocab]); records it (sampler.py:83-98)."""
        forced, extra = self._extra()
        if forced is not None:
            self.accept(forced)
            return forced
        if extra or self.sp.needs_logits(self.vv, self.produced):
            tok = self.sample(logits, extra)
        else:
            o = ops.verify_greedy(logits.reshape(1, 1, -1), None, vocab_valid=min(self.vv, logits.shape[-1]))
            tok = int(o.argmax[0, 0].item())
            self.last_logprob = float(o.logprobs[0, 0].item())
        self.accept(tok)
        return tok

    def sample(self, x, extra=()) -> int:
        """Sampler.sample (sampler.py:100-156) for one row; x is a GPU tensor [V] (a host array is uploaded)."""
        if not isinstance(x, torch.Tensor):
            x = torch.as_tensor(np.asarray(x, dtype=np.float32)).cuda()
        rng0 = self.rng
        u = self.uniform() if not self.sp.greedy else 0.0
        out = ops.sample_batch(x.reshape(1, -1), [self.sp], [u], [self.history], [self.produced], [list(extra)])
        flags = int(out.flags[0].item()) & 0xFFFFFFFF
        if flags & OUT_TIMEOUT:
            ops.reset_workspace(x.device)
            raise VsError("vs_sample_batch: an inter-workgroup wait timed out")
        if flags & OUT_NOFINITE:  # sampler.py:131-132 returns before drawing (:154): the generator is not advanced
            self.rng = rng0
        self.last_logprob = float(out.logprobs[0].item())
        return int(out.ids[0].item())


def sample_rows_for(logits: torch.Tensor, samplers: Sequence[Sampler], rows: Optional[Sequence[int]] = None):
    """One batched device call for the rows of logits [B, V] that the per-row loop of scheduler.py:416-425 would
    hand to Sampler.choose: returns the chosen token per sampler, updating each sampler's state exactly as
    `choose` does (the draw is consumed only by rows that sample)."""
    rows = list(range(len(samplers))) if rows is None else list(rows)
    toks: list = [None] * len(samplers)
    todo, sps, us, hists, prods, extras, rng0 = [], [], [], [], [], [], []
    for i, s in enumerate(samplers):
        forced, extra = s._extra()
        if forced is not None:
            s.accept(forced)
            toks[i] = forced
            continue
        todo.append(i)
        sp = s.sp
        if not (extra or sp.needs_logits(s.vv, s.produced)):
            # the GPU argmax over the valid vocabulary: a greedy row with no edits, same as the verify argmax
            sp = _ArgmaxOnly(sp)
        sps.append(sp)
        rng0.append(s.rng)
        us.append(s.uniform() if not sp.greedy else 0.0)
        hists.append(s.history if not isinstance(sp, _ArgmaxOnly) else [])
        prods.append(s.produced)
        extras.append(list(extra))
    if todo:
        sub = logits[[rows[i] for i in todo]]
        # argmax-only rows must not see columns >= vocab_valid (sampler.py:96 slices [:vv]); mask them to -inf
        need_vv = [k for k, sp in enumerate(sps) if isinstance(sp, _ArgmaxOnly) and samplers[todo[k]].vv < sub.shape[1]]
        if need_vv:
            sub = sub.clone()
            for k in need_vv:
                sub[k, samplers[todo[k]].vv:] = float("-inf")
        out = ops.sample_batch(sub, sps, us, hists, prods, extras)
        ids = out.ids.cpu().tolist()
        lps = out.logprobs.cpu().tolist()
        fl = out.flags.cpu().tolist()
        if any((f & 0xFFFFFFFF) & OUT_TIMEOUT for f in fl):
            ops.reset_workspace(logits.device)
            raise VsError("vs_sample_batch: an inter-workgroup wait timed out")
        for k, i in enumerate(todo):
            if (fl[k] & 0xFFFFFFFF) & OUT_NOFINITE:
                samplers[i].rng = rng0[k]  # no draw consumed (sampler.py:131-132)
            samplers[i].last_logprob = lps[k]
            samplers[i].accept(ids[k])
            toks[i] = ids[k]
    return toks


class _ArgmaxOnly:
    """A greedy view of a Sampling with no edits: the row takes np.argmax, first maximum."""

    def __init__(self, sp):
        self._sp = sp
        self.temperature, self.top_p, self.top_k, self.min_p = 1.0, 1.0, 1, 0.0
        self.presence_penalty = self.frequency_penalty = 0.0
        self.repetition_penalty = 1.0
        self.min_new_tokens = 0
        self.logit_bias, self.suppress_tokens, self.stop_token_ids = [], [], []
        self.greedy = True
