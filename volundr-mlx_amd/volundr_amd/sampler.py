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

from . import _lib, ops
from ._lib import OUT_NOFINITE, OUT_TIMEOUT, VsError

MASK = (1 << 64) - 1
SAMPLING_EPS = 1e-6


class TokenHistory:
    """The accepted tokens of a request, in order, in a growable int32 buffer (list-like: append, len, iteration,
    indexing, equality with a list). `array()` is a view of the filled part, which the packing step reads without
    converting a Python list every step. Ids are checked to lie in [0, 2^31) when appended."""

    __slots__ = ("_buf", "_n")

    def __init__(self, tokens=()):
        a = np.asarray(list(tokens) if not isinstance(tokens, np.ndarray) else tokens, dtype=np.int64).reshape(-1)
        if a.size and (a.min() < 0 or a.max() >= 2**31):
            raise ValueError("token ids must lie in [0, 2^31)")
        self._buf = np.empty(max(64, 2 * a.size), dtype=np.int32)
        self._buf[:a.size] = a
        self._n = int(a.size)

    def append(self, tok):
        tok = int(tok)
        if tok < 0 or tok >= 2**31:
            raise ValueError("token ids must lie in [0, 2^31)")
        if self._n == self._buf.size:
            nb = np.empty(2 * self._buf.size, dtype=np.int32)
            nb[:self._n] = self._buf[:self._n]
            self._buf = nb
        self._buf[self._n] = tok
        self._n += 1

    def array(self) -> np.ndarray:
        return self._buf[:self._n]

    def __array__(self, dtype=None, copy=None):
        a = self.array()
        return a.astype(dtype) if dtype is not None else a.copy()

    def __len__(self):
        return self._n

    def __iter__(self):
        return iter(self.array().tolist())

    def __getitem__(self, i):
        if isinstance(i, slice):
            return self.array()[i].tolist()
        return int(self.array()[i])

    def __eq__(self, other):
        try:
            return list(self) == list(other)
        except TypeError:
            return NotImplemented

    def __repr__(self):
        return f"TokenHistory({self.array().tolist()})"


class Budget:
    """Reasoning budget of a request (behaviour of volundr-mlx/sampler.py:18-55), written as a four-state machine.

    States and what `act(produced)` answers before output token `produced` is chosen:
      IDLE    no think span is open                                      -> ("none", None)
      OPEN    a span opened at output position `origin`; with d = produced - origin:
                d >= n           -> becomes FORCED                       -> ("force", end)
                soft != 0 and d >= 0.8 n                                 -> ("bias", [(end, soft)])
                otherwise                                                -> ("none", None)
      CLOSED  the model closed the span itself                           -> ("none", None)
      FORCED  the budget closed it                                       -> ("bias", [(start, -inf)]) for good
    Transitions on `accept(j, tok)` (tok is output token j): `start` in IDLE opens the span at origin j + 1; `end` in
    OPEN closes it (CLOSED). CLOSED and FORCED never reopen. The start of a request: if the last `start` among the
    prompt's final 16 tokens is not followed there by `end`, the span is already OPEN with origin 0.
    """

    IDLE, OPEN, CLOSED, FORCED = range(4)

    def __init__(self, n, soft, prompt, start, end):
        self.start, self.end, self.n, self.soft = start, end, int(n), float(soft)
        self.state, self.origin = Budget.IDLE, 0
        window = list(prompt)[-16:]
        opens = [i for i, tok in enumerate(window) if tok == start]
        if opens and end not in window[opens[-1] + 1:]:
            self.state = Budget.OPEN

    # the reference's field names, read by callers that inspect the budget
    @property
    def open(self):
        return self.origin if self.state == Budget.OPEN else None

    @property
    def closed(self):
        return self.state in (Budget.CLOSED, Budget.FORCED)

    @property
    def forced(self):
        return self.state == Budget.FORCED

    def accept(self, j, t):
        if t == self.start:  # a start token is never also read as an end token
            if self.state == Budget.IDLE:
                self.state, self.origin = Budget.OPEN, j + 1
        elif t == self.end and self.state == Budget.OPEN:
            self.state = Budget.CLOSED

    def act(self, produced):
        """-> ("none" | "force" | "bias", payload) before sampling output token `produced`."""
        if self.state == Budget.FORCED:
            return ("bias", [(self.start, -np.inf)])
        if self.state != Budget.OPEN:
            return ("none", None)
        spent = produced - self.origin
        if spent >= self.n:
            self.state = Budget.FORCED
            return ("force", self.end)
        if self.soft != 0.0 and spent >= 0.8 * self.n:
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
        self.history = TokenHistory()  # the accepted tokens, in order (the multiset behind `counts`)
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
        self.history.append(tok)  # checks the id first, so a rejected id leaves every field unchanged
        self.counts[tok] = self.counts.get(tok, 0) + 1
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
        _, host = _sample_checked(x.reshape(1, -1), [self.sp], [u], [self.history], [self.produced], [list(extra)])
        if int(host[2, 0].view(np.uint32)) & OUT_NOFINITE:  # sampler.py:131-132 returns before drawing (:154)
            self.rng = rng0  # the generator is not advanced
        self.last_logprob = float(host[1, 0].view(np.float32))
        return int(host[0, 0])


def _sample_checked(logits, sps, us, hists, prods, extras, argmax_vv=None):
    """ops.sample_batch with the recovery of a row barrier that could not complete (VS_OUT_TIMEOUT: other work held
    the CUs a row's workgroups needed at once). The flagged call committed nothing and left its workspace zeroed, so
    it is repeated once with a cooperative launch, which makes every workgroup resident together; a second timeout
    raises VsError."""
    out = ops.sample_batch(logits, sps, us, hists, prods, extras, argmax_vv=argmax_vv)
    host = out.block.cpu().numpy()  # ids, logprobs (as int32 bits), flags, keep: one copy
    if not (host[2].view(np.uint32) & OUT_TIMEOUT).any():
        return out, host
    L = _lib.load()
    ops.reset_workspace(logits.device)
    prev = L.vs_set_cooperative(1)  # this thread's setting; other threads keep theirs
    try:
        out = ops.sample_batch(logits, sps, us, hists, prods, extras, argmax_vv=argmax_vv)
        host = out.block.cpu().numpy()
    finally:
        L.vs_set_cooperative(prev)
    if (host[2].view(np.uint32) & OUT_TIMEOUT).any():
        ops.reset_workspace(logits.device)
        raise VsError("vs_sample_batch: an inter-workgroup wait timed out, also under a cooperative launch")
    return out, host


def sample_rows_for(logits: torch.Tensor, samplers: Sequence[Sampler], rows: Optional[Sequence[int]] = None):
    """One batched device call for the rows of logits [B, V] that the per-row loop of scheduler.py:416-425 would
    hand to Sampler.choose: returns the chosen token per sampler, updating each sampler's state exactly as
    `choose` does (budget force and bias, sampler.py:85-92; the draw is consumed only by rows that sample; rows that
    need no logits take the argmax over [:vocab_valid], sampler.py:95-96)."""
    rows = list(range(len(samplers))) if rows is None else list(rows)
    toks: list = [None] * len(samplers)
    todo, sps, us, hists, prods, extras, rng0, avv = [], [], [], [], [], [], [], []
    for i, s in enumerate(samplers):
        forced, extra = s._extra()
        if forced is not None:
            s.accept(forced)
            toks[i] = forced
            continue
        todo.append(i)
        sp = s.sp
        argmax_only = not (extra or sp.needs_logits(s.vv, s.produced))
        sps.append(sp)
        rng0.append(s.rng)
        us.append(s.uniform() if not sp.greedy else 0.0)
        hists.append([] if argmax_only else s.history)
        prods.append(s.produced)
        extras.append(list(extra))
        avv.append(s.vv if argmax_only else None)
    if todo:
        sel = [rows[i] for i in todo]
        step = sel[1] - sel[0] if len(sel) > 1 else 1
        if step > 0 and sel == list(range(sel[0], sel[-1] + 1, step)):
            sub = logits[sel[0]:sel[-1] + 1:step]  # evenly spaced rows: a strided view, no gather copy
        else:
            sub = logits[sel]
        _, host = _sample_checked(sub, sps, us, hists, prods, extras, argmax_vv=avv)
        ids = host[0].tolist()
        lps = host[1].view(np.float32).tolist()
        fl = host[2].view(np.uint32).tolist()
        for k, i in enumerate(todo):
            if fl[k] & OUT_NOFINITE:
                samplers[i].rng = rng0[k]  # no draw consumed (sampler.py:131-132)
            samplers[i].last_logprob = lps[k]
            samplers[i].accept(ids[k])
            toks[i] = ids[k]
    return toks
