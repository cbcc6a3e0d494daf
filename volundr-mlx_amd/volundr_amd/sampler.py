"""Token sampling with the call surface of volundr-mlx/sampler.py, computed by the HIP library.

`Sampler` keeps the reference's per-request state (the xorshift64* generator, the counts of generated tokens,
`produced`, the reasoning budget) on the host and runs Sampler.sample's arithmetic (sampler.py:100-156) on the GPU
through `ops.sample_batch`. Batched callers (the scheduler's per-row loop, scheduler.py:416-425) can instead call
`sample_rows_for` once for all rows that need the sampler.
"""
from __future__ import annotations

import threading
import time
import weakref
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib, ops
from ._lib import OUT_FORCED, OUT_NOFINITE, OUT_TIMEOUT, VsError

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
    the HIP library. `last_logprob` holds log p of the last sampled token under the distribution drawn from.

    Once `choose` / `sample_rows_for` has served the request, its state (rng, the accepted tokens, produced) lives
    in a device pool and the kernel advances it there; the host fields are a cache refreshed when read (`rng`,
    `counts`, `history`, `produced` copy the device state back on first access after a device step). Assigning one of
    them, `uniform()` and `accept()` change the host state, which the pool then takes over again at the next device
    step (the state is uploaded once). Mutating `counts` or `history` in place is not seen by the pool."""

    def __init__(self, sp, prompt=(), think_ids=(None, None), vocab_valid=248077, request_id=0):
        self.sp, self.vv = sp, vocab_valid
        seed = sp.seed if sp.seed is not None else time.time_ns() ^ ((request_id * 0x9E3779B97F4A7C15) & MASK)
        self._vs = None     # [pool, slot, valid, finalizer] while a device pool holds this request's state
        self._ahead = False  # the pool has advanced the state past the host copy
        self._rng = (int(seed) | 1) & MASK
        self._counts = {}
        self._history = TokenHistory()  # the accepted tokens, in order (the multiset behind `counts`)
        self._produced = 0
        self.budget = None
        self.last_logprob = None
        if sp.reasoning_budget and think_ids[0] is not None and think_ids[1] is not None:
            self.budget = Budget(sp.reasoning_budget, sp.reasoning_budget_soft_bias, prompt, *think_ids)

    # ---- host cache of the device-held state
    def _pull(self):
        """Copy the state the device pool advanced back into the host fields (synchronises)."""
        if not self._ahead:
            return
        self._ahead = False
        pool, q = self._vs[0], self._vs[1]
        rng, off, n, produced = pool.slot_state(q)
        have = len(self._history)
        if n > have:
            for t in pool.pool[off + have:off + n].cpu().tolist():
                self._history.append(t)
                self._counts[t] = self._counts.get(t, 0) + 1
        self._rng, self._produced = rng, produced

    def _host_changed(self):
        if self._vs is not None:
            self._vs[2] = False  # the pool re-takes the host state before its next step
            self._vs[0]._epoch += 1  # and its cached slot lists are stale

    def _field(name):  # noqa: N805
        attr = "_" + name

        def get(self):
            self._pull()
            return getattr(self, attr)

        def put(self, v):
            self._pull()
            setattr(self, attr, TokenHistory(v) if name == "history" and not isinstance(v, TokenHistory) else v)
            self._host_changed()

        return property(get, put)

    rng = _field("rng")
    counts = _field("counts")
    history = _field("history")
    produced = _field("produced")
    del _field

    def uniform(self) -> float:
        """xorshift64* (shifts 12, 25, 27; multiplier 0x2545F4914F6CDD1D), top 53 bits / 2^53 (sampler.py:69-75)."""
        self._pull()
        r = self._rng
        r ^= r >> 12
        r ^= (r << 25) & MASK
        r ^= r >> 27
        self._rng = r
        self._host_changed()
        return (((r * 0x2545F4914F6CDD1D) & MASK) >> 11) / float(1 << 53)

    def accept(self, tok):
        self._pull()
        tok = int(tok)
        self._history.append(tok)  # checks the id first, so a rejected id leaves every field unchanged
        self._counts[tok] = self._counts.get(tok, 0) + 1
        if self.budget is not None:
            self.budget.accept(self._produced, tok)
        self._produced += 1
        self._host_changed()

    def choose(self, logits) -> int:
        """The next token from a logits row (GPU tensor [vocab]); records it (sampler.py:83-98). Runs as a one-row
        sample_rows_for: the request's state stays on the device between calls."""
        return sample_rows_for(logits.reshape(1, -1), [self])[0]

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
        # every workgroup was resident, so the rows' workgroups cannot all have shared one XCD: from now on the
        # process exchanges row data at the device-coherent level (ops.coherent_exchange_fallback)
        ops.reset_workspace(logits.device)
        ops.coherent_exchange_fallback()
        out = ops.sample_batch(logits, sps, us, hists, prods, extras, argmax_vv=argmax_vv)
        host = out.block.cpu().numpy()
        if (host[2].view(np.uint32) & OUT_TIMEOUT).any():
            ops.reset_workspace(logits.device)
            raise VsError("vs_sample_batch: an inter-workgroup wait timed out, also under a cooperative launch")
    return out, host


_pools: dict = {}  # (device index, V) -> DeviceSamplers holding the state of the Samplers these routes served
_pool_lock = threading.Lock()


def _release(pool, slot):
    pool._released.append(slot)  # drained (the slot retired) at the pool's next use


def _pool_for(dev: torch.device, V: int):
    from .state import DeviceSamplers

    key = (dev.index, int(V))
    p = _pools.get(key)
    if p is None:
        p = DeviceSamplers([], V, hist_cap=4096, device=dev, capacity=64)
        p._released = []
        p._epoch = 0  # bumped by every admission, release and host-side change of a Sampler it holds
        p._slot_cache = {}  # ids of a batch's Samplers -> (epoch, their slots)
        _pools[key] = p
    while p._released:
        p.retire(p._released.pop(), write_back=False)
        p._epoch += 1
    return p


def _slot_in(pool, s) -> int:
    """The pool slot holding Sampler s's state. A Sampler seen for the first time, or whose host state changed since
    the pool last stepped it, is (re)admitted: its host state is uploaded once; later steps upload nothing of it."""
    ent = s._vs
    if ent is not None and ent[0] is pool and ent[2]:
        return ent[1]
    if ent is not None:
        s._pull()
        ent[3].detach()
        ent[0].retire(ent[1], write_back=False)
        ent[0]._epoch += 1
        s._vs = None
    q = pool.admit(weakref.proxy(s))
    s._vs = [pool, q, True, weakref.finalize(s, _release, pool, q)]
    pool._epoch += 1
    return q


def sample_rows_for(logits: torch.Tensor, samplers: Sequence[Sampler], rows: Optional[Sequence[int]] = None):
    """One batched device call for the rows of logits [B, V] that the per-row loop of scheduler.py:416-425 would
    hand to Sampler.choose: returns the chosen token per sampler, updating each sampler's state exactly as
    `choose` does (budget force and bias, sampler.py:85-92; the draw is consumed only by rows that sample; rows that
    need no logits take the argmax over [:vocab_valid], sampler.py:95-96).

    The samplers' state lives on the device (a DeviceSamplers pool per device and vocabulary), so a step uploads
    nothing per request: the kernel draws, applies the penalties from the device history and records the token
    there; each Sampler's host fields are refreshed from the device when next read."""
    ops._require_cuda(logits, "logits")
    if not samplers:
        return []
    if rows is None and logits.shape[0] == len(samplers):
        sub = logits
    else:
        rows = list(range(len(samplers))) if rows is None else list(rows)
        if len(rows) != len(samplers):
            raise ValueError("one logits row per sampler is required")
        step = rows[1] - rows[0] if len(rows) > 1 else 1
        if step > 0 and rows == list(range(rows[0], rows[-1] + 1, step)):
            sub = logits[rows[0]:rows[-1] + 1:step]  # evenly spaced rows: a strided view, no gather copy
        else:
            sub = logits[rows]
    if sub.stride(-1) != 1:
        sub = sub.contiguous()
    with _pool_lock:
        pool = _pool_for(logits.device, logits.shape[-1])
        # keyed by object ids, which hold no reference: an id is reused only after its Sampler died, and that
        # death queued a release, which bumps the epoch before this lookup (_pool_for drains the releases)
        key = tuple(map(id, samplers))
        ent = pool._slot_cache.get(key)
        if ent is not None and ent[0] == pool._epoch:
            slots = ent[1]
        else:
            slots = [e[1] if (e := s._vs) is not None and e[0] is pool and e[2] else _slot_in(pool, s)
                     for s in samplers]
            if len(pool._slot_cache) >= 64:
                pool._slot_cache.clear()
            pool._slot_cache[key] = (pool._epoch, slots)
        res = pool.step(sub, slots)
        for s, lp, f in zip(samplers, res.logprobs, res.flags):
            s._ahead = True
            if not f & OUT_FORCED:
                s.last_logprob = lp
    return res.ids
