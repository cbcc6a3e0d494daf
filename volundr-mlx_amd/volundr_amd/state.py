"""Per-request sampler state kept on the device, for a continuously changing batch (vs_sample_batch_state,
include/volundr_sampling.h).

Sampler (volundr-mlx/sampler.py:58-98) keeps three things per request on the host: the xorshift64* state behind
uniform(), the counts that accept() builds, and produced. The reference's engine creates one Sampler per request at
admission (scheduler.py:148-151) and calls choose() for whichever rows are live at each step (scheduler.py:402-425).
DeviceSamplers keeps that state in device tables with one slot per live request:

  * admit(sampler) gives the request a slot (its rng, history and produced are uploaded once); retire(slot) frees it
    and by default writes the state back into the Sampler. Only the rows of the changed slot move over PCIe.
  * step(logits) runs Sampler.choose for the live requests in `order` (row i of logits belongs to order[i]); or
    step(logits, slots) for any subset, in any order. The kernel draws uniform() itself, reads the request's token
    history from the device pool for the penalties, applies the min_new_tokens stop mask from its own produced
    count and appends the chosen token (Sampler.accept).
  * The reasoning budget (sampler.py:18-55, 85-92) stays host logic: before each step the host asks the request's
    Budget for its action, which needs no logits. A forced token goes to the device as a VS_ROW_FORCE row (recorded,
    no draw), a bias as the slot's bias entries (budget extra before logit_bias). The row is re-uploaded only when
    the action changes.
  * Histories never overflow: the host keeps an upper bound of every slot's history length and doubles the pool's
    per-slot capacity on the device before a step could fill it (Sampler.counts is unbounded, sampler.py:77-78).
  * A row whose row barrier timed out (VS_OUT_TIMEOUT: other work held the CUs its workgroups needed at once)
    committed nothing; step() repeats those rows once under a cooperative launch and raises only if that also times
    out (the recovery of Sampler.sample, sampler._sample_checked).

step(sync=True) copies the results back (one copy) and returns them as host lists, which is what an engine that
emits tokens needs every step; step(sync=False) returns the device outputs without waiting (no budget rows, and the
caller checks the flags). The host Sampler objects are refreshed by write_back() / retire().
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import OUT_HIST_FULL, OUT_TIMEOUT, ROW_DTYPE, STATE_DTYPE, VS_ROW_FORCE, VsError, check
from .ops import (_DTYPES, SampleOut, _require_cuda, _stream_handle, alloc_out, argmax_only_ok, coherent_exchange_fallback,
                  pack_rows,
                  reset_workspace, workspace)
from .sampler import TokenHistory

_NO_ACTION = ("none", None)
FOLD_AT = 256     # unmerged history tokens at which a slot's (id, count) table takes them in
FOLD_CHECK = 128  # steps between checks


@dataclass
class StepResult:
    """Host copies of one synchronous step's outputs (row i = the i-th slot of the step)."""
    ids: List[int]
    logprobs: List[float]
    flags: List[int]
    keep: List[int]
    out: SampleOut  # the kernel's outputs (pinned host memory, rewritten by the next step of as many rows)


def _alloc_out_host(n: int, dev: torch.device) -> SampleOut:
    """alloc_out in pinned host memory, which the kernel writes directly (the device addresses host memory)."""
    blk = torch.empty((4, n), dtype=torch.int32, pin_memory=dev.type == "cuda")
    return SampleOut(blk[0], blk[1].view(torch.float32), blk[2], blk[3], blk)


def _dev_copy(dst: torch.Tensor, src: np.ndarray):
    """Host array -> a slice of a device tensor (a byte tensor takes the array's bytes, a typed one its values)."""
    if src.size:
        a = np.ascontiguousarray(src)
        dst.copy_(torch.from_numpy(a.view(np.uint8).reshape(-1) if dst.dtype == torch.uint8 else a.reshape(-1)))


class DeviceSamplers:
    """Device-resident sampler state of a changing set of requests, one slot each.

    samplers : host Sampler objects (volundr_amd.Sampler) admitted at construction, in order (slots 0, 1, ...)
    vocab    : the logits row length V the steps will be called with
    hist_cap : initial history slots per request (the pool grows on the device when a request could fill it)
    capacity : initial number of slots (grows when more requests are admitted)
    grow_history : False keeps the pool's size fixed: a token accepted beyond hist_cap is then flagged
               VS_OUT_HIST_FULL and not counted by later penalties (a testing configuration)
    """

    def __init__(self, samplers: Sequence = (), vocab: int = 0, hist_cap: int = 4096, device=None,
                 capacity: Optional[int] = None, grow_history: bool = True):
        if vocab < 1:
            raise ValueError("vocab must be >= 1")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.dev, self.V = dev, int(vocab)
        self.grow_history = bool(grow_history)
        need = max(64, max((len(getattr(s, "history", ())) for s in samplers), default=0) + 64)
        cap = max(int(hist_cap), 1)
        if self.grow_history:
            cap = max(cap, need)
        self.cap = (cap + 63) // 64 * 64 if self.grow_history else cap
        self.S = max(int(capacity or 0), len(samplers), 1)
        self.EB = self.EM = 16  # bias / mask (suppress + stop) entries per slot
        self.slot_sampler: list = [None] * self.S
        self.order: List[int] = []  # live slots in admission order
        self._act: list = [None] * self.S  # the budget action each slot's uploaded row encodes
        self._edits: list = [None] * self.S  # per slot: (bias ids, bias vals, mask ids, n_supp) as uploaded
        self._hmax = np.zeros(self.S, dtype=np.int64)  # upper bound of each slot's device history length
        self._rawbase = np.zeros(self.S, dtype=np.int64)  # _hmax when the slot's table last took its history
        self._since_fold = 0  # steps since the tables were last checked
        self._budget = set()  # live slots whose request has a reasoning budget
        self._prod = [0] * self.S  # produced, as of the last synchronous step (budget rows need it)
        self.params_h = np.zeros(self.S, dtype=ROW_DTYPE)
        self._alloc_tables()
        self._slots_key = None  # the slots of the last step ...
        self._key_steps = 0     # ... the steps taken with them since _hmax was last brought up to date
        self._key_base = 0      # ... and their largest _hmax at that time
        self._keys: dict = {}   # slots tuple -> (index array, device int32 tensor, budget rows)
        self._host_out: dict = {}  # n -> (SampleOut in pinned host memory that synchronous steps write into, its
        #                            [4, n] int32 NumPy view, the flags as uint32, the logprobs as float32)
        self._argc: dict = {}  # the launch arguments of recent steps (keyed by every pointer they hold)
        self.out = alloc_out(max(len(samplers), 1), dev)
        for s in samplers:
            self.admit(s)

    # ------------------------------------------------------------------ tables
    def _alloc_tables(self):
        S, dev = self.S, self.dev
        self.params = torch.zeros(S * ROW_DTYPE.itemsize, dtype=torch.uint8, device=dev)
        self.state = torch.zeros(S * STATE_DTYPE.itemsize, dtype=torch.uint8, device=dev)
        self.pool = torch.zeros(S * self.cap, dtype=torch.int32, device=dev)
        # (id, count) tables: per slot a region of 4 * cap int32, two halves of `cap` pairs (vs_state_fold writes
        # the merged table to the half not in use)
        self.tabs = torch.zeros(S * 4 * self.cap, dtype=torch.int32, device=dev)
        self.bias_ids = torch.zeros(S * self.EB, dtype=torch.int32, device=dev)
        self.bias_vals = torch.zeros(S * self.EB, dtype=torch.float32, device=dev)
        self.mask_ids = torch.zeros(S * self.EM, dtype=torch.int32, device=dev)

    def _grow_slots(self, S2: int):
        """More slots: every table is re-allocated and the live slots' rows copied on the device."""
        old = (self.params, self.state, self.pool, self.tabs, self.bias_ids, self.bias_vals, self.mask_ids)
        S1 = self.S
        self.S = S2
        self._alloc_tables()
        for new, o in zip((self.params, self.state, self.pool, self.tabs, self.bias_ids, self.bias_vals,
                           self.mask_ids), old):
            new[:o.numel()].copy_(o)
        ph = np.zeros(S2, dtype=ROW_DTYPE)
        ph[:S1] = self.params_h
        self.params_h = ph
        for lst, fill in ((self.slot_sampler, None), (self._act, None), (self._edits, None), (self._prod, 0)):
            lst.extend([fill] * (S2 - S1))
        self._hmax = np.concatenate([self._hmax, np.zeros(S2 - S1, dtype=np.int64)])
        self._rawbase = np.concatenate([self._rawbase, np.zeros(S2 - S1, dtype=np.int64)])

    def _grow_history(self, need: int):
        """Per-slot history capacity >= need: a new pool and table pool, each slot's history and tables copied on the
        device, and every slot's hist_off / hist_cap / tab_off rewritten in place (stream-ordered before the next
        step)."""
        cap2 = self.cap
        while cap2 < need:
            cap2 *= 2
        S, cap1 = self.S, self.cap
        pool2 = torch.zeros(S * cap2, dtype=torch.int32, device=self.dev)
        pool2.view(S, cap2)[:, :cap1].copy_(self.pool.view(S, cap1))
        tabs2 = torch.zeros(S * 4 * cap2, dtype=torch.int32, device=self.dev)
        tabs2.view(S, 2, 2 * cap2)[:, :, :2 * cap1].copy_(self.tabs.view(S, 2, 2 * cap1))
        self.pool, self.tabs, self.cap = pool2, tabs2, cap2
        st64 = self.state.view(torch.int64).view(S, 6)
        q = torch.arange(S, dtype=torch.int64, device=self.dev)
        half = (st64[:, 4] % (4 * cap1)) // (2 * cap1)
        st64[:, 1].copy_(q * cap2)
        st64[:, 4].copy_(q * 4 * cap2 + half * 2 * cap2)
        self.state.view(torch.int32).view(S, 12)[:, 5].fill_(cap2)

    def _grow_edits(self, nb: int, nm: int):
        EB2, EM2 = self.EB, self.EM
        while EB2 < nb:
            EB2 *= 2
        while EM2 < nm:
            EM2 *= 2
        if (EB2, EM2) == (self.EB, self.EM):
            return
        self.EB, self.EM = EB2, EM2
        self.bias_ids = torch.zeros(self.S * EB2, dtype=torch.int32, device=self.dev)
        self.bias_vals = torch.zeros(self.S * EB2, dtype=torch.float32, device=self.dev)
        self.mask_ids = torch.zeros(self.S * EM2, dtype=torch.int32, device=self.dev)
        for q in range(self.S):  # every slot's entries move: re-pack and re-upload the live ones
            if self.slot_sampler[q] is not None:
                self._upload_row(q, self._act[q], force_edits=True)

    # ------------------------------------------------------------------ per-slot rows
    def _upload_row(self, q: int, action, force_edits: bool = False):
        """Pack slot q's params row for a budget action and upload what changed (params row, its edit entries)."""
        s = self.slot_sampler[q]
        sp = s.sp
        kind, val = action if action is not None else _NO_ACTION
        extra = list(val) if kind == "bias" else []
        avv = [s.vv] if (argmax_only_ok(sp, s.vv) and not extra) else None
        p = pack_rows([sp], [0.0], self.V, None, None, [extra], stop_always=True, argmax_vv=avv)
        nb, nm = p.bias_ids.size, p.mask_ids.size
        if nb > self.EB or nm > self.EM:
            self._act[q] = action
            self._grow_edits(nb, nm)  # re-uploads every live slot, this one included
            return
        row = p.params.copy()
        r = row[0]
        nsupp = int(r["supp_end"] - r["supp_begin"])
        b0, m0 = q * self.EB, q * self.EM
        r["bias_begin"], r["bias_end"] = b0, b0 + nb
        r["supp_begin"], r["supp_end"] = m0, m0 + nsupp
        r["stop_begin"], r["stop_end"] = m0 + nsupp, m0 + nm
        r["hist_begin"] = r["hist_end"] = 0
        if kind == "force":
            r["flags"] = int(r["flags"]) | VS_ROW_FORCE
            r["force_token"] = int(val)
        self.params_h[q] = r
        rb = ROW_DTYPE.itemsize
        _dev_copy(self.params[q * rb:(q + 1) * rb], row)
        edits = (p.bias_ids, p.bias_vals, p.mask_ids)
        prev = self._edits[q]
        if force_edits or prev is None or any(not np.array_equal(a, b) for a, b in zip(prev, edits)):
            _dev_copy(self.bias_ids[b0:b0 + nb], p.bias_ids)
            _dev_copy(self.bias_vals[b0:b0 + nb], p.bias_vals)
            _dev_copy(self.mask_ids[m0:m0 + nm], p.mask_ids)
            self._edits[q] = edits
        self._act[q] = action

    # ------------------------------------------------------------------ membership
    def admit(self, sampler, slot: Optional[int] = None) -> int:
        """Give a request a slot: its rng, history, produced and parameters are uploaded once. Returns the slot,
        which is appended to `order`."""
        if slot is None:
            free = [q for q in range(self.S) if self.slot_sampler[q] is None]
            if not free:
                self._grow_slots(2 * self.S)
                free = [q for q in range(self.S) if self.slot_sampler[q] is None]
            slot = free[0]
        elif not 0 <= slot < self.S or self.slot_sampler[slot] is not None:
            raise ValueError(f"slot {slot} is not a free slot")
        h = np.asarray(getattr(sampler, "history", []), dtype=np.int64).reshape(-1)
        if h.size + 1 > self.cap:
            if not self.grow_history:
                raise ValueError(f"history of {h.size} tokens exceeds hist_cap {self.cap}")
            self._grow_history(h.size + 64)
        q = slot
        self.slot_sampler[q] = sampler
        st = np.zeros(1, dtype=STATE_DTYPE)
        st[0]["rng"] = np.uint64(sampler.rng)
        st[0]["hist_off"] = q * self.cap
        st[0]["hist_len"] = h.size
        st[0]["hist_cap"] = self.cap
        st[0]["produced"] = int(sampler.produced)
        st[0]["min_new_tokens"] = int(sampler.sp.min_new_tokens)
        # the penalty counts of the history so far as a sorted (id, count) table (the content of Sampler.counts)
        ids, cnt = np.unique(h, return_counts=True) if h.size else (np.zeros(0, np.int64), np.zeros(0, np.int64))
        st[0]["tab_off"] = q * 4 * self.cap
        st[0]["tab_len"] = ids.size
        st[0]["hist_base"] = h.size
        sb = STATE_DTYPE.itemsize
        _dev_copy(self.state[q * sb:(q + 1) * sb], st)
        _dev_copy(self.pool[q * self.cap:q * self.cap + h.size], h.astype(np.int32))
        t0 = q * 4 * self.cap
        _dev_copy(self.tabs[t0:t0 + 2 * ids.size], np.stack([ids, cnt], axis=1).astype(np.int32).reshape(-1))
        self._flush()
        self._rawbase[q] = h.size
        self._hmax[q] = h.size
        self._prod[q] = int(sampler.produced)
        self._edits[q] = None
        self._upload_row(q, _NO_ACTION)
        if getattr(sampler, "budget", None) is not None:
            self._budget.add(q)
        self.order.append(q)
        return q

    def retire(self, slot: int, write_back: bool = True):
        """Free a slot (the request left the batch); by default its state is first copied into its Sampler."""
        if not 0 <= slot < self.S or self.slot_sampler[slot] is None:
            raise ValueError(f"slot {slot} is not live")
        if write_back:
            self._write_back_slots([slot])
        self.slot_sampler[slot] = None
        self._act[slot] = self._edits[slot] = None
        self._budget.discard(slot)
        self.order.remove(slot)
        self._flush()
        self._keys.clear()  # cached slot sets may name this slot

    @property
    def B(self) -> int:
        return len(self.order)

    @property
    def samplers(self):
        return [self.slot_sampler[q] for q in self.order]

    # ------------------------------------------------------------------ steps
    def _flush(self):
        """Bring the per-slot history bounds up to date with the steps taken since the slot set last changed."""
        if self._slots_key is not None and self._key_steps:
            self._hmax[self._keys[self._slots_key][0]] += self._key_steps
        self._slots_key, self._key_steps = None, 0

    def _prepare(self, slots: Sequence[int], sync: bool):
        """Budget actions, history capacity and the slots array for a step over `slots`. Returns the slots as a
        device int32 tensor."""
        key = tuple(slots)
        if key != self._slots_key:
            self._flush()
            ent = self._keys.get(key)
            if ent is None:
                for q in key:
                    if not 0 <= q < self.S or self.slot_sampler[q] is None:
                        raise ValueError(f"slot {q} is not live")
                if len(set(key)) != len(key):
                    raise ValueError("a request can take only one row of a step")
                if len(self._keys) >= 256:
                    self._keys.clear()
                # slots 0..n-1 in order need no slots array (the kernel then skips a dependent load)
                ident = key == tuple(range(len(key)))
                ent = (np.asarray(key, dtype=np.int64),
                       None if ident else torch.tensor(key, dtype=torch.int32).to(self.dev),
                       [(i, q) for i, q in enumerate(key) if q in self._budget])
                self._keys[key] = ent
            self._slots_key, self._key_base = key, int(self._hmax[ent[0]].max())
        ent = self._keys[key]
        if ent[2] and not sync:
            raise ValueError("requests with a reasoning budget need step(sync=True): the host decides the budget's "
                             "action from the tokens of the previous step")
        for _, q in ent[2]:
            act = self.slot_sampler[q].budget.act(self._prod[q])
            if act != self._act[q]:
                self._upload_row(q, act)
        need = self._key_base + self._key_steps + 1
        if need > self.cap and self.grow_history:
            self._grow_history(need + 64)
        self._since_fold += 1
        if self._since_fold >= FOLD_CHECK:
            self._fold_due()
        return ent[1]

    def _fold_due(self):
        """Merge the recent history of every slot with FOLD_AT or more tokens since its last merge into its (id, count)
        table (vs_state_fold, one launch). Checked every FOLD_CHECK steps, so a slot never holds more than
        FOLD_AT + FOLD_CHECK < 512 unmerged tokens."""
        key = self._slots_key
        self._flush()
        self._since_fold = 0
        due = [q for q in self.order if self._hmax[q] - self._rawbase[q] >= FOLD_AT]
        if due:
            st = torch.tensor(due, dtype=torch.int32).to(self.dev)
            L = _lib.load()
            check(L.vs_state_fold(self.state.data_ptr(), self.pool.data_ptr(), self.tabs.data_ptr(), self.cap,
                                  st.data_ptr(), len(due), _stream_handle(self.dev)), "vs_state_fold")
            for q in due:
                self._rawbase[q] = self._hmax[q]
            self._fold_keep = st  # alive until the launch has read it (the next fold replaces it)
        if key is not None:  # resume the current slot set's bookkeeping
            self._slots_key, self._key_base, self._key_steps = key, int(self._hmax[self._keys[key][0]].max()), 0

    def _launch(self, logits: torch.Tensor, slots_t: Optional[torch.Tensor], out: SampleOut):
        n = logits.shape[0]
        L = _lib.load()
        ws = workspace(self.dev, L.vs_sample_workspace_bytes(n, self.V))
        key = (logits.data_ptr(), logits.dtype, n, logits.stride(0), 0 if slots_t is None else slots_t.data_ptr(),
               out.ids.data_ptr(), ws.data_ptr(), self.pool.data_ptr(), self.params.data_ptr())
        a = self._argc.get(key)
        if a is None:
            if len(self._argc) >= 64:
                self._argc.clear()
            # every pointer of the call is in the key, the tables' own through params and pool (they are
            # re-allocated together), the stream through the workspace (one per stream)
            a = self._argc[key] = (
                logits.data_ptr(), _DTYPES[logits.dtype], n, self.V, logits.stride(0), self.params.data_ptr(),
                self.state.data_ptr(), self.pool.data_ptr(), self.tabs.data_ptr(),
                0 if slots_t is None else slots_t.data_ptr(), self.bias_ids.data_ptr(), self.bias_vals.data_ptr(),
                self.mask_ids.data_ptr(), out.ids.data_ptr(), out.logprobs.data_ptr(), out.flags.data_ptr(),
                out.keep.data_ptr(), ws.data_ptr(), ws.numel(), _stream_handle(self.dev))
        rc = L.vs_sample_batch_state(*a)
        if rc:
            check(rc, "vs_sample_batch_state")

    def _check_logits(self, logits: torch.Tensor, n: int):
        _require_cuda(logits, "logits")
        if logits.dim() != 2 or logits.shape != (n, self.V) or logits.stride(1) != 1:
            raise ValueError(f"logits must be [{n}, {self.V}] with unit stride along V")
        if logits.dtype not in _DTYPES:
            raise ValueError(f"unsupported logits dtype {logits.dtype}")

    def step(self, logits: torch.Tensor, slots: Optional[Sequence[int]] = None, sync: bool = True,
             out: Optional[SampleOut] = None):
        """Sampler.choose for the requests of `slots` (default: `order`) on logits [n, V], row i for slots[i]:
        draw, choose, accept, all on the device. sync=True returns a StepResult (host lists; timed-out rows
        repeated cooperatively; budget bookkeeping done); sync=False returns the device SampleOut at once."""
        slots = self.order if slots is None else slots
        n = len(slots)
        if n == 0:
            raise ValueError("no live requests to step")
        self._check_logits(logits, n)
        slots_t = self._prepare(slots, sync)
        hv = None
        if out is None:
            if sync:  # results land in pinned host memory: no copy, only the stream's completion is awaited
                hv = self._host_out.get(n)
                if hv is None:
                    o = _alloc_out_host(n, self.dev)
                    h = o.block.numpy()
                    hv = self._host_out[n] = (o, h, h[2].view(np.uint32), h[1].view(np.float32))
                out = hv[0]
            else:
                if self.out.ids.shape[0] != n:
                    self.out = alloc_out(n, self.dev)
                out = self.out
        self._launch(logits, slots_t, out)
        self._key_steps += 1
        if not sync:
            return out
        if hv is None:  # the caller's buffers
            if out.block.is_cuda:
                hb = torch.empty((4, n), dtype=torch.int32)
                hb.copy_(out.block)
            else:
                hb = out.block
                if self.dev.type == "cuda":
                    torch.cuda.current_stream(self.dev).synchronize()
            h = hb.numpy()
            hv = (out, h, h[2].view(np.uint32), h[1].view(np.float32))
        elif self.dev.type == "cuda":
            torch.cuda.current_stream(self.dev).synchronize()
        host, flv = hv[1], hv[2]
        fl = flv.tolist()
        anyf = 0
        for f in fl:
            anyf |= f
        if anyf & OUT_TIMEOUT:
            self._retry(logits, list(slots), np.nonzero(flv & OUT_TIMEOUT)[0], out)
            fl = flv.tolist()
            anyf = 0
            for f in fl:
                anyf |= f
        if anyf & OUT_HIST_FULL and self.grow_history:
            raise VsError("vs_sample_batch_state: a history slot was full (the pool should have grown)")
        ids = host[0].tolist()
        for i, q in self._keys[self._slots_key][2]:
            self.slot_sampler[q].budget.accept(self._prod[q], ids[i])
            self._prod[q] += 1
        return StepResult(ids, hv[3].tolist(), fl, host[3].tolist(), out)

    def _retry(self, logits, slots, bad, out):
        """Repeat the rows that reported VS_OUT_TIMEOUT (they committed nothing) under a cooperative launch; their
        results replace the flagged ones in `out`."""
        L = _lib.load()
        idx = bad.tolist()
        sub_t = torch.tensor([slots[i] for i in idx], dtype=torch.int32).to(self.dev)
        sub_x = logits[torch.tensor(idx, device=self.dev)].contiguous()
        sub_out = alloc_out(len(idx), self.dev)
        reset_workspace(self.dev)
        prev = L.vs_set_cooperative(1)
        try:
            self._launch(sub_x, sub_t, sub_out)
            sub = sub_out.block.cpu()
        finally:
            L.vs_set_cooperative(prev)
        if (sub[2].numpy().view(np.uint32) & OUT_TIMEOUT).any():
            # as in sampler._sample_checked: the device-coherent exchange from now on, and one more attempt
            reset_workspace(self.dev)
            coherent_exchange_fallback()
            self._launch(sub_x, sub_t, sub_out)
            sub = sub_out.block.cpu()
        if (sub[2].numpy().view(np.uint32) & OUT_TIMEOUT).any():
            reset_workspace(self.dev)
            raise VsError("vs_sample_batch_state: an inter-workgroup wait timed out, also under a cooperative launch")
        out.block[:, torch.tensor(idx, device=out.block.device)] = sub.to(out.block.device)

    def bind(self, logits_slots: Sequence[torch.Tensor]):
        """A callable f(i) running step(logits_slots[i], sync=False) for the current `order`, with every argument
        bound once (serving loops that reuse the same buffers and membership): one C call per step, and the host
        bookkeeping of step() (the history pool grows, the tables take in their recent tokens every FOLD_CHECK
        calls) done on a few integers. Not for requests with a reasoning budget."""
        n = len(self.order)
        for x in logits_slots:
            self._check_logits(x, n)
        if any(getattr(self.slot_sampler[q], "budget", None) is not None for q in self.order):
            raise ValueError("bind() does not serve requests with a reasoning budget; use step()")
        order = list(self.order)
        if self.out.ids.shape[0] != n:
            self.out = alloc_out(n, self.dev)
        fn = _lib.load().vs_sample_batch_state
        out = self.out
        ws = workspace(self.dev, _lib.load().vs_sample_workspace_bytes(n, self.V))
        slots = [x.data_ptr() for x in logits_slots]
        b = {"key": object()}  # no slot set yet: the first call binds

        def rebind():
            # the arguments of the launch; the pool and the tables move when the history grows
            slots_t = self._prepare(order, sync=False)
            b["key"] = self._slots_key
            b["rest"] = (_DTYPES[logits_slots[0].dtype], n, self.V, logits_slots[0].stride(0), self.params.data_ptr(),
                         self.state.data_ptr(), self.pool.data_ptr(), self.tabs.data_ptr(),
                         0 if slots_t is None else slots_t.data_ptr(), self.bias_ids.data_ptr(),
                         self.bias_vals.data_ptr(), self.mask_ids.data_ptr(), out.ids.data_ptr(),
                         out.logprobs.data_ptr(), out.flags.data_ptr(), out.keep.data_ptr(), ws.data_ptr(), ws.numel(),
                         _stream_handle(self.dev))
            b["keep"] = (list(logits_slots), slots_t, ws, self.params, self.state, self.pool, self.tabs,
                         self.bias_ids, self.mask_ids)

        def call(i: int = 0) -> SampleOut:
            if (self._slots_key is b["key"] and self._since_fold + 1 < FOLD_CHECK
                    and self._key_base + self._key_steps + 1 <= self.cap):
                self._since_fold += 1  # what _prepare would do for this slot set on this step
            else:
                rebind()
            rc = fn(slots[i], *b["rest"])
            if rc:
                check(rc, "vs_sample_batch_state")
            self._key_steps += 1
            return out

        return call

    # ------------------------------------------------------------------ host views
    def host_state(self) -> np.ndarray:
        """The device state of every slot as a STATE_DTYPE array (synchronises)."""
        return self.state.cpu().numpy().view(STATE_DTYPE).copy()

    def slot_state(self, slot: int):
        """(rng, hist_off, hist_len, produced) of one slot, read from the device (synchronises)."""
        sb = STATE_DTYPE.itemsize
        st = self.state[slot * sb:(slot + 1) * sb].cpu().numpy().view(STATE_DTYPE)[0]
        return int(st["rng"]), int(st["hist_off"]), int(st["hist_len"]), int(st["produced"])

    def history(self, slot: int):
        st = self.host_state()[slot]
        off, n = int(st["hist_off"]), int(st["hist_len"])
        return [int(t) for t in self.pool[off:off + n].cpu().tolist()]

    def _write_back_slots(self, slots):
        st = self.host_state()
        pool = self.pool.cpu().numpy()
        for q in slots:
            s = self.slot_sampler[q]
            off, n = int(st[q]["hist_off"]), int(st[q]["hist_len"])
            h = pool[off:off + n]
            s.rng = int(st[q]["rng"])
            s.history = TokenHistory(h)
            s.counts = {}
            for t in h.tolist():
                s.counts[t] = s.counts.get(t, 0) + 1
            s.produced = int(st[q]["produced"])

    def write_back(self):
        """Copy rng, counts/history and produced of every live slot back into its Sampler (synchronises)."""
        self._write_back_slots(list(self.order))
