"""Per-request sampler state kept on the device (vs_sample_batch_state, include/volundr_sampling.h).

Sampler (volundr-mlx/sampler.py:58-98) keeps three things per request on the host: the xorshift64* state behind
uniform(), the counts that accept() builds, and produced. DeviceSamplers keeps them in device memory for a fixed
set of requests, so that a serving loop's step is one kernel launch with nothing uploaded: the kernel draws
uniform() itself, reads the request's token history from a device pool for the penalties, applies the
min_new_tokens stop mask from its own produced count, and appends the chosen token (Sampler.accept) before it
returns. Requests with a reasoning budget stay on the host Sampler (the budget's force/bias decisions are host
logic, sampler.py:18-55).
"""
from __future__ import annotations

from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import STATE_DTYPE, check
from .ops import _DTYPES, SampleOut, _require_cuda, _stream_handle, alloc_out, argmax_only_ok, pack_rows, workspace
from .sampler import TokenHistory


class DeviceSamplers:
    """Device-resident state of the samplers of B requests, one row each.

    samplers : host Sampler objects (volundr_amd.Sampler); their rng, history and produced seed the device state
    vocab    : the logits row length V the steps will be called with
    hist_cap : history slots reserved per request (a token accepted beyond it is flagged VS_OUT_HIST_FULL and not
               counted by later penalties)
    """

    def __init__(self, samplers: Sequence, vocab: int, hist_cap: int = 4096, device=None):
        if not samplers:
            raise ValueError("at least one sampler is required")
        for s in samplers:
            if getattr(s, "budget", None) is not None:
                raise ValueError("requests with a reasoning budget keep their state on the host Sampler")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.dev, self.V, self.B, self.cap = dev, int(vocab), len(samplers), int(hist_cap)
        self.samplers = list(samplers)
        st = np.zeros(self.B, dtype=STATE_DTYPE)
        pool = np.zeros(self.B * self.cap, dtype=np.int32)
        for r, s in enumerate(self.samplers):
            h = np.asarray(getattr(s, "history", []), dtype=np.int64)
            if h.size > self.cap:
                raise ValueError(f"request {r}: history of {h.size} tokens exceeds hist_cap {self.cap}")
            st[r]["rng"] = np.uint64(s.rng)
            st[r]["hist_off"] = r * self.cap
            st[r]["hist_len"] = h.size
            st[r]["hist_cap"] = self.cap
            st[r]["produced"] = int(s.produced)
            st[r]["min_new_tokens"] = int(s.sp.min_new_tokens)
            pool[r * self.cap:r * self.cap + h.size] = h
        self.state = torch.from_numpy(st.view(np.uint8).copy()).to(dev)
        self.pool = torch.from_numpy(pool).to(dev)
        # requests that need no logits take Sampler.choose's argmax over [:vocab_valid] (sampler.py:95-96) whenever
        # their stop mask is off; the kernel applies the mask while its own produced < min_new_tokens
        avv = [s.vv if argmax_only_ok(s.sp, s.vv) else None for s in self.samplers]
        self.rows = pack_rows([s.sp for s in self.samplers], np.zeros(self.B), self.V, stop_always=True,
                              argmax_vv=avv).to(dev)
        self.out = alloc_out(self.B, dev)
        L = _lib.load()
        self._ws = workspace(dev, L.vs_sample_workspace_bytes(self.B, self.V))

    def step(self, logits: torch.Tensor, out: Optional[SampleOut] = None) -> SampleOut:
        """Sampler.choose for every request on logits [B, V]: draw, choose, accept, all on the device."""
        _require_cuda(logits, "logits")
        if logits.shape != (self.B, self.V) or logits.stride(1) != 1:
            raise ValueError(f"logits must be [{self.B}, {self.V}] with unit stride along V")
        if logits.dtype not in _DTYPES:
            raise ValueError(f"unsupported logits dtype {logits.dtype}")
        out = out if out is not None else self.out
        L = _lib.load()
        ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
        rows = self.rows
        rc = L.vs_sample_batch_state(logits.data_ptr(), _DTYPES[logits.dtype], self.B, self.V, logits.stride(0),
                                     rows.params.data_ptr(), self.state.data_ptr(), self.pool.data_ptr(),
                                     ptr(rows.bias_ids), ptr(rows.bias_vals), ptr(rows.mask_ids),
                                     out.ids.data_ptr(), out.logprobs.data_ptr(), out.flags.data_ptr(),
                                     out.keep.data_ptr(), self._ws.data_ptr(), self._ws.numel(),
                                     _stream_handle(self.dev))
        check(rc, "vs_sample_batch_state")
        return out

    def bind(self, logits_slots: Sequence[torch.Tensor]):
        """A callable f(i) running step() on logits_slots[i] with every argument bound once (for serving loops that
        reuse the same buffers): one C call, no host checks."""
        for x in logits_slots:
            _require_cuda(x, "logits")
            if x.shape != (self.B, self.V) or x.stride(1) != 1 or x.dtype not in _DTYPES:
                raise ValueError(f"logits slots must be [{self.B}, {self.V}] rows of a supported dtype")
        fn = _lib.load().vs_sample_batch_state
        ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
        rows, out = self.rows, self.out
        slots = [x.data_ptr() for x in logits_slots]
        rest = (_DTYPES[logits_slots[0].dtype], self.B, self.V, logits_slots[0].stride(0), rows.params.data_ptr(),
                self.state.data_ptr(), self.pool.data_ptr(), ptr(rows.bias_ids), ptr(rows.bias_vals),
                ptr(rows.mask_ids), out.ids.data_ptr(), out.logprobs.data_ptr(), out.flags.data_ptr(),
                out.keep.data_ptr(), self._ws.data_ptr(), self._ws.numel(), _stream_handle(self.dev))
        keep = list(logits_slots)

        def call(i: int = 0) -> SampleOut:
            rc = fn(slots[i], *rest)
            if rc:
                check(rc, "vs_sample_batch_state")
            return keep and out

        return call

    def host_state(self) -> np.ndarray:
        """The device state as a STATE_DTYPE array (synchronises)."""
        return self.state.cpu().numpy().view(STATE_DTYPE).copy()

    def history(self, r: int):
        st = self.host_state()[r]
        off, n = int(st["hist_off"]), int(st["hist_len"])
        return [int(t) for t in self.pool[off:off + n].cpu().tolist()]

    def write_back(self):
        """Copy rng, counts/history and produced back into the host Sampler objects (synchronises)."""
        st = self.host_state()
        pool = self.pool.cpu().numpy()
        for r, s in enumerate(self.samplers):
            off, n = int(st[r]["hist_off"]), int(st[r]["hist_len"])
            h = [int(t) for t in pool[off:off + n]]
            s.rng = int(st[r]["rng"])
            s.history = TokenHistory(h)
            s.counts = {}
            for t in h:
                s.counts[t] = s.counts.get(t, 0) + 1
            s.produced = int(st[r]["produced"])
