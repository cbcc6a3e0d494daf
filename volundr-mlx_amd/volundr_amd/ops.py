"""Batched device entry points over torch tensors: sample_batch (Sampler.sample for B rows) and verify_greedy.

Torch is the plumbing (device memory, the current stream); the arithmetic is in libvolundr_sampling.so, called
through its C ABI with raw device pointers. No CPU fallback exists: a missing library or a CPU tensor raises.
"""
from __future__ import annotations

import math
import threading
import warnings
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import ROW_DTYPE, VS_BF16, VS_F16, VS_F32, VS_ROW_ARGMAX_VV, VS_ROW_GREEDY, VS_ROW_HIST_PAIRS, check

_DTYPES = {torch.float32: VS_F32, torch.bfloat16: VS_BF16, torch.float16: VS_F16}
_ws_lock = threading.Lock()
_ws: dict = {}


def _stream_handle(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def workspace(dev: torch.device, nbytes: int, kind: str = "sample") -> torch.Tensor:
    """A zeroed workspace of >= nbytes for (device, current stream, kind); grown and re-zeroed on demand. The
    sampling and verify kernels keep different layouts, so each has its own."""
    key = (dev.index, _stream_handle(dev), kind)
    with _ws_lock:
        w = _ws.get(key)
        if w is None or w.numel() < nbytes:
            w = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=dev)
            check(_lib.load().vs_workspace_init(w.data_ptr(), w.numel(), key[1]), "vs_workspace_init")
            _ws[key] = w
        return w


_stage_lock = threading.Lock()
_stage: dict = {}


def _staging(dev: torch.device, nbytes: int):
    """A pinned host buffer of >= nbytes for uploads to `dev` (one per device, reused; the caller holds
    _stage_lock from here until its copy is issued and recorded): waits until the copy that last read it has
    finished, so the caller may overwrite it. Returns the [buffer, event] entry."""
    ent = _stage.get(dev.index)
    if ent is None or ent[0].numel() < nbytes:
        if ent is not None and ent[1] is not None:
            ent[1].synchronize()
        ent = [torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, pin_memory=True), None]
        _stage[dev.index] = ent
    if ent[1] is not None:
        ent[1].synchronize()
    return ent


def reset_workspace(dev: torch.device, kind: str = "sample"):
    """Re-zero a workspace of (device, current stream), e.g. after a row reported VS_OUT_TIMEOUT."""
    key = (dev.index, _stream_handle(dev), kind)
    with _ws_lock:
        w = _ws.get(key)
        if w is not None:
            check(_lib.load().vs_workspace_init(w.data_ptr(), w.numel(), key[1]), "vs_workspace_init")


def coherent_exchange_fallback():
    """Make every later sampling launch of the process exchange row data at the device-coherent level
    (VS_DEBUG_NO_XCD_EXCHANGE). The retry paths call it when rows still report VS_OUT_TIMEOUT under a cooperative
    launch: with every workgroup resident, that means the placement guard saw a row whose workgroups did not share
    one XCD. It replaces any testing flags set with vs_set_debug."""
    L = _lib.load()
    L.vs_set_debug(_lib.DEBUG_NO_XCD_EXCHANGE)
    warnings.warn("volundr_amd: rows reported VS_OUT_TIMEOUT under a cooperative launch; sampling now exchanges row "
                  "data at the device-coherent level (VS_DEBUG_NO_XCD_EXCHANGE)", RuntimeWarning, stacklevel=3)


def _require_cuda(t: torch.Tensor, name: str):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the token-selection path runs only on the HIP device)")


def _wrap_id(t: int, V: int) -> Optional[int]:
    """NumPy indexing of a [V] row by a single id that passed the reference's `t < V` test (negative ids index from
    the end; below -V NumPy raises)."""
    t = int(t)
    if t >= V:
        return None
    if t < 0:
        if t < -V:
            raise IndexError(f"index {t} is out of bounds for axis 0 with size {V}")
        t += V
    return t


@dataclass
class PackedRows:
    """Host-packed per-row inputs of vs_sample_batch (numpy), see pack_rows."""
    params: np.ndarray      # ROW_DTYPE [B]
    hist: np.ndarray        # int32
    bias_ids: np.ndarray    # int32
    bias_vals: np.ndarray   # float32
    mask_ids: np.ndarray    # int32

    def to(self, dev) -> "DeviceRows":
        """One host-to-device copy: the five arrays laid end to end (each at a 256-byte offset) in one staging
        buffer, viewed back into typed device tensors."""
        parts = [self.params.view(np.uint8).reshape(-1)] + [np.ascontiguousarray(a).view(np.uint8).reshape(-1)
                                                            for a in (self.hist, self.bias_ids, self.bias_vals,
                                                                      self.mask_ids)]
        offs, n = [], 0
        for p in parts:
            offs.append(n)
            n += (p.size + 255) // 256 * 256
        n = max(n, 256)
        dev = torch.device(dev)
        buf = torch.empty(n, dtype=torch.uint8, device=dev)
        with _stage_lock:
            ent = _staging(dev, n)
            host = ent[0].numpy()
            for o, p in zip(offs, parts):
                host[o:o + p.size] = p
            buf.copy_(ent[0][:n], non_blocking=True)  # from pinned memory: asynchronous, on the current stream
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(dev))
            ent[1] = ev  # the buffer is overwritten only once this copy has completed

        def view(i, dt):
            sz = parts[i].size
            return buf[offs[i]:offs[i] + sz].view(dt) if sz else None
        return DeviceRows(buf[:parts[0].size], view(1, torch.int32), view(2, torch.int32), view(3, torch.float32),
                          view(4, torch.int32), len(self.params))


@dataclass
class DeviceRows:
    params: torch.Tensor
    hist: Optional[torch.Tensor]
    bias_ids: Optional[torch.Tensor]
    bias_vals: Optional[torch.Tensor]
    mask_ids: Optional[torch.Tensor]
    B: int


def argmax_only_ok(sp, vocab_valid: int) -> bool:
    """True when Sampling.needs_logits(vocab_valid, produced) (session.py:469-474) is False for some produced count:
    a greedy request with no bias, neutral penalties and no suppressed id below vocab_valid. Whether its stop mask
    is active (produced < min_new_tokens) is the one per-step condition left; the kernel decides it."""
    return (sp.greedy and not sp.logit_bias and sp.repetition_penalty == 1.0 and sp.frequency_penalty == 0.0
            and sp.presence_penalty == 0.0 and not any(t < vocab_valid for t in sp.suppress_tokens))


def _pairs_of(hr) -> np.ndarray:
    """Penalty counts as int32 (id, count) pairs, ids ascending: from a counts dict (Sampler.counts) or a history."""
    if isinstance(hr, dict):
        if not hr:
            return np.zeros(0, np.int32)
        ids = np.fromiter(hr.keys(), dtype=np.int64, count=len(hr))
        cnt = np.fromiter(hr.values(), dtype=np.int64, count=len(hr))
        o = np.argsort(ids, kind="stable")
        ids, cnt = ids[o], cnt[o]
    else:
        h = hr.array() if hasattr(hr, "array") else np.asarray([] if hr is None else hr, dtype=np.int64).reshape(-1)
        if h.size == 0:
            return np.zeros(0, np.int32)
        ids, cnt = np.unique(h, return_counts=True)
    if ids.size and (ids.min() < 0 or ids.max() >= 2**31 or cnt.max() >= 2**31):
        raise ValueError("counts must hold ids in [0, 2^31) and counts below 2^31")
    return np.stack([ids, cnt], axis=1).astype(np.int32).reshape(-1)


def pack_rows(samplings: Sequence, u, V: int, histories=None, produced=None, extras=None,
              stop_always: bool = False, argmax_vv=None, hist_pairs: bool = False) -> PackedRows:
    """Pack the per-row parameters the way Sampler.sample reads them (volundr-mlx/sampler.py:100-156).

    samplings : Sampling-like objects (session.Sampling); u : B uniform draws in [0, 1)
    histories : per-row token histories (iterables of ints: the tokens Sampler.accept recorded) or None
    produced  : per-row Sampler.produced (the min_new_tokens stop mask, sampler.py:123), default 0
    extras    : per-row budget biases [(id, bias)] applied before logit_bias (sampler.py:104-106)
    stop_always : pack the stop ids of every row with min_new_tokens > 0 whatever `produced` is (the state entry
                  point applies them while its device-side produced < min_new_tokens)
    argmax_vv : per-row vocab_valid or None: a row given one is a request that needs no logits while its stop mask
                is off, and then takes mx.argmax(logits[:vv]) as Sampler.choose does (sampler.py:95-96); its
                Sampling must pass argmax_only_ok and it must carry no extras
    hist_pairs : pass each row's penalty counts as a sorted (id, count) table (VS_ROW_HIST_PAIRS) instead of the raw
                history; a history may then also be given as a counts dict (Sampler.counts)
    """
    B = len(samplings)
    u = np.asarray(u, dtype=np.float64).reshape(-1)
    if u.size != B:
        raise ValueError("one uniform draw per row is required")
    uf = u.tolist()
    rows, hist_parts, bias_i, bias_v, mask = [], [], [], [], []
    hpos = bpos = mpos = 0
    for r, sp in enumerate(samplings):
        k = sp.top_k if sp.top_k else 0          # sampler.py:133: None and 0 mean off
        if k < 0:
            k = 1                                # max(min(k, n), 1) == 1 for k < 0 (:134)
        flags = VS_ROW_GREEDY if sp.greedy else 0
        vv = V
        vvr = None if argmax_vv is None else argmax_vv[r]
        if vvr is not None:
            vvr = int(vvr)
            if vvr < 1:
                raise ValueError("vocab_valid must be >= 1")
            if not argmax_only_ok(sp, vvr) or (extras is not None and extras[r]):
                raise ValueError(f"row {r} needs the sampler's logits: it cannot take the argmax-only route")
            flags |= VS_ROW_ARGMAX_VV
            vv = min(vvr, V)
        hr = None if histories is None else histories[r]
        if hist_pairs or isinstance(hr, dict):
            h = _pairs_of(hr)
            if hpos % 2:  # pairs start at an even word
                hist_parts.append(np.zeros(1, np.int32))
                hpos += 1
            if h.size:
                flags |= VS_ROW_HIST_PAIRS
        elif hasattr(hr, "array"):
            h = hr.array()  # TokenHistory: int32, ids checked on append
        else:
            h = np.asarray([] if hr is None else hr, dtype=np.int64).reshape(-1)
            if h.size and (h.min() < 0 or h.max() >= 2**31):
                raise ValueError("token histories must hold ids in [0, 2^31)")
            h = h.astype(np.int32)
        hb = hpos
        if h.size:
            hist_parts.append(h)
            hpos += h.size
        # additive biases in application order: budget extra, then logit_bias (sampler.py:104-109)
        items = []
        for t, d in list(extras[r] if extras is not None and extras[r] else []) + list(sp.logit_bias):
            w = _wrap_id(t, V)
            if w is not None:
                items.append((w, np.float32(d)))
        bb = bpos
        if items:
            ids = np.asarray([i for i, _ in items], dtype=np.int32)
            vals = np.asarray([v for _, v in items], dtype=np.float32)
            o = np.argsort(ids, kind="stable")
            bias_i.append(ids[o])
            bias_v.append(vals[o])
            bpos += len(items)
        sb = mpos
        if sp.suppress_tokens:
            sup = sorted({w for w in (_wrap_id(t, V) for t in sp.suppress_tokens) if w is not None})
            mask.append(np.asarray(sup, dtype=np.int32))
            mpos += len(sup)
        se = mpos
        pr = 0 if produced is None else int(produced[r])
        if (stop_always or pr < sp.min_new_tokens) and sp.min_new_tokens > 0 and sp.stop_token_ids:
            st = sorted({w for w in (_wrap_id(t, V) for t in sp.stop_token_ids) if w is not None})
            mask.append(np.asarray(st, dtype=np.int32))
            mpos += len(st)
        # field order of ROW_DTYPE (vs_row_params)
        rows.append((sp.temperature, sp.repetition_penalty, sp.frequency_penalty, sp.presence_penalty,
                     min(int(k), 2**31 - 1), flags, float(sp.top_p), float(sp.min_p), uf[r], hb, hpos,
                     bb, bpos, sb, se, se, mpos, vv, 0))
    P = np.array(rows, dtype=ROW_DTYPE) if rows else np.zeros(0, dtype=ROW_DTYPE)
    cat = lambda xs, dt: np.concatenate(xs).astype(dt) if xs else np.zeros(0, dt)  # noqa: E731
    return PackedRows(P, cat(hist_parts, np.int32), cat(bias_i, np.int32), cat(bias_v, np.float32),
                      cat(mask, np.int32))


@dataclass
class SampleOut:
    ids: torch.Tensor       # int32 [B]
    logprobs: torch.Tensor  # float32 [B]
    flags: torch.Tensor     # int32 view of the uint32 VS_OUT_* bits [B]
    keep: torch.Tensor      # int32 [B]
    block: Optional[torch.Tensor] = None  # int32 [4, B] holding the four rows above, when allocated together


def alloc_out(B: int, dev) -> SampleOut:
    """The four outputs as rows of one [4, B] int32 block (logprobs viewed as float32), so one copy brings all back."""
    blk = torch.empty(4, B, dtype=torch.int32, device=dev)
    return SampleOut(blk[0], blk[1].view(torch.float32), blk[2], blk[3], blk)


def sample_rows(logits: torch.Tensor, rows: DeviceRows, out: Optional[SampleOut] = None) -> SampleOut:
    """vs_sample_batch on device-resident inputs (no host work besides the launch)."""
    _require_cuda(logits, "logits")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [B, V] with unit stride along V")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    B, V = logits.shape
    if B != rows.B:
        raise ValueError("params and logits disagree on B")
    dev = logits.device
    out = out if out is not None else alloc_out(B, dev)
    L = _lib.load()
    nbytes = L.vs_sample_workspace_bytes(B, V)
    ws = workspace(dev, nbytes)
    ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
    rc = L.vs_sample_batch(logits.data_ptr(), _DTYPES[logits.dtype], B, V, logits.stride(0), rows.params.data_ptr(),
                           ptr(rows.hist), ptr(rows.bias_ids), ptr(rows.bias_vals), ptr(rows.mask_ids),
                           out.ids.data_ptr(), out.logprobs.data_ptr(), out.flags.data_ptr(), out.keep.data_ptr(),
                           ws.data_ptr(), ws.numel(), _stream_handle(dev))
    check(rc, "vs_sample_batch")
    return out


def sample_batch(logits: torch.Tensor, samplings: Sequence, u, histories=None, produced=None,
                 extras=None, argmax_vv=None, hist_pairs: bool = False) -> SampleOut:
    """Sampler.sample (sampler.py:100-156) for every row of logits [B, V], with the uniform draws supplied (rows
    given an argmax_vv take Sampler.choose's argmax over [:vv] instead, see pack_rows)."""
    _require_cuda(logits, "logits")
    rows = pack_rows(samplings, u, logits.shape[-1], histories, produced, extras, argmax_vv=argmax_vv,
                     hist_pairs=hist_pairs).to(logits.device)
    return sample_rows(logits, rows)


@dataclass
class VerifyOut:
    argmax: torch.Tensor   # int32 [B, T]
    accept: torch.Tensor   # int32 [B]
    logprobs: torch.Tensor  # float32 [B, T]


def verify_greedy(logits: torch.Tensor, drafts: Optional[torch.Tensor], vocab_valid: Optional[int] = None,
                  out: Optional[VerifyOut] = None) -> VerifyOut:
    """Greedy verify (spec/specdec.py:326-327, scheduler.py:462-463): logits [B, T, V] (or [T, V]), drafts
    [B, T-1] int32 = inp[:, 1:] -> first-max argmax over [:vocab_valid], accept length, chosen-token logprob."""
    _require_cuda(logits, "logits")
    if logits.dim() == 2:
        logits = logits.unsqueeze(0)
    if logits.dim() != 3 or logits.stride(2) != 1 or logits.stride(0) != logits.shape[1] * logits.stride(1):
        raise ValueError("logits must be [B, T, V] with rows evenly strided")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    B, T, V = logits.shape
    vv = V if vocab_valid is None else int(vocab_valid)
    dev = logits.device
    if T > 1:
        if drafts is None:
            raise ValueError("drafts [B, T-1] are required when T > 1")
        _require_cuda(drafts, "drafts")
        drafts = drafts.reshape(B, T - 1).to(torch.int32).contiguous()
    if out is None:
        out = VerifyOut(torch.empty(B, T, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev),
                        torch.empty(B, T, dtype=torch.float32, device=dev))
    L = _lib.load()
    nbytes = L.vs_verify_workspace_bytes(B, T, V)
    ws = workspace(dev, nbytes, "verify")
    rc = L.vs_verify_greedy(logits.data_ptr(), _DTYPES[logits.dtype], B, T, V, logits.stride(1), vv,
                            drafts.data_ptr() if T > 1 else 0, out.argmax.data_ptr(), out.accept.data_ptr(),
                            out.logprobs.data_ptr(), ws.data_ptr(), ws.numel(), _stream_handle(dev))
    check(rc, "vs_verify_greedy")
    return out


def emitted(drafts_row, argmax_row, nacc: int):
    """Tokens one verify step emits for a request (specdec.py:335-336): accepted drafts + the bonus token."""
    return [int(t) for t in drafts_row[:nacc]] + [int(argmax_row[nacc])]


def fix_scale(V: int) -> float:
    """Fixed-point scale of the probability masses used by the cooperative select (mirrors the library)."""
    return math.ldexp(1.0, 63 - max(0, (V - 1).bit_length()))


class PreparedSample:
    """vs_sample_batch with every argument bound once (device-resident logits slots, params, outputs, workspace),
    for serving loops that call the same batch shape every step: __call__(i) launches on logits slot i with no
    host work besides the C call."""

    def __init__(self, logits_slots: Sequence[torch.Tensor], rows: DeviceRows, out: Optional[SampleOut] = None):
        x0 = logits_slots[0]
        _require_cuda(x0, "logits")
        B, V = x0.shape
        self.dev = x0.device
        self.out = out if out is not None else alloc_out(B, self.dev)
        L = _lib.load()
        self._fn = L.vs_sample_batch
        ws = workspace(self.dev, L.vs_sample_workspace_bytes(B, V))
        self._ws = ws
        ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
        self._slots = [x.data_ptr() for x in logits_slots]
        self._keep = (list(logits_slots), rows, self.out)
        self._rest = (_DTYPES[x0.dtype], B, V, x0.stride(0), rows.params.data_ptr(), ptr(rows.hist),
                      ptr(rows.bias_ids), ptr(rows.bias_vals), ptr(rows.mask_ids), self.out.ids.data_ptr(),
                      self.out.logprobs.data_ptr(), self.out.flags.data_ptr(), self.out.keep.data_ptr(),
                      ws.data_ptr(), ws.numel(), _stream_handle(self.dev))

    def __call__(self, slot: int = 0) -> SampleOut:
        rc = self._fn(self._slots[slot], *self._rest)
        if rc:
            check(rc, "vs_sample_batch")
        return self.out


class PreparedVerify:
    """vs_verify_greedy with every argument bound once (see PreparedSample)."""

    def __init__(self, logits_slots: Sequence[torch.Tensor], drafts: torch.Tensor, vocab_valid: Optional[int] = None):
        x0 = logits_slots[0]
        _require_cuda(x0, "logits")
        B, T, V = x0.shape
        self.dev = x0.device
        vv = V if vocab_valid is None else int(vocab_valid)
        drafts = drafts.reshape(B, T - 1).to(torch.int32).contiguous()
        self.out = VerifyOut(torch.empty(B, T, dtype=torch.int32, device=self.dev),
                             torch.empty(B, dtype=torch.int32, device=self.dev),
                             torch.empty(B, T, dtype=torch.float32, device=self.dev))
        L = _lib.load()
        self._fn = L.vs_verify_greedy
        ws = workspace(self.dev, L.vs_verify_workspace_bytes(B, T, V), "verify")
        self._slots = [x.data_ptr() for x in logits_slots]
        self._keep = (list(logits_slots), drafts, ws)
        self._rest = (_DTYPES[x0.dtype], B, T, V, x0.stride(1), vv, drafts.data_ptr(), self.out.argmax.data_ptr(),
                      self.out.accept.data_ptr(), self.out.logprobs.data_ptr(), ws.data_ptr(), ws.numel(),
                      _stream_handle(self.dev))

    def __call__(self, slot: int = 0) -> VerifyOut:
        rc = self._fn(self._slots[slot], *self._rest)
        if rc:
            check(rc, "vs_verify_greedy")
        return self.out


def topk_batch(logits: torch.Tensor, k: int):
    """(ids int32 [B, k], vals float32 [B, k]): the k largest logits of each row, value descending, ties to the lower
    id; rows with fewer than k finite logits pad with -1 / -inf (spec/dflash.py:232-236)."""
    _require_cuda(logits, "logits")
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [B, V] with unit stride along V")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    B, V = logits.shape
    dev = logits.device
    ids = torch.empty(B, k, dtype=torch.int32, device=dev)
    vals = torch.empty(B, k, dtype=torch.float32, device=dev)
    L = _lib.load()
    ws = workspace(dev, L.vs_sample_workspace_bytes(B, V))
    check(L.vs_topk_batch(logits.data_ptr(), _DTYPES[logits.dtype], B, V, logits.stride(0), int(k), ids.data_ptr(),
                          vals.data_ptr(), ws.data_ptr(), ws.numel(), _stream_handle(dev)), "vs_topk_batch")
    return ids, vals


def _codebooks(A: torch.Tensor, B: torch.Tensor):
    for t, nm in ((A, "A"), (B, "B")):
        _require_cuda(t, nm)
        if t.dtype != torch.bfloat16 or t.dim() != 2 or not t.is_contiguous():
            raise ValueError(f"codebook {nm} must be a contiguous bf16 [vocab, rank] tensor")
    if A.shape != B.shape:
        raise ValueError("codebooks A and B differ in shape")
    return A.shape


def draft_walk(uval: torch.Tensor, cid: torch.Tensor, hp: torch.Tensor, A: torch.Tensor, B: torch.Tensor,
               anchor: torch.Tensor) -> torch.Tensor:
    """The drafter's greedy walk (spec/dflash.py:50-60) for n blocks: uval float32 [n, S, K] / cid int32 [n, S, K]
    (value descending), hp float32 [n, S, R], bf16 codebooks [vocab, R], anchor int32 [n] -> drafts int32 [n, S]."""
    vocab, R = _codebooks(A, B)
    if uval.dim() == 2:
        uval, cid, hp, anchor = uval[None], cid[None], hp[None], anchor.reshape(1)
    n, S, K = uval.shape
    for t, nm in ((uval, "uval"), (cid, "cid"), (hp, "hp"), (anchor, "anchor")):
        _require_cuda(t, nm)
    uval = uval.to(torch.float32).contiguous()
    cid = cid.to(torch.int32).contiguous()
    hp = hp.to(torch.float32).contiguous()
    anchor = anchor.reshape(n).to(torch.int32).contiguous()
    if tuple(cid.shape) != (n, S, K) or tuple(hp.shape) != (n, S, R):
        raise ValueError("uval, cid and hp disagree on shape")
    dev = uval.device
    out = torch.empty(n, S, dtype=torch.int32, device=dev)
    check(_lib.load().vs_draft_walk(uval.data_ptr(), cid.data_ptr(), K, hp.data_ptr(), A.data_ptr(), B.data_ptr(),
                                    vocab, R, anchor.data_ptr(), n, S, K, out.data_ptr(), _stream_handle(dev)),
          "vs_draft_walk")
    return out


def draft_propose(logits: torch.Tensor, hp: torch.Tensor, A: torch.Tensor, B: torch.Tensor, anchor: torch.Tensor,
                  vocab_valid: Optional[int] = None) -> torch.Tensor:
    """DFlash2Drafter.propose after the head (spec/dflash.py:228-240) for n blocks: logits [n, S, V] (or [S, V]) of
    the block rows 1..S, hp float32 [n, S, R], bf16 codebooks, anchor int32 [n] -> drafts int32 [n, S]. Only the
    first vocab_valid logits of a row are candidates."""
    vocab, R = _codebooks(A, B)
    _require_cuda(logits, "logits")
    if logits.dim() == 2:
        logits, hp, anchor = logits[None], hp[None], anchor.reshape(1)
    if logits.dim() != 3 or logits.stride(2) != 1 or logits.stride(0) != logits.shape[1] * logits.stride(1):
        raise ValueError("logits must be [n, S, V] with rows evenly strided")
    if logits.dtype not in _DTYPES:
        raise ValueError(f"unsupported logits dtype {logits.dtype}")
    n, S, V = logits.shape
    vv = V if vocab_valid is None else int(vocab_valid)
    _require_cuda(hp, "hp")
    _require_cuda(anchor, "anchor")
    hp = hp.to(torch.float32).contiguous()
    anchor = anchor.reshape(n).to(torch.int32).contiguous()
    if tuple(hp.shape) != (n, S, R):
        raise ValueError("hp must be [n, S, rank]")
    dev = logits.device
    out = torch.empty(n, S, dtype=torch.int32, device=dev)
    L = _lib.load()
    ws = workspace(dev, L.vs_draft_workspace_bytes(n, S, vv), "draft")
    check(L.vs_draft_propose(logits.data_ptr(), _DTYPES[logits.dtype], n, S, vv, logits.stride(1), hp.data_ptr(),
                             A.data_ptr(), B.data_ptr(), vocab, R, anchor.data_ptr(), out.data_ptr(), ws.data_ptr(),
                             ws.numel(), _stream_handle(dev)), "vs_draft_propose")
    return out


class PreparedPropose:
    """vs_draft_propose with every argument bound once (see PreparedSample): __call__(i) runs the top-16 and the
    walk on logits slot i ([n, S, V] each) into self.out."""

    def __init__(self, logits_slots: Sequence[torch.Tensor], hp: torch.Tensor, A: torch.Tensor, B: torch.Tensor,
                 anchor: torch.Tensor, vocab_valid: Optional[int] = None):
        vocab, R = _codebooks(A, B)
        x0 = logits_slots[0]
        _require_cuda(x0, "logits")
        if x0.dim() != 3 or x0.stride(2) != 1 or x0.stride(0) != x0.shape[1] * x0.stride(1):
            raise ValueError("logits must be [n, S, V] with rows evenly strided")
        n, S, V = x0.shape
        vv = V if vocab_valid is None else int(vocab_valid)
        hp = hp.to(torch.float32).contiguous()
        anchor = anchor.reshape(n).to(torch.int32).contiguous()
        if tuple(hp.shape) != (n, S, R):
            raise ValueError("hp must be [n, S, rank]")
        self.dev = x0.device
        self.out = torch.empty(n, S, dtype=torch.int32, device=self.dev)
        L = _lib.load()
        self._fn = L.vs_draft_propose
        ws = workspace(self.dev, L.vs_draft_workspace_bytes(n, S, vv), "draft")
        self._slots = [x.data_ptr() for x in logits_slots]
        self._keep = (list(logits_slots), hp, A, B, anchor, ws)
        self._rest = (_DTYPES[x0.dtype], n, S, vv, x0.stride(1), hp.data_ptr(), A.data_ptr(), B.data_ptr(), vocab,
                      R, anchor.data_ptr(), self.out.data_ptr(), ws.data_ptr(), ws.numel(), _stream_handle(self.dev))

    def __call__(self, slot: int = 0) -> torch.Tensor:
        rc = self._fn(self._slots[slot], *self._rest)
        if rc:
            check(rc, "vs_draft_propose")
        return self.out


def lmhead_verify_greedy(h: torch.Tensor, W: torch.Tensor, drafts: Optional[torch.Tensor],
                         vocab_valid: Optional[int] = None, return_logits: bool = False, out: Optional[VerifyOut] = None):
    """lm_head (bf16) + greedy verify in one launch (volundr.py:958-968 -> spec/specdec.py:326-327): h bf16 [B, T, K]
    (or [T, K]) final hidden states, W bf16 [N, K] -> VerifyOut (argmax [B, T], accept [B], logprobs [B, T]); with
    return_logits also the bf16 logits [B, T, N]."""
    _require_cuda(h, "h")
    _require_cuda(W, "W")
    if h.dtype != torch.bfloat16 or W.dtype != torch.bfloat16:
        raise ValueError("h and W must be bf16")
    if h.dim() == 2:
        h = h.unsqueeze(0)
    if h.dim() != 3 or W.dim() != 2 or h.shape[2] != W.shape[1]:
        raise ValueError("h must be [B, T, K] and W [N, K]")
    B, T_, K = h.shape
    N = W.shape[0]
    h2 = h.reshape(B * T_, K)
    if h2.stride(1) != 1 or W.stride(1) != 1:
        raise ValueError("h and W need unit stride along K")
    vv = N if vocab_valid is None else int(vocab_valid)
    dev = h.device
    if T_ > 1:
        if drafts is None:
            raise ValueError("drafts [B, T-1] are required when T > 1")
        _require_cuda(drafts, "drafts")
        drafts = drafts.reshape(B, T_ - 1).to(torch.int32).contiguous()
    if out is None:
        out = VerifyOut(torch.empty(B, T_, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev),
                        torch.empty(B, T_, dtype=torch.float32, device=dev))
    logits = torch.empty(B, T_, N, dtype=torch.bfloat16, device=dev) if return_logits else None
    L = _lib.load()
    ws = workspace(dev, L.vs_lmhead_workspace_bytes(B, T_), "lmhead")
    check(L.vs_lmhead_verify_greedy(h2.data_ptr(), h2.stride(0), W.data_ptr(), W.stride(0), N, K, vv, B, T_,
                                    drafts.data_ptr() if T_ > 1 else 0, out.argmax.data_ptr(), out.accept.data_ptr(),
                                    out.logprobs.data_ptr(), logits.data_ptr() if logits is not None else 0, N,
                                    ws.data_ptr(), ws.numel(), _stream_handle(dev)), "vs_lmhead_verify_greedy")
    return (out, logits) if return_logits else out


LMHEAD_SAMPLE_KMAX = 64  # largest top_k the fused head-and-sample path serves
LMHEAD_SAMPLE_RMAX = 16  # rows per call


def lmhead_sample_ok(sp, V: int, history=None, produced: int = 0, extra=()) -> bool:
    """True when vs_lmhead_sample serves this row without its logits: no logit edits (bias, suppressed ids, an
    active stop range, penalties over a non-empty history) and either greedy or 1 <= top_k <= 64."""
    if extra or sp.logit_bias or any(_wrap_id(t, V) is not None for t in sp.suppress_tokens):
        return False
    if produced < sp.min_new_tokens and sp.min_new_tokens > 0 and sp.stop_token_ids and \
            any(_wrap_id(t, V) is not None for t in sp.stop_token_ids):
        return False
    if history is not None and len(history) and (sp.repetition_penalty != 1.0 or sp.frequency_penalty != 0.0
                                                  or sp.presence_penalty != 0.0):
        return False
    return sp.greedy or (sp.top_k is not None and 1 <= sp.top_k <= LMHEAD_SAMPLE_KMAX)


def lmhead_sample(h: torch.Tensor, W: torch.Tensor, samplings: Sequence, u, histories=None, produced=None,
                  argmax_vv=None, out: Optional[SampleOut] = None) -> SampleOut:
    """lm_head (bf16, volundr.py:958-968) + Sampler.sample (sampler.py:100-156) for R <= 16 decode rows in two launches
    with no logits in HBM: h bf16 [R, K] final hidden states, W bf16 [N, K]. Rows that need their logits (see
    lmhead_sample_ok) make the whole call take the unfused path (the bf16 matmul, then sample_batch)."""
    _require_cuda(h, "h")
    _require_cuda(W, "W")
    if h.dtype != torch.bfloat16 or W.dtype != torch.bfloat16:
        raise ValueError("h and W must be bf16")
    if h.dim() != 2 or W.dim() != 2 or h.shape[1] != W.shape[1]:
        raise ValueError("h must be [R, K] and W [N, K]")
    R, K = h.shape
    N = W.shape[0]
    if h.stride(1) != 1 or W.stride(1) != 1:
        raise ValueError("h and W need unit stride along K")
    if len(samplings) != R:
        raise ValueError("one Sampling per row")
    dev = h.device
    prods = [0] * R if produced is None else list(produced)
    ok = R <= LMHEAD_SAMPLE_RMAX and all(
        lmhead_sample_ok(sp, N, None if histories is None else histories[r], prods[r])
        for r, sp in enumerate(samplings))
    if not ok:
        logits = h @ W.t()
        rows = pack_rows(samplings, u, N, histories, produced, argmax_vv=argmax_vv).to(dev)
        return sample_rows(logits, rows, out)
    rows = pack_rows(samplings, u, N, histories, produced, argmax_vv=argmax_vv).to(dev)
    out = out if out is not None else alloc_out(R, dev)
    L = _lib.load()
    ws = workspace(dev, L.vs_lmhead_sample_workspace_bytes(R), "lmsample")
    check(L.vs_lmhead_sample(h.data_ptr(), h.stride(0), W.data_ptr(), W.stride(0), N, K, R, rows.params.data_ptr(),
                             out.ids.data_ptr(), out.logprobs.data_ptr(), out.flags.data_ptr(), out.keep.data_ptr(),
                             ws.data_ptr(), ws.numel(), _stream_handle(dev)), "vs_lmhead_sample")
    return out
