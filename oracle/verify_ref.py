"""NumPy restatement of greedy speculative verify. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference arithmetic:
  * tok  = argmax(logits[..., :vv]) with the first maximum on ties        volundr-mlx/spec/specdec.py:326,
                                                                          volundr-mlx/scheduler.py:462
  * nacc = sum(cumprod(inp[:, 1:] == tok[:, :-1]))                        specdec.py:327, scheduler.py:463
  * emitted = inp[1:nacc+1] + [tok[nacc]]                                 specdec.py:335-336, scheduler.py:465-470
  * logprob (build-defined; the reference has none): x[tok] - logsumexp(x[:vv]) on float32 logits, the log-softmax
    form of volundr-mlx/spec/check_verify.py:27-30, evaluated here in float64.
`drafts` is inp[:, 1:], shape [B, T-1].

Pinning: tests/test_oracle.py checks emitted on hand cases and against the identity emitted == tok[:nacc+1] (the
accepted drafts equal the argmax prefix), argmax against a Python loop (strict `>` scan keeps the first maximum), the
accept length against the hand cases all-match -> T-1, first-mismatch -> 0, and a planted exact tie -> the lower
index, and the logprob against math.fsum of exp on small rows. NaN handling of mx.argmax is unpinned: this oracle
(like np.argmax) ranks NaN above every number.
"""
from __future__ import annotations

import numpy as np


def to_f32(logits) -> np.ndarray:
    """bf16 arrays arrive as uint16 bit patterns or torch-converted float32; both become float32 exactly."""
    a = np.asarray(logits)
    if a.dtype == np.uint16:
        return (a.astype(np.uint32) << 16).view(np.float32)
    return a.astype(np.float32)


def verify(logits, drafts, vocab_valid: int):
    """-> (argmax int32 [B,T], accept int32 [B], logprob float64 [B,T])."""
    x = to_f32(logits)[..., :vocab_valid]
    B, T = x.shape[0], x.shape[1]
    tok = np.argmax(x, axis=-1).astype(np.int32)                       # first max
    drafts = np.asarray(drafts, dtype=np.int32).reshape(B, T - 1)
    eq = (drafts == tok[:, :-1]).astype(np.int32)
    acc = np.cumprod(eq, axis=1).sum(axis=1).astype(np.int32) if T > 1 else np.zeros(B, np.int32)
    xd = x.astype(np.float64)
    m = xd.max(axis=-1, keepdims=True)
    lse = (m + np.log(np.exp(xd - m).sum(axis=-1, keepdims=True)))[..., 0]
    lp = np.take_along_axis(xd, tok[..., None].astype(np.int64), axis=-1)[..., 0] - lse
    return tok, acc, lp


def emitted(drafts_row, tok_row, nacc: int):
    """Tokens one verify step emits for a request: the accepted drafts plus the bonus token."""
    return [int(t) for t in drafts_row[:nacc]] + [int(tok_row[nacc])]
