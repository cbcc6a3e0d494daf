"""NumPy restatement of the bf16 lm_head followed by greedy verify. TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).

Reference arithmetic:
  * logits = lm_head(h): h bf16 [R, K] times the bf16 weight [N, K] transposed, a bf16 result
    (volundr-mlx/volundr.py:958-968; spec/verify.py:223), i.e. one rounding to bf16 (nearest even) of the sum of
    products. The reference's float32 summation order is its own; here the sum is exact (float64 of bf16 products is
    exact per product, and a K <= 8192 sum of them carries a relative error far below a bf16 ulp), so the logits of
    this oracle are the correctly rounded ones and a float32 accumulation can differ from them by one bf16 ulp only
    where the exact value lies within the float32 error bound of a bf16 rounding midpoint (`ambiguous`).
  * then greedy verify on those logits (oracle/verify_ref.py: specdec.py:326-327).

Pinning: tests/test_oracle_lmhead.py checks bf16_rne against torch's float32 -> bfloat16 conversion (round to
nearest even) on random, halfway and special values, logits_exact against a pure-Python fsum on small shapes, and
the ambiguity bound against perturbed values.
"""
from __future__ import annotations

import numpy as np

from . import verify_ref


def bf16_rne(x) -> np.ndarray:
    """float32 (or float64, first rounded to float32) -> bf16 bit patterns (uint16), round to nearest even; NaN stays
    NaN (quiet)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    un = np.where(nan, 0, u)
    r = ((un + 0x7FFF + ((un >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def logits_exact(h_bits, w_bits) -> np.ndarray:
    """float64 sums of the bf16 products, [R, N] (before the bf16 rounding)."""
    h = bf16_to_f32(h_bits).astype(np.float64)
    w = bf16_to_f32(w_bits).astype(np.float64)
    return h @ w.T


def fp32_error_bound(h_bits, w_bits) -> np.ndarray:
    """|fp32 accumulation - exact| <= K * 2^-24 * sum |h||w| (any summation order; a generous first-order bound)."""
    h = np.abs(bf16_to_f32(h_bits).astype(np.float64))
    w = np.abs(bf16_to_f32(w_bits).astype(np.float64))
    K = h.shape[1]
    return K * 2.0 ** -24 * (h @ w.T)


def logits_bf16(h_bits, w_bits):
    """(bf16 bit patterns [R, N] of the correctly rounded logits, ambiguous bool [R, N]): `ambiguous` marks logits
    whose exact value lies within the float32 accumulation bound of a bf16 rounding boundary, where a float32 sum in
    another order may round to the neighbouring bf16 value."""
    ex = logits_exact(h_bits, w_bits)
    eb = fp32_error_bound(h_bits, w_bits)
    # float64 -> bf16 directly (no float32 step): round the float64 value to 8 significant bits, nearest even
    lo_b = bf16_rne((ex - eb).astype(np.float32))
    hi_b = bf16_rne((ex + eb).astype(np.float32))
    m, e = np.frexp(ex)
    q = np.ldexp(np.round(np.ldexp(m, 8)), e - 8)  # np.round: half to even
    b = bf16_rne(q.astype(np.float32))
    return b, (lo_b != hi_b)


def verify(h_bits, w_bits, drafts, vocab_valid: int, B: int, T: int):
    """-> (logit bits [R, N], ambiguous [R, N], argmax [B, T], accept [B], logprob [B, T]) on the correctly rounded
    logits."""
    b, amb = logits_bf16(h_bits, w_bits)
    tok, acc, lp = verify_ref.verify(b.reshape(B, T, -1), drafts, vocab_valid)
    return b, amb, tok, acc, lp
