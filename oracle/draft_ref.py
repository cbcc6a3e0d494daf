"""Test-only oracle (CPU, NumPy) of the DFlash2 drafter's candidate selection: the vocab top-16 of each block row and
the greedy walk over the 7 slots (volundr-mlx/spec/dflash.py:228-240 and :50-60). Used only by tests/ as the checker.

* topk_sorted(x, k): the k largest logits of a row, value descending; ties at the k-th value and inside the list go
  to the lower id (dflash.py:232-235 uses argpartition + argsort, whose order among equal values is
  implementation-defined: the lower id is this build's rule).
* walk(uval, cid, hp, A, B, anchor): dflash.py:50-60: for e in 0..6: a = A[pred] (bf16 -> f32) * hp[e];
  s = uval[e] + B[cid[e]] (bf16 -> f32) @ a; pred = cid[e][first argmax of s]. The float32 dot products are summed
  in a fixed order here; the reference's matmul order is its own, so the drafts agree except where two scores lie
  within rounding of each other (`near_tie`).
"""
from __future__ import annotations

import numpy as np


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16) to float32."""
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def topk_sorted(x: np.ndarray, k: int):
    """(ids int32 [k], vals float32 [k]) of the k largest finite logits, value descending, ties to the lower id;
    rows with fewer finite logits are padded with id -1 and value -inf (dflash.py:232-235)."""
    x = np.asarray(x, dtype=np.float32)
    fin = np.nonzero(np.isfinite(x))[0]
    order = fin[np.lexsort((fin, -x[fin].astype(np.float64)))][:k]
    ids = np.full(k, -1, np.int32)
    vals = np.full(k, -np.inf, np.float32)
    ids[:order.size] = order
    vals[:order.size] = x[order]
    return ids, vals


def scores(uval_e, cid_e, hp_e, A, B, pred):
    """s = uval[e] + B[cid[e]] @ (A[pred] * hp[e]) in float32, products summed left to right (dflash.py:56-57)."""
    a = (bf16_to_f32(A[pred]) * np.asarray(hp_e, np.float32)).astype(np.float32)
    s = np.zeros(len(cid_e), np.float32)
    for c, tok in enumerate(cid_e):
        b = bf16_to_f32(B[tok])
        acc = np.float32(0.0)
        for j in range(a.size):
            acc = np.float32(acc + np.float32(b[j] * a[j]))
        s[c] = np.float32(np.float32(uval_e[c]) + acc)
    return s


def walk(uval, cid, hp, A, B, anchor: int, rtol: float = 1e-5):
    """(drafts int32 [slots], near_tie bool [slots]) of dflash.py:50-60. near_tie[e]: the best and second-best scores
    of slot e lie within rtol * (1 + max |s|), where a different summation order may pick the other one."""
    pred = int(anchor)
    out, tie = [], []
    for e in range(len(cid)):
        s = scores(uval[e], cid[e], hp[e], A, B, pred)
        j = int(np.argmax(s))
        srt = np.sort(s)[::-1]
        tie.append(len(s) > 1 and float(srt[0] - srt[1]) <= rtol * (1.0 + float(np.abs(s).max())))
        pred = int(cid[e][j])
        out.append(pred)
    return np.asarray(out, np.int32), np.asarray(tie, bool)
