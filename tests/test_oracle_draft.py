"""CPU pinning of oracle/draft_ref.py (the drafter's top-16 and walk, volundr-mlx/spec/dflash.py:50-60, 228-240)
against pure-Python brute force and closed forms."""
import math

import numpy as np

from oracle import draft_ref as D


def _bf16(x):
    """float32 -> bf16 bits, round to nearest even (test data only)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def test_bf16_widening_exact():
    assert D.bf16_to_f32(np.array([0x3F80, 0xC000, 0x0000, 0x7F80], np.uint16)).tolist() == [1.0, -2.0, 0.0, math.inf]


def test_topk_sorted_brute_force():
    rng = np.random.default_rng(0)
    for _ in range(30):
        n = int(rng.integers(1, 60))
        x = rng.integers(-5, 6, size=n).astype(np.float32)  # many ties
        if rng.random() < 0.3:
            x[rng.integers(0, n)] = -np.inf
        k = int(rng.integers(1, 20))
        ids, vals = D.topk_sorted(x, k)
        want = sorted((i for i in range(n) if math.isfinite(x[i])), key=lambda i: (-float(x[i]), i))[:k]
        assert ids[:len(want)].tolist() == want
        assert all(i == -1 for i in ids[len(want):]) and all(v == -np.inf for v in vals[len(want):])
        assert vals[:len(want)].tolist() == [float(x[i]) for i in want]


def test_walk_brute_force():
    rng = np.random.default_rng(1)
    vocab, rank, K, slots = 40, 8, 4, 7
    A = _bf16(rng.standard_normal((vocab, rank)))
    B = _bf16(rng.standard_normal((vocab, rank)))
    cid = rng.integers(0, vocab, size=(slots, K)).astype(np.int32)
    uval = np.sort(rng.standard_normal((slots, K)).astype(np.float32), axis=1)[:, ::-1]
    hp = rng.standard_normal((slots, rank)).astype(np.float32)
    got, _ = D.walk(uval, cid, hp, A, B, anchor=3)
    pred = 3
    for e in range(slots):
        a = [float(np.float32(D.bf16_to_f32(A[pred][j:j + 1])[0] * hp[e][j])) for j in range(rank)]
        best, bj = None, 0
        for c in range(K):
            acc = 0.0
            for j in range(rank):
                acc = float(np.float32(acc + float(np.float32(D.bf16_to_f32(B[cid[e][c]][j:j + 1])[0] * a[j]))))
            s = float(np.float32(uval[e][c] + acc))
            if best is None or s > best:
                best, bj = s, c
        pred = int(cid[e][bj])
        assert got[e] == pred


def test_walk_closed_forms():
    rng = np.random.default_rng(2)
    vocab, rank, K = 30, 16, 16
    cid = rng.integers(0, vocab, size=(7, K)).astype(np.int32)
    uval = np.sort(rng.standard_normal((7, K)).astype(np.float32), axis=1)[:, ::-1].copy()
    hp = rng.standard_normal((7, rank)).astype(np.float32)
    Z = np.zeros((vocab, rank), np.uint16)
    A = _bf16(rng.standard_normal((vocab, rank)))
    # no successor term: every slot takes its first (largest) candidate
    assert D.walk(uval, cid, hp, A, Z, 0)[0].tolist() == cid[:, 0].tolist()
    # no hidden projection: the same
    assert D.walk(uval, cid, np.zeros_like(hp), A, A, 0)[0].tolist() == cid[:, 0].tolist()
    # equal values: the first maximum (position 0) wins the tie
    flat = np.zeros_like(uval)
    assert D.walk(flat, cid, hp, A, Z, 0)[0].tolist() == cid[:, 0].tolist()
    # a successor row that dominates: one-hot codebooks make s[c] = uval + b[c] . a
    B = np.zeros((vocab, rank), np.uint16)
    A1 = np.zeros((vocab, rank), np.uint16)
    A1[:, 0] = _bf16(np.ones(vocab, np.float32))
    hp1 = np.zeros((7, rank), np.float32)
    hp1[:, 0] = 1.0
    B[cid[0][5], 0] = _bf16(np.float32(100.0))
    d, _ = D.walk(uval, cid, hp1, A1, B, 0)
    assert d[0] == cid[0][5]
