"""GPU parity of the DFlash2 drafter's candidate selection (volundr-mlx/spec/dflash.py:228-240 top-16, :50-60 walk)
against oracle/draft_ref.py: vs_topk_batch bit-exact (ids and float32 values, ties to the lower id), vs_draft_walk
and vs_draft_propose exact except at slots whose best two scores lie within fp32 rounding (the walk's sum order
differs from the oracle's), where the comparison stops for that block."""
import numpy as np
import pytest
import torch

from oracle import draft_ref as D
from volundr_amd import draft_propose, draft_walk, topk_batch

pytestmark = pytest.mark.gpu


def _bf16_bits(x):
    """float32 -> bf16 bit patterns, round to nearest even (test data only)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16_tensor(bits, dev):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)


def _check_walk(got, uval, cid, hp, A, B, anchors):
    """Compare block by block; a near tie in the oracle ends the comparison of that block at that slot."""
    checked = 0
    for b in range(len(anchors)):
        want, tie = D.walk(uval[b], cid[b], hp[b], A, B, int(anchors[b]))
        for e in range(len(want)):
            if tie[e]:
                break
            assert got[b][e] == want[e], (b, e, got[b].tolist(), want.tolist())
            checked += 1
    return checked


# 14 rows: 18 workgroups per row (lists merged by heads); 16, 20 and 64 rows: 16, 12 and 4 (merged by rank)
@pytest.mark.parametrize("V,k,dt,B", [(163840, 16, torch.float32, 14), (151936, 16, torch.bfloat16, 14),
                                      (5003, 1, torch.float32, 14), (40000, 50, torch.float16, 14),
                                      (163840, 256, torch.bfloat16, 14), (163840, 50, torch.float32, 16),
                                      (151936, 16, torch.bfloat16, 20), (5003, 1, torch.float32, 16),
                                      (40000, 256, torch.float16, 20), (163840, 20, torch.bfloat16, 64),
                                      (70000, 3, torch.float32, 64)])
def test_topk_batch_exact(dev, V, k, dt, B):
    g = torch.Generator().manual_seed(V + k + B)
    x = (torch.randn(B, V, generator=g) * 3).to(dt)
    ids, vals = topk_batch(x.to(dev), k)
    xf = x.float().numpy()
    for r in range(x.shape[0]):
        wi, wv = D.topk_sorted(xf[r], k)
        assert ids[r].cpu().numpy().tolist() == wi.tolist(), r
        np.testing.assert_array_equal(vals[r].cpu().numpy(), wv)


@pytest.mark.parametrize("B", [6, 16, 40])
def test_topk_batch_ties_and_short_rows(dev, B):
    rng = np.random.default_rng(5 + B)
    V = 9000
    x = rng.integers(-3, 4, size=(B, V)).astype(np.float32)  # heavy ties: the lower id wins
    x[1, :] = -np.inf
    x[1, [7, 4000, 8999]] = [1.0, 1.0, -2.0]  # three finite logits: 13 of 16 padded
    x[2, :] = -np.inf  # no finite logit at all
    x[3, 100:200] = np.nan  # NaN never enters the list
    x[4, :] = -np.inf
    x[4, 8990:] = rng.standard_normal(10)  # every finite logit in the last workgroup's chunk: one list is full
    x[5, ::700] = np.inf  # +inf is not finite: never listed
    ids, vals = topk_batch(torch.from_numpy(x).to(dev), 16)
    for r in range(B):
        wi, wv = D.topk_sorted(x[r], 16)
        assert ids[r].cpu().numpy().tolist() == wi.tolist(), r
        np.testing.assert_array_equal(vals[r].cpu().numpy(), wv)


def _walk_case(seed, n, vocab=2000, R=256, S=7, K=16, distinct=False):
    rng = np.random.default_rng(seed)
    A = _bf16_bits(rng.standard_normal((vocab, R)) * 0.2)
    B = _bf16_bits(rng.standard_normal((vocab, R)) * 0.2)
    if distinct:  # no id appears twice anywhere in the case
        cid = rng.permutation(vocab)[:n * S * K].reshape(n, S, K).astype(np.int32)
    else:
        cid = np.stack([np.stack([rng.choice(vocab, K, replace=False) for _ in range(S)])
                        for _ in range(n)]).astype(np.int32)
    uval = -np.sort(-rng.standard_normal((n, S, K)).astype(np.float32), axis=2)
    hp = rng.standard_normal((n, S, R)).astype(np.float32)
    anchors = rng.integers(0, vocab, n).astype(np.int32)
    return A, B, cid, uval, hp, anchors


@pytest.mark.parametrize("seed,n,R", [(0, 1, 256), (1, 64, 256), (2, 300, 128), (3, 8, 16)])
def test_walk_matches_oracle(dev, seed, n, R):
    A, B, cid, uval, hp, anchors = _walk_case(seed, n, R=R)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    got = draft_walk(t(uval), t(cid), t(hp), _bf16_tensor(A, dev), _bf16_tensor(B, dev), t(anchors)).cpu().numpy()
    checked = _check_walk(got, uval, cid, hp, A, B, anchors)
    assert checked >= 0.9 * n * 7  # near ties are rare with these scales


def test_walk_closed_forms(dev):
    A, B, cid, uval, hp, anchors = _walk_case(7, 16, distinct=True)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    Z = np.zeros_like(B)
    # no successor term: every slot takes its first (largest) candidate
    got = draft_walk(t(uval), t(cid), t(hp), _bf16_tensor(A, dev), _bf16_tensor(Z, dev), t(anchors)).cpu().numpy()
    assert got.tolist() == cid[:, :, 0].tolist()
    # equal logits and no successor term: the first maximum (position 0) still wins
    got = draft_walk(t(np.zeros_like(uval)), t(cid), t(hp), _bf16_tensor(A, dev), _bf16_tensor(Z, dev),
                     t(anchors)).cpu().numpy()
    assert got.tolist() == cid[:, :, 0].tolist()
    # one-hot codebooks: s[c] = uval[c] + B[c][0] * A[pred][0] * hp[0]; a large B entry on one candidate decides
    # (ids are distinct across the case, so exactly one candidate per slot carries it)
    vocab, R = A.shape
    A1 = np.zeros_like(A)
    A1[:, 0] = _bf16_bits(np.ones(vocab))
    B1 = np.zeros_like(B)
    hp1 = np.zeros_like(hp)
    hp1[:, :, 0] = 1.0
    win = 11
    for b in range(cid.shape[0]):
        for e in range(cid.shape[1]):
            B1[cid[b, e, win], 0] = _bf16_bits(np.float32(100.0))
    got = draft_walk(t(uval), t(cid), t(hp1), _bf16_tensor(A1, dev), _bf16_tensor(B1, dev), t(anchors)).cpu().numpy()
    assert got.tolist() == cid[:, :, win].tolist()


def test_walk_invalid_ids(dev):
    A, B, cid, uval, hp, anchors = _walk_case(9, 4)
    Z = np.zeros_like(B)
    vocab = A.shape[0]
    cid = cid.copy()
    cid[0, 2, 0] = -1          # an invalid first candidate: the next valid one (no successor term) wins
    cid[1, 3, :] = vocab + 5   # a slot with no valid candidate: it and every later slot are -1
    anchors = anchors.copy()
    anchors[2] = vocab         # an invalid anchor: the whole block is -1
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    got = draft_walk(t(uval), t(cid), t(hp), _bf16_tensor(A, dev), _bf16_tensor(Z, dev), t(anchors)).cpu().numpy()
    assert got[0].tolist() == [cid[0, e, 1 if e == 2 else 0] for e in range(7)]
    assert got[1].tolist() == [cid[1, e, 0] for e in range(3)] + [-1] * 4
    assert got[2].tolist() == [-1] * 7
    assert got[3].tolist() == cid[3, :, 0].tolist()


@pytest.mark.parametrize("n,V,vv,dt", [(1, 152064, 151936, torch.bfloat16), (6, 40000, 40000, torch.float32),
                                       (3, 163840, 163000, torch.float16)])
def test_propose_matches_oracle(dev, n, V, vv, dt):
    S, R, K = 7, 256, 16
    rng = np.random.default_rng(n + V)
    A = _bf16_bits(rng.standard_normal((V, R)) * 0.1)
    B = _bf16_bits(rng.standard_normal((V, R)) * 0.1)
    hp = rng.standard_normal((n, S, R)).astype(np.float32)
    anchors = rng.integers(0, vv, n).astype(np.int32)
    x = (torch.randn(n, S, V, generator=torch.Generator().manual_seed(n)) * 4).to(dt)
    got = draft_propose(x.to(dev), torch.from_numpy(hp).to(dev), _bf16_tensor(A, dev), _bf16_tensor(B, dev),
                        torch.from_numpy(anchors).to(dev), vocab_valid=vv).cpu().numpy()
    xf = x.float().numpy()
    cid = np.zeros((n, S, K), np.int32)
    uval = np.zeros((n, S, K), np.float32)
    for b in range(n):
        for e in range(S):
            cid[b, e], uval[b, e] = D.topk_sorted(xf[b, e, :vv], K)
    checked = _check_walk(got, uval, cid, hp, A, B, anchors)
    assert checked >= 0.8 * n * S


def test_propose_calls_of_shrinking_size(dev):
    """Back-to-back calls on one workspace, each with fewer rows than the last: every call must find the sampler's
    counters zeroed whatever the previous call's lists left behind."""
    S, R, V = 7, 256, 50000
    rng = np.random.default_rng(42)
    A = _bf16_bits(rng.standard_normal((V, R)) * 0.1)
    B = _bf16_bits(rng.standard_normal((V, R)) * 0.1)
    Ad, Bd = _bf16_tensor(A, dev), _bf16_tensor(B, dev)
    for n in (9, 4, 1, 4):
        hp = rng.standard_normal((n, S, R)).astype(np.float32)
        anchors = rng.integers(0, V, n).astype(np.int32)
        x = torch.from_numpy((rng.standard_normal((n, S, V)) * 4).astype(np.float32))
        got = draft_propose(x.to(dev), torch.from_numpy(hp).to(dev), Ad, Bd, torch.from_numpy(anchors).to(dev))
        xf = x.numpy()
        cid = np.zeros((n, S, 16), np.int32)
        uval = np.zeros((n, S, 16), np.float32)
        for b in range(n):
            for e in range(S):
                cid[b, e], uval[b, e] = D.topk_sorted(xf[b, e], 16)
        assert _check_walk(got.cpu().numpy(), uval, cid, hp, A, B, anchors) >= 0.8 * n * S, n
