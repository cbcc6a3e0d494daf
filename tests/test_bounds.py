"""CPU checks of the two selection bounds the sampling kernel relies on, restated in NumPy on randomised cases:

* the TOPK merge bound (csrc/vs_sample.hip, the merge of the last workgroup of a row): with r = ceil(k / G) heads per
  workgroup list, M = the lowest key of the keff-th largest head value is never above the row's keff-th largest key,
  for both list formats (a sorted list's first r keys; the first r of an unsorted list's eight wave maxima,
  descending), so every key of the row's top keff survives the filter x >= M;
* the fixed-point normaliser of the value-bin path: when every kept mass is >= exp(-span) with
  span <= ln(scale) - ln(1e6), the exact integer sum of round(mass * scale), divided by scale, is within 5e-7
  relative of the float64 sum of the masses, for the whole kept set and for every prefix of it.

Keys follow the kernel's layout: ord32(value) << 32 | (0xFFFFFFFF - index)."""
import math

import numpy as np
import pytest


def ord32(x):
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, ~u & 0xFFFFFFFF, u | 0x80000000)


def keys_of(vals, idx):
    return (ord32(vals) << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx.astype(np.uint64))


def heads_bound(head_keys, keff):
    """The kernel's bisection: th = the largest 32-bit value reached by >= keff heads; M = th << 32 (0 if fewer
    than keff heads are non-zero)."""
    hh = (head_keys >> np.uint64(32)).astype(np.uint64)
    if int((hh != 0).sum()) < keff:
        return np.uint64(0)
    th = 0
    for b in range(31, -1, -1):
        c = th | (1 << b)
        if int((hh >= c).sum()) >= keff:
            th = c
    return np.uint64(th) << np.uint64(32)


@pytest.mark.parametrize("seed", range(40))
def test_topk_merge_bound_never_cuts_the_top(seed):
    rng = np.random.default_rng(seed)
    G = int(rng.choice([3, 8, 16, 40, 64]))
    k = int(rng.integers(1, 8 * G + 1))
    chunk = int(rng.choice([64, 500, 2048]))
    V = G * chunk
    scale = float(rng.choice([0.1, 1.0, 3.0]))
    vals = (rng.standard_normal(V) * scale).astype(np.float32)
    if seed % 5 == 0:
        vals = np.round(vals)  # heavy ties
    if seed % 7 == 0:
        vals[: V // 2] = -np.inf  # half the workgroups without finite logits
    finite = np.isfinite(vals)
    keys = np.where(finite, keys_of(vals, np.arange(V)), np.uint64(0))
    n = int(finite.sum())
    keff = max(1, min(k, n))
    r = (k + G - 1) // G
    heads = []
    for g in range(G):
        kg = np.sort(keys[g * chunk:(g + 1) * chunk])[::-1]
        if seed % 2 == 0:  # sorted format: the list's first r keys
            heads.extend(kg[:r].tolist())
        else:  # unsorted format: eight wave maxima (waves own strided positions), descending, first r
            part = keys[g * chunk:(g + 1) * chunk]
            wmax = sorted((int(part[w::8].max()) if part[w::8].size else 0 for w in range(8)), reverse=True)
            heads.extend(wmax[:r])
    M = heads_bound(np.array(heads, dtype=np.uint64), keff)
    top = np.sort(keys)[::-1][:keff]
    assert int(top[-1]) >= int(M)
    assert int((keys >= M).sum()) >= keff


@pytest.mark.parametrize("bits", [10, 14, 18, 20])
def test_fixed_point_normaliser_within_5e7(bits):
    rng = np.random.default_rng(bits)
    scale = 2.0 ** (63 - bits)
    span_max = math.log(scale) - math.log(1e6)
    for trial in range(20):
        n = int(rng.integers(2, min(2 ** bits, 20000)))
        span = float(rng.uniform(0, span_max))
        d = -rng.uniform(0, span, size=n)
        d[0] = 0.0  # the row maximum: mass exactly 1
        pr = np.exp(d.astype(np.float32)).astype(np.float64)  # masses as the kernel computes them (float32 exp)
        fx = np.floor(pr * scale + 0.5).astype(np.uint64)
        # every prefix (the top-p cut and the draw use prefixes in descending order)
        order = np.argsort(-pr, kind="stable")
        cf = np.cumsum(pr[order])
        cfx = np.cumsum(fx[order].astype(object))  # exact integer sums
        zfix = np.array([float(v) for v in cfx]) / scale
        rel = np.abs(zfix - cf) / cf
        assert rel.max() <= 5e-7, (bits, trial, rel.max())
