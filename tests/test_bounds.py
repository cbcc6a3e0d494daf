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


BOUND_BITS = 16  # bits of the ord32 value the kernel's bisections resolve (vs_sample.hip BOUND_BITS)


def heads_bound(head_keys, keff, bits=BOUND_BITS):
    """The kernel's bisection over the top `bits` bits: th = the largest such value reached by >= keff heads;
    M = th << 32 (0 if fewer than keff heads are non-zero)."""
    hh = (head_keys >> np.uint64(32)).astype(np.uint64)
    if int((hh != 0).sum()) < keff:
        return np.uint64(0)
    th = 0
    for b in range(31, 31 - bits, -1):
        c = th | (1 << b)
        if int((hh >= c).sum()) >= keff:
            th = c
    return np.uint64(th) << np.uint64(32)


@pytest.mark.parametrize("bits", [16, 32])
@pytest.mark.parametrize("seed", range(40))
def test_topk_merge_bound_never_cuts_the_top(seed, bits):
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
    M = heads_bound(np.array(heads, dtype=np.uint64), keff, bits)
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
        fx = np.rint(pr * scale).astype(np.uint64)
        # every prefix (the top-p cut and the draw use prefixes in descending order)
        order = np.argsort(-pr, kind="stable")
        cf = np.cumsum(pr[order])
        cfx = np.cumsum(fx[order].astype(object))  # exact integer sums
        zfix = np.array([float(v) for v in cfx]) / scale
        rel = np.abs(zfix - cf) / cf
        assert rel.max() <= 5e-7, (bits, trial, rel.max())


def test_truncated_bound_is_close():
    """The 16-bit bound is below the exact one by less than a factor 1 + 2^-7 in value (positive values)."""
    rng = np.random.default_rng(5)
    for _ in range(200):
        vals = (np.abs(rng.standard_normal(64)) * rng.choice([0.01, 1, 100]) + 1e-3).astype(np.float32)
        keys = keys_of(vals, np.arange(64))
        keff = int(rng.integers(1, 65))
        exact = heads_bound(keys, keff, 32) >> np.uint64(32)
        trunc = heads_bound(keys, keff, 16) >> np.uint64(32)
        assert trunc <= exact
        ve = np.array([exact & 0x7FFFFFFF], np.uint32).view(np.float32)[0]
        vt = np.array([trunc & 0x7FFFFFFF], np.uint32).view(np.float32)[0]
        assert vt <= ve <= vt * (1 + 2.0 ** -7) * (1 + 1e-7)


def fixed_mass(e, S):
    """The kernel's float32 form of round-to-nearest-even(e * 2^S) for a float32 0 <= e <= 1 (vs_sample.hip
    fixed_mass): the part at and above 2^32, truncated, and the exact rest below it, rounded."""
    f = np.float32
    e = f(e)
    h = np.trunc(e * f(2.0 ** (S - 32)))
    r = f(np.float64(e * f(2.0 ** S)) - np.float64(h) * 2.0 ** 32)  # the fma: one rounding of the exact value
    assert np.float64(r) == np.float64(e) * 2.0 ** S - np.float64(h) * 2.0 ** 32  # the rest is exact
    return (int(h) << 32) | int(np.rint(r))


@pytest.mark.parametrize("S", [29, 38, 45, 46, 56, 62])
def test_fixed_mass_matches_float64_rounding(S):
    rng = np.random.default_rng(S)
    es = np.concatenate([np.exp(-rng.random(4000) * 60).astype(np.float32),
                         np.array([0.0, 1.0, 0.5, 2.0 ** -S, 2.0 ** -(S + 1), 3 * 2.0 ** -(S + 1),
                                   5 * 2.0 ** -(S + 1), 3 * 2.0 ** -(S + 2), 1e-30, 1e-40, 2.0 ** -24],
                                  np.float32)])
    for e in es:
        want = int(np.rint(np.float64(e) * 2.0 ** S))  # ties to even
        assert fixed_mass(float(e), S) == want, (e, S)
