"""Seeded synthetic inputs for the measured configurations (host NumPy; shapes and distributions as stated in the
benchmark configuration list). Used by bench.py and the tests; never by the sampling path itself.

  C1  B=1, V=163840 fp32 ~ N(0, 3^2), 5 spikes set to +12; T=1, top-k 20, top-p 1, no penalties
  C2  verify [1, 17, V] bf16 ~ N(0, 2^2), per-position argmax planted at +10, ~1% rows with an exact tie at a
      higher index; drafts [1, 16] equal to the argmax for a seeded prefix length in 0..16
  C3  B=16 fp32 3*Student-t(3); T ~ U[0.6,1.2], top-k in {0,20,50}, top-p in {0.8,0.95,1}, repetition U[1.05,1.2],
      presence U[0,0.5]; histories [16, 4096] Zipf(1.1) folded into [0, V) as (z-1) % V
  C4  verify [4, 17, V] bf16 as C2; drafts [4, 16]
  C5  B=16 fp32 ~ N(0, 0.1^2); T=1, top-k off, top-p 0.95, repetition 1.1; histories [16, 32768] uniform over V
"""
from __future__ import annotations

import numpy as np

from .session import Sampling

V_DEFAULT = 163840


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 to bfloat16 (round to nearest even) and return the uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def c1(seed=0, V=V_DEFAULT):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((1, V)) * 3.0).astype(np.float32)
    x[0, rng.choice(V, 5, replace=False)] = 12.0
    sp = [Sampling(temperature=1.0, top_k=20, top_p=1.0)]
    return dict(logits=x, params=sp, u=rng.random(1), hists=None)


def verify_case(B, T=17, seed=0, V=V_DEFAULT, tie_frac=0.01, sigma=2.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B, T, V)) * sigma).astype(np.float32)
    am = rng.integers(0, V, size=(B, T))
    for b in range(B):
        for t in range(T):
            x[b, t, am[b, t]] = 10.0
            if rng.random() < tie_frac and am[b, t] + 1 < V:  # exact tie at a higher index: the lower one wins
                x[b, t, rng.integers(am[b, t] + 1, V)] = 10.0
    bits = f32_to_bf16_bits(x)
    am = np.argmax(bf16_bits_to_f32(bits), axis=-1)  # the true first-max argmax (a 5-sigma draw can beat +10)
    L = rng.integers(0, T, size=B)                 # accept length 0..T-1
    drafts = rng.integers(0, V, size=(B, T - 1)).astype(np.int32)
    for b in range(B):
        drafts[b, : L[b]] = am[b, : L[b]]
        if L[b] < T - 1:
            drafts[b, L[b]] = (am[b, L[b]] + 1) % V
    return dict(logits_bf16=bits, drafts=drafts, accept=L.astype(np.int32), planted=am)


def c2(seed=0, V=V_DEFAULT, tie_frac=0.01):
    return verify_case(1, 17, seed, V, tie_frac)


def c4(seed=0, V=V_DEFAULT, tie_frac=0.01):
    return verify_case(4, 17, seed, V, tie_frac)


def c3(seed=0, V=V_DEFAULT, B=16, H=4096):
    rng = np.random.default_rng(seed)
    x = (rng.standard_t(3, size=(B, V)) * 3.0).astype(np.float32)
    params = []
    for _ in range(B):
        params.append(Sampling(temperature=float(rng.uniform(0.6, 1.2)), top_k=int(rng.choice([0, 20, 50])),
                               top_p=float(rng.choice([0.8, 0.95, 1.0])),
                               repetition_penalty=float(rng.uniform(1.05, 1.2)),
                               presence_penalty=float(rng.uniform(0.0, 0.5)), frequency_penalty=0.0))
    z = rng.zipf(1.1, size=(B, H))
    hists = ((z - 1) % V).astype(np.int32)
    return dict(logits=x, params=params, u=rng.random(B), hists=hists)


def c5(seed=0, V=V_DEFAULT, B=16, H=32768):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B, V)) * 0.1).astype(np.float32)
    params = [Sampling(temperature=1.0, top_k=0, top_p=0.95, repetition_penalty=1.1) for _ in range(B)]
    hists = rng.integers(0, V, size=(B, H)).astype(np.int32)
    return dict(logits=x, params=params, u=rng.random(B), hists=hists)


CONFIGS = {"c1": c1, "c2": c2, "c3": c3, "c4": c4, "c5": c5}
