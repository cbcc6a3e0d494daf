"""Independent brute-force sampler for tiny vocabularies (pure Python: sorted(), math.exp, math.fsum).

Used only to pin the NumPy oracle: it shares the reference's definition (volundr-mlx/sampler.py:100-156) but none
of the oracle's code paths (no argpartition, lexsort, cumsum or searchsorted).
"""
import math
import struct


def f32(v: float) -> float:
    return struct.unpack("f", struct.pack("f", v))[0]


def brute_sample(x, sp, u, counts=None, produced=0):
    x = [f32(v) for v in x]
    V = len(x)
    for t, b in sp.logit_bias:
        if t < V:
            x[t] = f32(x[t] + f32(b))
    for t in sp.suppress_tokens:
        if t < V:
            x[t] = -math.inf
    r, fp, pp = f32(sp.repetition_penalty), f32(sp.frequency_penalty), f32(sp.presence_penalty)
    for t, c in (counts or {}).items():
        if t >= V:
            continue
        v = x[t]
        if sp.repetition_penalty != 1.0:
            v = f32(v / r) if v > 0 else f32(v * r)
        x[t] = f32(v - f32(f32(fp * c) + pp))
    if produced < sp.min_new_tokens:
        for t in sp.stop_token_ids:
            if t < V:
                x[t] = -math.inf
    if sp.greedy:
        best = 0
        for i in range(V):
            if x[i] > x[best] or (math.isnan(x[i]) and not math.isnan(x[best])):
                best = i
        return best
    fin = [i for i in range(V) if math.isfinite(x[i])]
    order = sorted(fin, key=lambda i: (-x[i], i))
    k = sp.top_k if sp.top_k else len(fin)
    k = max(1, min(k, len(fin)))
    t = f32(sp.temperature)
    if k < len(fin):
        order = order[:k]
    elif len(fin) > 4096:
        m = x[order[0]]
        thr = f32(f32(m / t) - 40.0)
        order = [i for i in order if f32(x[i] / t) >= thr]
    xs0 = f32(x[order[0]] / t)
    pr = [math.exp(f32(f32(x[i] / t) - xs0)) for i in order]
    S = math.fsum(pr)
    p = [q / S for q in pr]
    keep = len(p)
    if sp.top_p < 1.0:
        acc = 0.0
        for i, q in enumerate(p):
            acc += q
            if acc >= sp.top_p:
                keep = i + 1
                break
    if sp.min_p > 0.0:
        cnt = next((i for i, q in enumerate(p) if q < p[0] * sp.min_p), len(p))
        keep = min(keep, max(cnt, 1))
    z = math.fsum(p[:keep])
    target = u * z
    acc = 0.0
    for i in range(keep):
        acc += p[i]
        if acc >= target:
            return order[i]
    return order[keep - 1]
