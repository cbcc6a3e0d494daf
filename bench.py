"""Benchmark of the token-selection hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3]

A step is one vs_sample_batch call over the B=16 x V=163840 mixed-parameter batch (configuration C3, the one
the headline metric is quoted on), with logits, parameters and histories already resident in HBM. Logits, parameters
and histories rotate over `--slots` device copies (> 256 MB in total by default), so every step reads them from HBM
and not from the 256 MB Infinity Cache. Printed (one JSON line on stdout):
  value       end-to-end microseconds per step (host-issued launches back to back, HIP events on the launch stream)
  roofline    algorithmic bytes per launch / per-launch time (HIP events around the K back-to-back launches on the
              launch stream; rocprofv3's average kernel duration agrees within a few percent) vs 8 TB/s
  cpu_baseline  the NumPy restatement of sampler.py (oracle/) on a bounded sample of the same rows, 1 core
  graph_us_per_step  the same step captured in a HIP graph (hipGraph via torch.cuda.CUDAGraph), replayed
The other configurations (C1, C2, C4, C5) are reported under "other_configs" with the same method, and "c3_state"
is C3 through vs_sample_batch_state (the per-request sampler state on the device; each step also accepts),
"c3_dropin" C3 through sample_rows_for and the Sampler.choose loop (host work included, wall clock),
"c3_greedy" C3's logits and histories with every row greedy (temperature 0);
"c3_raw" / "c5_raw" the same rows with the raw token histories as the penalty input (the default, --hist-form pairs,
passes each request's sorted (id, count) table, the form of Sampler.counts, built outside the timed region);
"draft_propose" is the DFlash2 drafter's top-16 + candidate walk (vs_draft_propose) at the drafter's vocabulary;
"lmhead_verify_*" is the bf16 lm_head with greedy verify fused in (vs_lmhead_verify_greedy), beside the unfused
torch matmul + vs_verify_greedy; "lmhead_sample_b16" the head with top-k sampling fused in (vs_lmhead_sample) beside
the matmul + vs_sample_batch; "read_ceiling" one streaming read of a buffer of the head weight's size
(vs_stream_read), the rate the head kernels stream against.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "volundr-mlx_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "sampling step latency µs + HBM GB/s at B=16, V=163840 on 1 MI355X"
WORKLOADS = {
    "c1": "C1: B=1 V=163840 fp32, top-k 20 (BASELINE configs[0])",
    "c2": "C2: greedy verify [1,17,163840] bf16 + drafts [1,16] (BASELINE configs[1])",
    "c3": "C3: B=16 V=163840 fp32 mixed-parameter sampling, histories 16x4096 (BASELINE configs[2])",
    "c3_raw": "C3 with each history passed as its 4096 raw token ids instead of the (id, count) table",
    "c4": "C4: greedy verify [4,17,163840] bf16 + drafts [4,16] (BASELINE configs[3])",
    "c5": "C5: B=16 V=163840 fp32 near-flat, top-p 0.95, histories 16x32768 (BASELINE configs[4])",
    "c5_raw": "C5 with each history passed as its 32768 raw token ids instead of the (id, count) table",
}
HIST_FORM = ("; penalty state passed as each request's sorted (id, count) table, the form of Sampler.counts "
             "(sampler.py:77-78, 113-122), built from the history outside the timed region")
PEAK_GBPS = 8000.0
V = 163840


def algo_bytes_sample(d, B):
    """Logits read once + the penalty state read once (raw histories: 4 bytes per token; (id, count) tables: 8 bytes
    per distinct id) + per-row params + outputs (ids, logprob, flags, keep)."""
    import numpy as np

    x = d["logits"]
    if d["hists"] is None:
        h = 0
    elif d.get("hist_pairs"):
        h = sum(8 * int(np.unique(r).size) for r in d["hists"])
    else:
        h = d["hists"].size * 4
    return x.size * 4 + h + B * 96 + B * 16


def algo_bytes_verify(d):
    B, T, _ = d["logits_bf16"].shape
    return d["logits_bf16"].size * 2 + d["drafts"].size * 4 + B * T * 8 + B * 4


def time_calls(torch, call, nslots, steps, warmup):
    """-> (end-to-end us per step, average kernel us from per-launch event pairs)."""
    for i in range(warmup):
        call(i % nslots)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(steps):
        call(i % nslots)
    t1.record()
    torch.cuda.synchronize()
    e2e = t0.elapsed_time(t1) * 1000.0 / steps
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i in range(steps):
        ev[i][0].record()
        call(i % nslots)
        ev[i][1].record()
    torch.cuda.synchronize()
    kern = sum(a.elapsed_time(b) for a, b in ev) * 1000.0 / steps
    return e2e, kern


def time_graph(torch, make_call, nslots, steps, warmup):
    """-> us per step of the same calls captured in a HIP graph (up to 200 launches per graph), replayed back to
    back. The call is bound on a side stream outside the capture (its workspace is zeroed there, eagerly), then
    captured on that stream: only the kernels are recorded."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call = make_call()
        for i in range(warmup):
            call(i % nslots)
    torch.cuda.synchronize()
    n = max(1, min(steps, 200))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for i in range(n):
            call(i % nslots)
    reps = max(steps // n, 3)
    g.replay()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1000.0 / (reps * n)


def prepared_slots(torch, dev, d, nslots):
    """-> (call(i), last output): nslots copies of the batch, logits and packed rows (parameters and histories)
    each in its own device buffers, so that a rotation over them reads every input from HBM rather than from the
    Infinity Cache; call(i) launches vs_sample_batch on copy i."""
    from volundr_amd import ops

    x = torch.from_numpy(d["logits"]).to(dev)
    rows = ops.pack_rows(d["params"], d["u"], V, d["hists"], hist_pairs=d.get("hist_pairs", False))
    preps = [ops.PreparedSample([x if i == 0 else x.clone()], rows.to(dev)) for i in range(nslots)]
    return (lambda i: preps[i](0)), preps


def bench_sample_graph(torch, dev, d, steps, warmup, nslots):
    """The benchmarked vs_sample_batch call, captured in a HIP graph (time_graph)."""
    return time_graph(torch, lambda: prepared_slots(torch, dev, d, nslots)[0], nslots, steps, warmup)


def bench_sample(torch, dev, d, steps, warmup, nslots):
    B = d["logits"].shape[0]
    call, preps = prepared_slots(torch, dev, d, nslots)
    cold = time_calls(torch, call, nslots, steps, warmup)
    warm = time_calls(torch, call, 1, steps, warmup)
    out = preps[0].out
    flags = out.flags.cpu().numpy()
    assert not any((int(f) & 0xFFFFFFFF) >> 31 for f in flags), "timeout flag set"
    return cold, warm, algo_bytes_sample(d, B), out


def bench_dropin(torch, dev, d, steps):
    """The drop-in routes of sampler.py as a scheduler calls them, host work included: one
    sample_rows_for(logits, samplers) per step (packing, uploads, one launch, the result copies), and the per-row
    Sampler.choose loop of scheduler.py:416-425. Wall-clock us per step (both return host ints, so both synchronise)."""
    from volundr_amd import Sampler
    from volundr_amd.sampler import sample_rows_for

    B, Vx = d["logits"].shape
    x = torch.from_numpy(d["logits"]).to(dev)

    def mk():
        ss = []
        for r, sp in enumerate(d["params"]):
            s = Sampler(sp, vocab_valid=Vx, request_id=r)
            for tok in (d["hists"][r] if d["hists"] is not None else ()):
                s.accept(int(tok))
            ss.append(s)
        return ss

    n = max(steps // 5, 50)
    ss = mk()
    for _ in range(3):
        sample_rows_for(x, ss)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        sample_rows_for(x, ss)
    batched = (time.perf_counter() - t0) * 1e6 / n
    ss = mk()
    for i, s in enumerate(ss):
        s.choose(x[i])
    torch.cuda.synchronize()
    nl = max(n // 4, 3)
    t0 = time.perf_counter()
    for _ in range(nl):
        for i, s in enumerate(ss):
            s.choose(x[i])
    loop = (time.perf_counter() - t0) * 1e6 / nl
    # a serving engine holding the requests in a DeviceSamplers table: one synchronous step per batch
    from volundr_amd import DeviceSamplers

    ds = DeviceSamplers(mk(), Vx, hist_cap=8192, device=dev)
    for _ in range(3):
        ds.step(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        ds.step(x)
    served = (time.perf_counter() - t0) * 1e6 / n
    return batched, loop, served


def bench_state(torch, dev, d, steps, warmup, nslots):
    """C3 through vs_sample_batch_state: the same rows with the sampler state (draw, history, produced) on the
    device, each call also accepting its token; the history pool has room for every call of the run."""
    from volundr_amd import DeviceSamplers, Sampler

    B, V = d["logits"].shape
    samplers = []
    for r, sp in enumerate(d["params"]):
        s = Sampler(sp, vocab_valid=V, request_id=r)
        s.rng = 0x9E3779B97F4A7C15 ^ r
        for tok in (d["hists"][r] if d["hists"] is not None else ()):
            s.accept(int(tok))
        samplers.append(s)
    h0 = 0 if d["hists"] is None else d["hists"].shape[1]
    ds = DeviceSamplers(samplers, V, hist_cap=h0 + 4 * (steps + warmup) + 64, device=dev)
    x = torch.from_numpy(d["logits"]).to(dev)
    slots = [x] + [x.clone() for _ in range(nslots - 1)]
    call = ds.bind(slots)
    cold = time_calls(torch, call, nslots, steps, warmup)
    warm = time_calls(torch, call, 1, steps, warmup)
    flags = ds.out.flags.cpu().numpy()
    assert not any((int(f) & 0xFFFFFFFF) >> 31 for f in flags), "timeout flag set"
    return cold, warm, algo_bytes_sample(d, B)


def bench_verify(torch, dev, d, steps, warmup, nslots):
    import numpy as np

    from volundr_amd import ops

    x = torch.from_numpy(d["logits_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
    slots = [x] + [x.clone() for _ in range(nslots - 1)]
    call = ops.PreparedVerify(slots, torch.from_numpy(d["drafts"]).to(dev))
    cold = time_calls(torch, call, nslots, steps, warmup)
    warm = time_calls(torch, call, 1, steps, warmup)
    acc = call.out.accept.cpu().numpy()
    return cold, warm, algo_bytes_verify(d), int(acc.sum() + len(acc))


DRAFT_V, DRAFT_VV, DRAFT_S, DRAFT_R = 248320, 248077, 7, 256


def bench_draft(torch, dev, steps, warmup, nslots):
    """DFlash2 propose after the head (spec/dflash.py:228-240): top-16 of the 7 block rows' bf16 logits
    [7, 248320] over the 248077 valid ids, then the 7-slot walk over rank-256 bf16 codebooks [248320, 256]."""
    from volundr_amd import ops

    g = torch.Generator(device=dev).manual_seed(6)
    x = (torch.randn(1, DRAFT_S, DRAFT_V, generator=g, device=dev) * 4).to(torch.bfloat16)
    slots = [x] + [x.clone() for _ in range(nslots - 1)]
    A = (torch.randn(DRAFT_V, DRAFT_R, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    B = (torch.randn(DRAFT_V, DRAFT_R, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    hp = torch.randn(1, DRAFT_S, DRAFT_R, generator=g, device=dev)
    anchor = torch.tensor([1234], dtype=torch.int32, device=dev)
    call = ops.PreparedPropose(slots, hp, A, B, anchor, vocab_valid=DRAFT_VV)
    cold = time_calls(torch, call, nslots, steps, warmup)
    warm = time_calls(torch, call, 1, steps, warmup)
    # logits once, the predecessor rows (anchor + 6 x 16 candidates) and successor rows (7 x 16), hp, drafts
    algo = DRAFT_S * DRAFT_VV * 2 + (1 + (DRAFT_S - 1) * 16 + DRAFT_S * 16) * DRAFT_R * 2 + DRAFT_S * DRAFT_R * 4 \
        + DRAFT_S * 4
    return cold, warm, algo


LMH_N, LMH_VV, LMH_K = 248320, 248077, 5120


def bench_lmhead(torch, dev, steps, warmup, B=1, T=17):
    """lm_head + greedy verify at the model's head (volundr.py:958-968: hidden 5120 -> vocab 248320, bf16) for B
    requests of T positions: the fused kernel (vs_lmhead_verify_greedy) and, for comparison, torch's bf16 matmul
    (hipBLASLt) writing the logits followed by vs_verify_greedy reading them."""
    from volundr_amd import ops

    g = torch.Generator(device=dev).manual_seed(5)
    h = torch.randn(B, T, LMH_K, generator=g, device=dev).to(torch.bfloat16)
    W = (torch.randn(LMH_N, LMH_K, generator=g, device=dev) / 16).to(torch.bfloat16)
    drafts = torch.randint(0, LMH_VV, (B, T - 1), generator=g, device=dev, dtype=torch.int32)
    out = ops.VerifyOut(torch.empty(B, T, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev),
                        torch.empty(B, T, dtype=torch.float32, device=dev))
    fused = lambda i: ops.lmhead_verify_greedy(h, W, drafts, vocab_valid=LMH_VV, out=out)  # noqa: E731
    lg = torch.empty(B * T, LMH_N, dtype=torch.bfloat16, device=dev)
    h2 = h.reshape(B * T, LMH_K)

    def unfused(i):
        torch.matmul(h2, W.T, out=lg)
        ops.verify_greedy(lg.view(B, T, LMH_N), drafts, LMH_VV)

    # Blocks of 10 calls, fused and unfused alternating, the median block of each: a single block now and then
    # runs ~15 us per call slower (on either path), which a plain mean over a few calls turns into noise.
    for _ in range(max(warmup // 10, 3)):
        fused(0)
        unfused(0)
    torch.cuda.synchronize()

    def block(fn, n=10):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / n

    fb, ub = [], []
    for _ in range(max(steps // 50, 3)):
        fb.append(block(fused))
        ub.append(block(unfused))
    med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
    algo = LMH_N * LMH_K * 2 + B * T * LMH_K * 2 + B * T * 8 + B * 4
    return (med(fb), med(fb)), (med(ub), med(ub)), algo


def bench_lmhead_sample(torch, dev, steps, warmup, R=16):
    """lm_head + Sampler.sample for R decode rows with top-k (and a greedy row), fused (vs_lmhead_sample: the GEMM
    keeps each workgroup's candidates, a second launch draws) against torch's bf16 matmul writing the logits followed
    by vs_sample_batch reading them. Same head as bench_lmhead; the row parameters of C3's top-k rows (k 20 / 50,
    top-p, temperature) with no penalties."""
    import numpy as np

    from volundr_amd import ops
    from volundr_amd.session import Sampling

    g = torch.Generator(device=dev).manual_seed(7)
    h = torch.randn(R, LMH_K, generator=g, device=dev).to(torch.bfloat16)
    W = (torch.randn(LMH_N, LMH_K, generator=g, device=dev) / 16).to(torch.bfloat16)
    rng = np.random.default_rng(8)
    sps = [Sampling(temperature=float(rng.uniform(0.6, 1.2)), top_k=int(rng.choice([20, 50])),
                    top_p=float(rng.choice([0.8, 0.95, 1.0]))) for _ in range(R - 1)] + [Sampling(temperature=0.0)]
    u = rng.random(R)
    rows = ops.pack_rows(sps, u, LMH_N, None).to(dev)
    out = ops.alloc_out(R, dev)
    L = ops._lib.load()
    ws = ops.workspace(dev, L.vs_lmhead_sample_workspace_bytes(R), "lmsample")
    st = ops._stream_handle(dev)

    def fused(i):
        L.vs_lmhead_sample(h.data_ptr(), LMH_K, W.data_ptr(), LMH_K, LMH_N, LMH_K, R, rows.params.data_ptr(),
                           out.ids.data_ptr(), out.logprobs.data_ptr(), out.flags.data_ptr(), out.keep.data_ptr(),
                           ws.data_ptr(), ws.numel(), st)

    lg = torch.empty(R, LMH_N, dtype=torch.bfloat16, device=dev)
    out2 = ops.alloc_out(R, dev)

    def unfused(i):
        torch.matmul(h, W.T, out=lg)
        ops.sample_rows(lg, rows, out2)

    for _ in range(max(warmup // 10, 3)):
        fused(0)
        unfused(0)
    torch.cuda.synchronize()

    def block(fn, n=10):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(n):
            fn(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / n

    fb, ub = [], []
    for _ in range(max(steps // 50, 3)):
        fb.append(block(fused))
        ub.append(block(unfused))
    med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
    algo = LMH_N * LMH_K * 2 + R * LMH_K * 2 + R * 96 + R * 16
    return med(fb), med(ub), algo


def read_ceiling(torch, dev, steps):
    """The streaming ceiling of the head kernels: vs_stream_read over a buffer of the lm_head weight's size (2.54 GB),
    one 512-thread workgroup per CU (the head kernel's grid) and four per CU; GB/s of the median of 10-call blocks."""
    from volundr_amd import _lib

    L = _lib.load()
    nbytes = LMH_N * LMH_K * 2
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    out = torch.zeros(4096, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream(dev).cuda_stream
    res = {"bytes": nbytes}
    for mult in (1, 4):
        call = lambda i: _lib.check(L.vs_stream_read(buf.data_ptr(), nbytes, cus * mult, out.data_ptr(), stream),  # noqa
                                    "vs_stream_read")
        for _ in range(3):
            call(0)
        torch.cuda.synchronize()
        blocks = []
        for _ in range(max(steps // 100, 5)):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(10):
                call(i)
            e1.record()
            torch.cuda.synchronize()
            blocks.append(e0.elapsed_time(e1) * 100.0)  # us per call
        us = sorted(blocks)[len(blocks) // 2]
        res[f"{mult}_per_cu"] = {"us": round(us, 1), "gbps": round(nbytes / (us * 1e-6) / 1e9, 1),
                                 "frac_of_8tbs": round(nbytes / (us * 1e-6) / 1e12 / 8.0, 4)}
    del buf
    return res


def launch_floor(torch, dev, steps):
    """Microseconds per launch of an empty kernel issued back to back through the library's C ABI, for a
    one-workgroup grid and for full-chip grids of 512-thread workgroups: one launch per Python call (the way the
    benchmark loops issue the sampling kernel, host overhead included) and 100 launches per call (the device-side
    floor: dispatch, start-up and completion of a kernel of that shape)."""
    from volundr_amd import _lib

    L = _lib.load()
    stream = torch.cuda.current_stream(dev).cuda_stream
    res = {}
    for key, (blocks, threads, lds) in {"1x64": (1, 64, 0), "256x512": (256, 512, 0),
                                         "256x512_lds96k": (256, 512, 96 * 1024)}.items():
        for reps in (1, 100):
            call = lambda i: _lib.check(L.vs_launch_floor(blocks, threads, lds, reps, stream),  # noqa: E731
                                        "vs_launch_floor")
            e2e, _ = time_calls(torch, call, 1, max(steps // reps, 5), 5)
            res[f"{key}{'' if reps == 1 else '_device'}"] = round(e2e / reps, 2)
    return res


def boundary_rows(d, out):
    """For the benched seed, computed outside the timed region: the oracle's count of rows whose draw lies within
    1e-6 of a CDF boundary or whose top-p cut lies within 1e-6 of a cumulative boundary (the rows the parity
    contract would excuse; near-flat top-p rows have CDF steps of ~7e-6, so many qualify), and how many rows'
    tokens and kept-set sizes actually differ from the oracle's."""
    from oracle import sampler_ref as S

    ids = out.ids.cpu().numpy()
    keep = out.keep.cpu().numpy()
    nb = nd = nk = 0
    for i in range(d["logits"].shape[0]):
        c = S.counts_from_history(d["hists"][i]) if d["hists"] is not None else {}
        r = S.sample(d["logits"][i], d["params"][i], float(d["u"][i]), c)
        nb += int(r.kind == "sample" and (r.draw_boundary or r.topp_boundary))
        nd += int(ids[i] != r.token)
        nk += int(r.kind == "sample" and keep[i] != r.keep)
    return {"boundary_rows": nb, "token_mismatches": nd, "keep_mismatches": nk, "rows": int(d["logits"].shape[0])}


def cpu_baseline(d, budget_s=10.0):
    """The reference's algorithm on the host, single-threaded, for about budget_s seconds: sampler.py:100-156 as
    written there (np.argpartition for top-k rows, lexsort, float64 exp / cumsum / searchsorted; the restatement
    oracle.sampler_ref.sample_plain), row by row as scheduler.py:424 calls it, with each request's counts dict built
    outside the timed loop (the reference keeps it across steps)."""
    from oracle import sampler_ref as S

    B = d["logits"].shape[0]
    counts = [S.counts_from_history(h) for h in d["hists"]] if d["hists"] is not None else [{}] * B
    n = 0
    t0 = time.perf_counter()
    while True:
        for i in range(B):
            S.sample_plain(d["logits"][i], d["params"][i], float(d["u"][i]), counts[i])
        n += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = (time.perf_counter() - t0) / n
    return {"value": round(dt * 1e6, 1), "unit": "us/step", "cores": 1, "kind": "port",
            "sample": f"{n} passes over the {B} rows of the same synthetic batch: sampler.py:100-156 restated "
                      f"with the reference's own NumPy calls (argpartition top-k, lexsort, exp, cumsum, "
                      f"searchsorted), counts dicts built outside the timed loop; 1 thread, "
                      f"os.cpu_count()={os.cpu_count()}",
            "tokens_per_s": round(B / dt, 1)}


def load_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (profiles/traffic_<name>.json)."""
    p = ROOT / "profiles" / f"traffic_{name}.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("bytes_per_launch")
        except Exception:
            return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--slots", type=int, default=32, help="rotating logits buffers (cold-HBM measurement)")
    ap.add_argument("--config", default="c3")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--hist-form", choices=("pairs", "raw"), default="pairs",
                    help="penalty input: sorted (id, count) tables (Sampler.counts) or the raw token histories")
    ap.add_argument("--no-others", action="store_true")
    ap.add_argument("--others", default="", help="comma-separated subset of other_configs to run (default: all)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB --steps times (rocprof counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the token-selection path is per-row and needs no collectives; "
              "run it with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from volundr_amd import synth

    dev = torch.device("cuda:0")
    if a.copy_calibration:
        n = a.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(a.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4, "steps": a.steps}))
        return
    d = synth.CONFIGS[a.config](seed=0)
    d["hist_pairs"] = a.hist_form == "pairs"
    verify = "logits_bf16" in d
    if verify:
        (e2e, kern), (e2e_w, kern_w), algo, ntok = bench_verify(torch, dev, d, a.steps, a.warmup, a.slots)
        B = d["logits_bf16"].shape[0]
    else:
        (e2e, kern), (e2e_w, kern_w), algo, sout = bench_sample(torch, dev, d, a.steps, a.warmup, a.slots)
        B = d["logits"].shape[0]
        ntok = B
    others = {}

    def entry(e2e_, ev_, e2e_w_, ab_, ntok_):
        return {"us_per_step": round(e2e_, 2), "warm_us_per_step": round(e2e_w_, 2),
                "kernel_us_event_pairs": round(ev_, 2), "algo_bytes": ab_,
                "hbm_gbps": round(ab_ / (e2e_ * 1e-6) / 1e9, 1), "tokens_per_s": round(ntok_ / (e2e_ * 1e-6), 1)}

    want = set(x for x in a.others.split(",") if x)
    sel = lambda name: not want or name in want  # noqa: E731
    if not a.no_others:
        for name in ("c1", "c3", "c5"):
            if name == a.config or not sel(name):
                continue
            dd = synth.CONFIGS[name](seed=0)
            dd["hist_pairs"] = a.hist_form == "pairs"
            (oe, ok), (we, wk), ab, oout = bench_sample(torch, dev, dd, a.steps, a.warmup, a.slots)
            others[name] = entry(oe, ok, we, ab, dd["logits"].shape[0])
            if not a.no_cpu:
                others[name].update(boundary_rows(dd, oout))
        for name in ("c3", "c5"):  # the same rows with the raw token histories as the penalty input
            if a.hist_form != "pairs" or not sel(name + "_raw"):
                continue
            dd = synth.CONFIGS[name](seed=0)
            (oe, ok), (we, wk), ab, oout = bench_sample(torch, dev, dd, a.steps, a.warmup, a.slots)
            others[name + "_raw"] = entry(oe, ok, we, ab, dd["logits"].shape[0])
            others[name + "_raw"]["workload"] = WORKLOADS[name + "_raw"]
        if sel("c3_greedy"):
            # C3's logits and histories with every row greedy (temperature 0, same penalties): the argmax class
            from volundr_amd.session import Sampling
            dd = synth.CONFIGS["c3"](seed=0)
            dd["params"] = [Sampling(temperature=0.0, repetition_penalty=p.repetition_penalty,
                                     presence_penalty=p.presence_penalty) for p in dd["params"]]
            dd["hist_pairs"] = a.hist_form == "pairs"
            (oe, ok), (we, wk), ab, oout = bench_sample(torch, dev, dd, a.steps, a.warmup, a.slots)
            others["c3_greedy"] = entry(oe, ok, we, ab, dd["logits"].shape[0])
        if sel("c3_dropin"):
            dd = synth.CONFIGS["c3"](seed=0)
            bt, lp, sv = bench_dropin(torch, dev, dd, a.steps)
            others["c3_dropin"] = {"sample_rows_for_us_per_step": round(bt, 1), "choose_loop_us_per_step": round(lp, 1),
                                   "device_samplers_step_us_per_step": round(sv, 1),
                                   "workload": "C3 through the drop-in routes, host work included (wall clock, the "
                                               "token ids back on the host): one sample_rows_for per step, the "
                                               "per-row Sampler.choose loop, and DeviceSamplers.step (sync)"}
        if sel("c3_state"):
            dd = synth.CONFIGS["c3"](seed=0)
            (oe, ok), (we, wk), ab = bench_state(torch, dev, dd, a.steps, a.warmup, a.slots)
            others["c3_state"] = entry(oe, ok, we, ab, dd["logits"].shape[0])
        for name in ("c2", "c4"):
            if name == a.config or not sel(name):
                continue
            dd = synth.CONFIGS[name](seed=0)
            (oe, ok), (we, wk), ab, nt = bench_verify(torch, dev, dd, a.steps, a.warmup, a.slots)
            others[name] = entry(oe, ok, we, ab, nt)
        if sel("draft_propose"):
            (oe, ok), (we, wk), ab = bench_draft(torch, dev, a.steps, a.warmup, a.slots)
            others["draft_propose"] = entry(oe, ok, we, ab, DRAFT_S)
            others["draft_propose"]["workload"] = ("DFlash2 propose: top-16 of bf16 logits [7, 248320] (248077 valid) "
                                                   "+ 7-slot walk, rank-256 codebooks; 2 kernels per step")
        for (bb, tt) in ((1, 17), (4, 17), (16, 1)):
            key = f"lmhead_verify_b{bb}t{tt}"
            if not sel(key):
                continue
            (fe, fk), (ue, uk), ab = bench_lmhead(torch, dev, a.steps, a.warmup, bb, tt)
            others[key] = entry(fe, fk, fe, ab, bb * tt)
            what = "greedy decode (argmax + logprob)" if tt == 1 else "greedy verify"
            others[key]["workload"] = (f"bf16 lm_head 5120 -> 248320 + {what}, B={bb} T={tt}: fused kernel; "
                                       "'unfused_us_per_step' = torch bf16 matmul (logits to HBM) + vs_verify_greedy; "
                                       "both the median of alternating 10-call blocks")
            others[key]["unfused_us_per_step"] = round(ue, 2)
            others[key]["frac_of_8tbs"] = round(ab / (fe * 1e-6) / 1e12 / 8.0, 4)
        if sel("lmhead_sample_b16"):
            fe, ue, ab = bench_lmhead_sample(torch, dev, a.steps, a.warmup)
            others["lmhead_sample_b16"] = entry(fe, fe, fe, ab, 16)
            others["lmhead_sample_b16"].update({
                "workload": "bf16 lm_head 5120 -> 248320 + Sampler.sample for 16 decode rows (15 top-k 20/50 rows "
                            "with temperature and top-p, 1 greedy): vs_lmhead_sample (candidates kept in the GEMM "
                            "epilogue, no logits in HBM, 2 launches); 'unfused_us_per_step' = torch bf16 matmul + "
                            "vs_sample_batch; both the median of alternating 10-call blocks",
                "unfused_us_per_step": round(ue, 2), "frac_of_8tbs": round(ab / (fe * 1e-6) / 1e12 / 8.0, 4)})
        if sel("read_ceiling"):
            others["read_ceiling"] = read_ceiling(torch, dev, a.steps)
            others["read_ceiling"]["workload"] = ("vs_stream_read: one streaming read of a buffer the size of the "
                                                  "lm_head weight (the ceiling the fused head kernels stream against)")
    cpu = None if (a.no_cpu or verify) else cpu_baseline(d)
    parity = None if (a.no_cpu or verify) else boundary_rows(d, sout)
    floor = launch_floor(torch, dev, a.steps)
    # the same step captured in a HIP graph and replayed (host launch cost out of the loop)
    graph = None if verify else round(bench_sample_graph(torch, dev, d, a.steps, a.warmup, a.slots), 2)
    # One kernel per step, launched back to back: the per-step time is the kernel's average launch duration plus
    # the inter-dispatch gap (rocprofv3 --kernel-trace agrees within a few percent); per-launch event pairs add
    # their own overhead and are reported separately.
    ach = algo / (e2e * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(e2e, 2), "unit": "us", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(e2e / 1000.0, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if verify else "f32", "data": "synthetic",
        "config": {"workload": WORKLOADS[a.config] + (HIST_FORM if d.get("hist_pairs") and d.get("hists") is not None
                                                      else ""), "B": B, "V": V,
                   "history_len": None if verify or d["hists"] is None else int(d["hists"].shape[1]),
                   "logit_slots": a.slots},
        "tokens_per_s": round(ntok / (e2e * 1e-6), 1),
        "hbm_gbps": round(algo / (e2e * 1e-6) / 1e9, 1),
        "kernel_us_event_pairs": round(kern, 2), "warm_us_per_step": round(e2e_w, 2),
        "warm_kernel_us_event_pairs": round(kern_w, 2),
        "kernels_per_step": 1,
        "graph_us_per_step": graph,
        "launch_floor_us": floor,
        "parity": parity,
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(ach / PEAK_GBPS, 4), "traffic": load_traffic(a.config),
                     "algo_bytes": algo},
        "cpu_baseline": cpu,
        "other_configs": others,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
