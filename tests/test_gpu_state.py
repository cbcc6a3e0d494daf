"""GPU parity of vs_sample_batch_state (the per-request sampler state on the device) against the oracle driven the
way Sampler.choose drives it (volundr-mlx/sampler.py:67-98): a sequence of steps, the uniform drawn only when a row
reaches the draw, every chosen token accepted into the history, produced counting the steps."""
import numpy as np
import pytest
import torch

from oracle import sampler_ref as S
from parity import check_sample
from volundr_amd import DeviceSamplers, Sampler
from volundr_amd._lib import OUT_HIST_FULL, OUT_TIMEOUT
from volundr_amd.ops import SampleOut
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu


class HostRef:
    """The oracle with Sampler's state: rng, counts (as a history), produced."""

    def __init__(self, sp, seed):
        self.sp = sp
        self.rng = S.seed_state(seed)
        self.hist = []
        self.produced = 0

    def step(self, x):
        nxt, u = S.xorshift64s_next(self.rng)
        r = S.sample(x, self.sp, u, S.counts_from_history(self.hist), self.produced)
        return r, nxt

    def accept(self, tok, drew, nxt):
        if drew:
            self.rng = nxt
        self.hist.append(int(tok))
        self.produced += 1


def _slice(out, r):
    return SampleOut(out.ids[r:r + 1], out.logprobs[r:r + 1], out.flags[r:r + 1], out.keep[r:r + 1])


@pytest.mark.parametrize("V", [5003, 40000])
def test_device_state_sequence(dev, V):
    rng = np.random.default_rng(V)
    sps = [Sampling(top_k=20, temperature=0.9, repetition_penalty=1.3, seed=11),
           Sampling(top_p=0.9, temperature=1.2, presence_penalty=0.5, frequency_penalty=0.2, seed=12),
           Sampling(temperature=0.0, repetition_penalty=1.5, seed=13),  # greedy: never draws
           Sampling(top_k=50, top_p=0.8, min_p=0.05, seed=14, min_new_tokens=3, stop_token_ids=[7, 9]),
           Sampling(temperature=0.7, seed=15, logit_bias=[(3, 2.0)], suppress_tokens=[5]),
           Sampling(top_k=300, temperature=1.0, repetition_penalty=0.8, seed=16)]
    samplers = [Sampler(sp, vocab_valid=V) for sp in sps]
    refs = [HostRef(sp, sp.seed) for sp in sps]
    ds = DeviceSamplers(samplers, V, hist_cap=64, device=dev)
    steps = 12
    for step in range(steps):
        x = (rng.standard_normal((len(sps), V)) * 2.5).astype(np.float32)
        x[:, 7] = x[:, 9] = 8.0  # the stop ids lead until min_new_tokens is reached
        print(f"[state V={V}] step {step}", flush=True)
        out = ds.step(torch.from_numpy(x).to(dev), sync=False)
        torch.cuda.synchronize()
        ids = out.ids.cpu().numpy()
        for r, ref in enumerate(refs):
            res, nxt = ref.step(x[r])
            check_sample(_slice(out, r), [res], f"state V{V} step {step} row {r}")
            ref.accept(ids[r], res.kind == "sample", nxt)  # follow the device on a boundary row
    st = ds.host_state()
    for r, ref in enumerate(refs):
        assert int(st[r]["rng"]) == ref.rng, f"row {r}: rng"
        assert int(st[r]["produced"]) == steps
        assert ds.history(r) == ref.hist
    assert int(st[2]["rng"]) == S.seed_state(13)  # the greedy row never drew
    ds.write_back()
    assert samplers[0].produced == steps and samplers[0].history == refs[0].hist


def test_device_state_history_full(dev):
    V = 3000
    sp = Sampling(top_k=5, repetition_penalty=2.0, seed=3)
    s = Sampler(sp, vocab_valid=V)
    for t in (1, 2, 3):
        s.accept(t)
    ds = DeviceSamplers([s], V, hist_cap=4, device=dev, grow_history=False)
    rng = np.random.default_rng(1)
    flags = []
    for _ in range(3):
        out = ds.step(torch.from_numpy(rng.standard_normal((1, V)).astype(np.float32)).to(dev), sync=False)
        flags.append(int(out.flags.cpu()[0]) & 0xFFFFFFFF)
    assert not flags[0] & OUT_HIST_FULL and flags[1] & OUT_HIST_FULL and flags[2] & OUT_HIST_FULL
    assert not any(f & OUT_TIMEOUT for f in flags)
    st = ds.host_state()[0]
    assert int(st["hist_len"]) == 4 and int(st["produced"]) == 6
    assert ds.history(0)[:3] == [1, 2, 3]


def test_device_state_bind_matches_step(dev):
    V = 8000
    rng = np.random.default_rng(9)
    sps = [Sampling(top_k=10, seed=21, repetition_penalty=1.2), Sampling(top_p=0.9, seed=22)]
    a = DeviceSamplers([Sampler(sp, vocab_valid=V) for sp in sps], V, hist_cap=16, device=dev)
    b = DeviceSamplers([Sampler(sp, vocab_valid=V) for sp in sps], V, hist_cap=16, device=dev)
    xs = [torch.from_numpy(rng.standard_normal((2, V)).astype(np.float32)).to(dev) for _ in range(3)]
    call = b.bind(xs)
    for i, x in enumerate(xs):
        ia = a.step(x, sync=False).ids.clone()
        ib = call(i).ids.clone()
        assert torch.equal(ia, ib)
    assert np.array_equal(a.host_state(), b.host_state())
    assert a.history(0) == b.history(0)


def test_bound_calls_grow_and_fold_like_step(dev):
    """600 bound calls from a pool of 16 tokens: the history grows and the tables take in the recent tokens on the
    same schedule as step(); a step() between bound calls keeps the bookkeeping. Tokens, slot states, tables and
    histories equal those of step() throughout."""
    V = 3000
    rng = np.random.default_rng(19)
    sps = [Sampling(top_k=20, seed=23, repetition_penalty=1.3, frequency_penalty=0.1),
           Sampling(top_p=0.9, seed=24, presence_penalty=0.5)]
    a = DeviceSamplers([Sampler(sp, vocab_valid=V) for sp in sps], V, hist_cap=16, device=dev)
    b = DeviceSamplers([Sampler(sp, vocab_valid=V) for sp in sps], V, hist_cap=16, device=dev)
    xs = [torch.from_numpy(rng.standard_normal((2, V)).astype(np.float32) * 2).to(dev) for _ in range(4)]
    call = b.bind(xs)
    print("[state] 600 bound calls", flush=True)
    for k in range(600):
        x = xs[k % 4]
        ia = a.step(x, sync=False).ids.clone()
        ib = (b.step(x, sync=False) if k == 300 else call(k % 4)).ids.clone()
        assert torch.equal(ia, ib), f"call {k}"
    assert np.array_equal(a.host_state(), b.host_state())
    st = b.host_state()
    assert all(int(st[q]["hist_base"]) >= 256 for q in range(2))  # folded under the bound calls
    assert torch.equal(a.tabs, b.tabs) and b.cap > 600
    assert a.history(0) == b.history(0) and len(b.history(1)) == 600
