"""Continuous batching on the device-resident sampler state (DeviceSamplers.admit / retire / step), against the
oracle driven as the reference's engine drives Sampler.choose: a Sampler is created when a request is admitted
(volundr-mlx/scheduler.py:148-151) and choose() runs for whichever requests are live at each step
(scheduler.py:402-425), budget force and bias included (sampler.py:85-92). Requests join and leave over 20 steps;
rows are stepped in admission order, in a reversed order and as a subset; one request's history outgrows the pool
(which then grows on the device). Tokens, logprobs, rng states, histories and produced counts are compared."""
import numpy as np
import pytest
import torch

from oracle import sampler_ref as S
from parity import LP_ATOL, LP_RTOL
from volundr_amd import DeviceSamplers, Sampler
from volundr_amd._lib import OUT_FORCED
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu

V, VV = 50000, 49900
THINK, UNTHINK = 1000, 1001
PAD_HOT = V - 7


class OracleRequest:
    """The oracle's view of one request: rng, the tokens produced (forced ones included), the prompt."""

    def __init__(self, sp, prompt=(), think=(None, None), history=()):
        self.sp, self.prompt, self.think = sp, list(prompt), think
        self.rng = S.seed_state(sp.seed)
        self.pre = list(history)  # tokens accepted before admission (count for the penalties, not for produced)
        self.gen = []

    def step(self, x):
        nxt, u = S.xorshift64s_next(self.rng)
        if self.pre:  # a request with earlier tokens and no budget: its penalties count them too
            assert not self.sp.reasoning_budget and self.sp.needs_logits(VV, len(self.gen))
            r = S.sample(x, self.sp, u, S.counts_from_history(self.pre + self.gen), len(self.gen))
        else:
            r = S.choose(x, self.sp, VV, u, self.gen, self.prompt, self.think)
        return r, nxt

    def accept(self, tok, r, nxt):
        if r.kind == "sample":
            self.rng = nxt
        self.gen.append(int(tok))


def _logits(rng, n):
    x = np.clip(rng.standard_normal((n, V)) * 2.0, -9.0, 9.0).astype(np.float32)
    x[:, PAD_HOT] = 12.0   # the row maximum sits in the padding: argmax-only requests must skip it
    x[:, 11] = 10.5        # the largest valid logit
    x[:, UNTHINK] = 9.5    # close behind: the budget's soft bias on it decides
    return x


def _check(label, tok, lp, r):
    if r.kind == "sample" and (r.draw_boundary or r.topp_boundary) and tok != r.token:
        return
    assert tok == r.token, f"{label}: token {tok} != oracle {r.token} ({r.kind})"
    if r.kind != "force":
        assert abs(lp - r.logprob) <= LP_RTOL * abs(r.logprob) + LP_ATOL, f"{label}: logprob {lp} vs {r.logprob}"
    else:
        assert lp == 0.0


REQUESTS = {
    "A": (Sampling(top_p=0.9, temperature=1.1, presence_penalty=0.4, repetition_penalty=1.2, seed=31), (), None),
    "B": (Sampling(temperature=0.0, seed=32), (), None),                                        # argmax-only
    "C": (Sampling(temperature=0.0, reasoning_budget=3, seed=33), (5, THINK), None),            # forced at step 3
    "D": (Sampling(top_k=20, temperature=0.8, min_new_tokens=3, stop_token_ids=[11], seed=34), (), None),
    "E": (Sampling(temperature=0.0, reasoning_budget=6, reasoning_budget_soft_bias=0.5, seed=35), (THINK,), None),
    "F": (Sampling(top_k=50, repetition_penalty=1.3, frequency_penalty=0.1, seed=36), (), "long"),
    "G": (Sampling(top_p=0.8, logit_bias=[(UNTHINK, 1.5), (3, -2.0)], suppress_tokens=[11], seed=37), (), None),
}
# step -> (admit, retire) before that step
SCHEDULE = {0: ("ABC", ""), 3: ("D", "B"), 6: ("E", ""), 10: ("F", "A"), 14: ("G", "C"), 17: ("", "D")}


def test_continuous_batching_against_oracle(dev):
    rng = np.random.default_rng(123)
    ds = DeviceSamplers([], V, hist_cap=64, device=dev, capacity=2)  # grows to more slots and a larger pool
    live, slot_of, host, orc, done = [], {}, {}, {}, {}
    forced_seen = 0
    for step in range(20):
        adm, ret = SCHEDULE.get(step, ("", ""))
        for name in ret:
            ds.retire(slot_of[name])  # writes the device state back into the host Sampler
            done[name] = host[name]
            live.remove(name)
        for name in adm:
            sp, prompt, hist = REQUESTS[name]
            think = (THINK, UNTHINK) if sp.reasoning_budget else (None, None)
            s = Sampler(sp, prompt=prompt, think_ids=think, vocab_valid=VV)
            pre = []
            if hist == "long":  # accepted before admission (not counted in produced): 100 tokens, pool of 64
                pre = rng.integers(0, VV, 100).tolist()
                for t in pre:
                    s.history.append(t)
                    s.counts[t] = s.counts.get(t, 0) + 1
            host[name] = s
            orc[name] = OracleRequest(sp, prompt, think, pre)
            slot_of[name] = ds.admit(s)
            live.append(name)
        names = list(live)
        if step in (8, 15):
            names = names[::-1]                    # rows in any order
        if step == 12:
            names = names[:-1]                     # a subset: the last request sits this step out
        x = _logits(rng, len(names))
        print(f"[batching] step {step}: {''.join(names)}", flush=True)
        res = ds.step(torch.from_numpy(x).to(dev), [slot_of[n] for n in names])
        for i, name in enumerate(names):
            r, nxt = orc[name].step(x[i])
            _check(f"step {step} {name}", res.ids[i], res.logprobs[i], r)
            if r.kind == "force":
                assert res.flags[i] & OUT_FORCED
                forced_seen += 1
            orc[name].accept(res.ids[i], r, nxt)
    ds.write_back()
    for name, s in list(host.items()):
        o = orc[name]
        assert s.rng == o.rng, f"{name}: rng"
        assert list(s.history) == o.pre + o.gen, f"{name}: history"
        assert s.produced == len(o.gen), f"{name}: produced"
    assert forced_seen == 2                               # C at its third thinking token, E at its sixth
    assert orc["C"].gen[3] == UNTHINK and orc["E"].gen[6] == UNTHINK
    assert orc["B"].gen == [11] * 3                       # argmax over [:vv] skips the padding maximum
    assert ds.cap > 64 and ds.S > 2                       # the pool and the slot table grew


def test_admit_retire_reuses_slots(dev):
    """A retired slot is reused by the next admission, and the new request starts from its own state."""
    rng = np.random.default_rng(5)
    sp = Sampling(top_k=10, repetition_penalty=1.5, seed=41)
    ds = DeviceSamplers([Sampler(sp, vocab_valid=VV)], V, hist_cap=64, device=dev)
    for _ in range(3):
        ds.step(torch.from_numpy(_logits(rng, 1)).to(dev))
    old = ds.samplers[0]
    ds.retire(0)
    assert old.produced == 3 and len(old.history) == 3
    fresh = Sampler(Sampling(top_k=10, repetition_penalty=1.5, seed=41), vocab_valid=VV)
    q = ds.admit(fresh)
    assert q == 0
    x = _logits(rng, 1)
    res = ds.step(torch.from_numpy(x).to(dev))
    o = OracleRequest(fresh.sp)
    r, _ = o.step(x[0])
    _check("reused slot", res.ids[0], res.logprobs[0], r)
    assert ds.history(0) == [res.ids[0]]


def test_long_run_folds_the_tables(dev):
    """700 steps of penalised sampling: each slot's (id, count) table takes in its recent tokens every 256 or so
    (vs_state_fold); every step must equal the oracle over the whole history, and the tables must hold exactly the
    counts of the history they cover."""
    from volundr_amd._lib import STATE_DTYPE

    Vs = 3000
    rng = np.random.default_rng(31)
    sps = [Sampling(top_k=30, repetition_penalty=1.3, frequency_penalty=0.05, presence_penalty=0.2, seed=71),
           Sampling(top_p=0.9, temperature=1.2, repetition_penalty=1.1, seed=72),
           Sampling(temperature=0.0, repetition_penalty=2.0, frequency_penalty=0.5, seed=73)]
    ss = [Sampler(sp, vocab_valid=Vs) for sp in sps]
    pre = rng.integers(0, Vs, 300).tolist()
    for t in pre:  # an earlier history for the first request: its table is built at admission
        ss[0].history.append(t)
        ss[0].counts[t] = ss[0].counts.get(t, 0) + 1
    hists = [list(pre), [], []]
    refs = []
    for r, sp in enumerate(sps):
        refs.append([S.seed_state(sp.seed)])
    ds = DeviceSamplers(ss, Vs, hist_cap=256, device=dev)
    print("[batching] long run: 700 steps, 3 rows", flush=True)
    for step in range(700):
        x = (rng.standard_normal((3, Vs)) * 1.5).astype(np.float32)
        res = ds.step(torch.from_numpy(x).to(dev))
        for r, sp in enumerate(sps):
            nxt, u = S.xorshift64s_next(refs[r][0])
            want = S.sample(x[r], sp, u, S.counts_from_history(hists[r]), len(hists[r]) - (300 if r == 0 else 0))
            _check(f"long step {step} row {r}", res.ids[r], res.logprobs[r], want)
            if want.kind == "sample":
                refs[r][0] = nxt
            hists[r].append(res.ids[r])
    st = ds.host_state()
    tabs = ds.tabs.cpu().numpy()
    for r in range(3):
        q = ds.order[r]
        base, off, n = int(st[q]["hist_base"]), int(st[q]["tab_off"]), int(st[q]["tab_len"])
        assert base > 256 and base <= len(hists[r])  # folded at least once
        ids, cnt = np.unique(np.asarray(hists[r][:base]), return_counts=True)
        tab = tabs[off:off + 2 * n].reshape(-1, 2)
        assert np.array_equal(tab[:, 0], ids) and np.array_equal(tab[:, 1], cnt), f"row {r}: table"
        assert ds.history(q) == hists[r]
    assert ds.cap > 256  # the pool (and the tables) grew past the first capacity


def test_fold_leaves_a_slot_whose_table_cannot_fit(dev):
    """vs_state_fold with a tab_cap below the slot's table plus its recent tokens changes nothing (the tokens stay
    counted from the history), and the next steps still equal the oracle."""
    from volundr_amd import _lib
    from volundr_amd.ops import _stream_handle

    Vs = 2000
    rng = np.random.default_rng(41)
    sp = Sampling(top_k=40, repetition_penalty=1.4, frequency_penalty=0.2, seed=81)
    ds = DeviceSamplers([Sampler(sp, vocab_valid=Vs)], Vs, hist_cap=512, device=dev)
    hist, ref = [], [S.seed_state(sp.seed)]

    def step():
        x = (rng.standard_normal((1, Vs)) * 1.5).astype(np.float32)
        res = ds.step(torch.from_numpy(x).to(dev))
        nxt, u = S.xorshift64s_next(ref[0])
        want = S.sample(x[0], sp, u, S.counts_from_history(hist), len(hist))
        _check(f"step {len(hist)}", res.ids[0], res.logprobs[0], want)
        if want.kind == "sample":
            ref[0] = nxt
        hist.append(res.ids[0])

    for _ in range(100):
        step()
    before = ds.host_state().copy()
    assert int(before[0]["hist_len"]) - int(before[0]["hist_base"]) == 100
    sl = torch.zeros(1, dtype=torch.int32, device=dev)
    L = _lib.load()
    _lib.check(L.vs_state_fold(ds.state.data_ptr(), ds.pool.data_ptr(), ds.tabs.data_ptr(), 50, sl.data_ptr(), 1,
                               _stream_handle(dev)), "vs_state_fold")
    assert np.array_equal(ds.host_state(), before)
    for _ in range(20):
        step()


@pytest.mark.parametrize("n_hist", [0, 2047, 2048, 2049, 6000])
def test_state_tables_around_the_prefetch_size(dev, n_hist):
    """State rows whose (id, count) tables hold up to PAIRS_ALL = 2048 entries (loaded whole) and beyond (bracketed
    by probes, the table entries and the recent tokens merged in one pass): 400 steps at V = 163840 (the first fold
    comes at step 384: checks every 128 steps, 256 recent tokens due) against the oracle over the whole history."""
    Vb = 163840
    rng = np.random.default_rng(n_hist + 5)
    sps = [Sampling(top_k=50, repetition_penalty=1.3, frequency_penalty=0.05, presence_penalty=0.3, seed=95),
           Sampling(top_p=0.9, repetition_penalty=0.8, frequency_penalty=-0.1, seed=96),
           Sampling(temperature=0.0, repetition_penalty=1.5, seed=97)]
    ss = [Sampler(sp, vocab_valid=Vb) for sp in sps]
    hists = []
    for s in ss:
        # n_hist distinct ids (some repeated) spread over the vocabulary: a table of about n_hist entries
        ids = rng.choice(Vb, size=n_hist, replace=False) if n_hist else np.zeros(0, dtype=np.int64)
        h = np.concatenate([ids, ids[: n_hist // 3]]).astype(np.int64)
        rng.shuffle(h)
        for t in h.tolist():
            s.history.append(t)
            s.counts[t] = s.counts.get(t, 0) + 1
        hists.append(h.tolist())
    pre = [len(h) for h in hists]
    refs = [S.seed_state(sp.seed) for sp in sps]
    ds = DeviceSamplers(ss, Vb, hist_cap=max(pre) + 512, device=dev)
    print(f"[batching] tables of {n_hist} entries, 400 steps", flush=True)
    for step in range(400):
        x = (rng.standard_normal((3, Vb)) * 2.0).astype(np.float32)
        if hists[0]:  # logits that the penalties decide: the history's ids near the top
            x[:, hists[0][:64]] += 4.0
        res = ds.step(torch.from_numpy(x).to(dev))
        for r, sp in enumerate(sps):
            nxt, u = S.xorshift64s_next(refs[r])
            want = S.sample(x[r], sp, u, S.counts_from_history(hists[r]), len(hists[r]) - pre[r])
            _check(f"tables {n_hist} step {step} row {r}", res.ids[r], res.logprobs[r], want)
            if want.kind == "sample":
                refs[r] = nxt
            hists[r].append(res.ids[r])
    st = ds.host_state()
    assert all(int(st[q]["hist_base"]) > pre[r] for r, q in enumerate(ds.order))  # folded during the run
