"""The timeout path of the sampling kernel, forced from the host with a tiny spin limit (vs_set_spin_limit), so
that every kernel still exits normally: FULL-class rows, whose workgroups meet at row barriers, report
VS_OUT_TIMEOUT instead of hanging; rows that finished are correct; no request state is committed for a flagged row;
and the workspace is left zeroed, so the next ordinary call is exact without a reset."""
import numpy as np
import pytest
import torch

from volundr_amd import DeviceSamplers, Sampler, _lib, ops, synth
from volundr_amd._lib import OUT_TIMEOUT
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu


def _flags(out):
    return [int(f) & 0xFFFFFFFF for f in out.flags.cpu().tolist()]


def _forced(fn):
    L = _lib.load()
    L.vs_set_spin_limit(1)
    try:
        r = fn()
        torch.cuda.synchronize()
    finally:
        L.vs_set_spin_limit(0)
    return r


def test_timeouts_flagged_and_workspace_left_clean(dev):
    d = synth.CONFIGS["c3"](seed=1)
    x = torch.from_numpy(d["logits"]).to(dev)
    V = x.shape[1]
    rows = ops.pack_rows(d["params"], d["u"], V, d["hists"]).to(dev)
    clean = ops.sample_rows(x, rows)
    ids0, lp0, fl0 = clean.ids.cpu().tolist(), clean.logprobs.cpu().tolist(), _flags(clean)
    assert not any(f & OUT_TIMEOUT for f in fl0)
    print("[timeout] forced run, c3 seed 1", flush=True)
    t = _forced(lambda: ops.sample_rows(x, rows))
    fl = _flags(t)
    timed = [bool(f & OUT_TIMEOUT) for f in fl]
    assert any(timed)
    ids = t.ids.cpu().tolist()
    for r in range(len(fl)):
        if not timed[r]:
            assert ids[r] == ids0[r], r
    again = ops.sample_rows(x, rows)  # no reset: the timed-out rows left the workspace zeroed
    assert again.ids.cpu().tolist() == ids0
    assert again.logprobs.cpu().tolist() == lp0
    assert _flags(again) == fl0


def test_sampler_falls_back_to_a_cooperative_launch(dev):
    """A row whose barrier times out under a plain launch is repeated with a cooperative launch (the spin limit
    applies to plain launches only): Sampler.sample returns the same token and logprob as an unforced call, and
    consumes one draw, as the reference's sample() does."""
    sp = Sampling(temperature=0.8, top_p=0.9)  # FULL class on a full-vocabulary row: row barriers
    x = torch.randn(163840, generator=torch.Generator().manual_seed(2)).to(dev)
    a = Sampler(sp, vocab_valid=163840, request_id=3)
    b = Sampler(sp, vocab_valid=163840, request_id=3)
    b.rng = a.rng
    want = a.sample(x)
    print("[timeout] forced Sampler.sample", flush=True)
    got = _forced(lambda: b.sample(x))
    assert got == want and b.last_logprob == a.last_logprob and b.rng == a.rng
    assert len(b.history) == 0  # sample() does not accept


def test_sample_rows_for_falls_back(dev):
    from volundr_amd.sampler import sample_rows_for

    d = synth.CONFIGS["c3"](seed=3)
    x = torch.from_numpy(d["logits"]).to(dev)
    mk = lambda: [Sampler(sp, vocab_valid=x.shape[1], request_id=r) for r, sp in enumerate(d["params"])]  # noqa
    a, b = mk(), mk()
    for sa, sb in zip(a, b):
        sb.rng = sa.rng
    want = sample_rows_for(x, a)
    got = _forced(lambda: sample_rows_for(x, b))
    assert got == want and [s.rng for s in a] == [s.rng for s in b]


def test_device_state_not_committed_for_timed_out_rows(dev):
    d = synth.CONFIGS["c3"](seed=2)
    B, V = d["logits"].shape
    samplers = []
    for r, sp in enumerate(d["params"]):
        s = Sampler(sp, vocab_valid=V, request_id=r)
        s.rng = 0x1234567 ^ r
        samplers.append(s)
    ds = DeviceSamplers(samplers, V, hist_cap=64, device=dev)
    x = torch.from_numpy(d["logits"]).to(dev)
    st0 = ds.host_state().copy()
    out = _forced(lambda: ds.step(x, sync=False))
    fl = _flags(out)
    st1 = ds.host_state()
    assert any(f & OUT_TIMEOUT for f in fl)
    for r in range(B):
        if fl[r] & OUT_TIMEOUT:
            assert st1[r]["produced"] == st0[r]["produced"] and st1[r]["rng"] == st0[r]["rng"], r
            assert st1[r]["hist_len"] == st0[r]["hist_len"], r
        else:
            assert st1[r]["produced"] == st0[r]["produced"] + 1, r
    out2 = ds.step(x, sync=False)  # the next step runs normally
    assert not any(f & OUT_TIMEOUT for f in _flags(out2))


def _forced_later(fn, debug=0):
    """fn under a one-poll spin limit that spares each row's first barrier: every workgroup passes it, then at a
    later barrier the early arrivals give up while the last one passes and goes on alone."""
    L = _lib.load()
    L.vs_set_spin_limit(1)
    L.vs_set_debug(_lib.DEBUG_SPIN_LATER_BARRIERS | debug)
    try:
        r = fn()
        torch.cuda.synchronize()
    finally:
        L.vs_set_spin_limit(0)
        L.vs_set_debug(0)
    return r


def _near_flat_rows(seed, B=2, V=163840):
    g = np.random.default_rng(seed)
    x = (g.standard_normal((B, V)) * 0.1).astype(np.float32)
    sps = [Sampling(temperature=1.0, top_p=0.95), Sampling(temperature=0.8, top_p=0.9)][:B]
    return x, sps, g.random(B)


def _other_paths(case, V=163840):
    g = np.random.default_rng(11)
    if case == "topk_radix":  # top-k above the list class: a cooperative radix select over row barriers
        x = (g.standard_normal((2, V)) * 0.1).astype(np.float32)
        sps = [Sampling(top_k=3000, top_p=0.9), Sampling(top_k=1000)]
    elif case == "min_p":  # min-p on a large kept set: the radix path
        x = (g.standard_normal((2, V)) * 0.5).astype(np.float32)
        sps = [Sampling(min_p=0.2), Sampling(min_p=0.5, top_p=0.9)]
    else:  # heavy-tailed rows whose kept sets are small: gathered before the second barrier
        x = (g.standard_t(3, (2, V)) * 3.0).astype(np.float32)
        sps = [Sampling(top_p=0.9), Sampling(temperature=0.7)]
    return x, sps, g.random(2)


@pytest.mark.parametrize("case", ["c5", "b1_near_flat", "b2_near_flat", "c5_radix", "topk_radix", "min_p",
                                  "small_kept"])
def test_timeout_after_a_passed_barrier_flags_the_row(dev, case):
    """A workgroup that gives up at a later row barrier skips the work after it (the gathers that the row's last
    workgroup resolves, the later radix rounds): the row must come back flagged VS_OUT_TIMEOUT, never as a token
    resolved from partial data or as an unwritten result, and the workspace must be left clean."""
    debug = 0
    if case.startswith("c5"):
        d = synth.CONFIGS["c5"](seed=4)
        xn, sps, u, hists = d["logits"], d["params"], d["u"], d["hists"]
        debug = _lib.DEBUG_FORCE_RADIX if case == "c5_radix" else 0
    elif "near_flat" in case:
        xn, sps, u = _near_flat_rows(5, B=1 if case.startswith("b1") else 2)
        hists = None
    else:
        xn, sps, u = _other_paths(case)
        hists = None
    x = torch.from_numpy(xn).to(dev)
    rows = ops.pack_rows(sps, u, x.shape[1], hists).to(dev)
    L = _lib.load()
    L.vs_set_debug(debug)
    try:
        clean = ops.sample_rows(x, rows)
        ids0, lp0, k0, fl0 = clean.ids.cpu().tolist(), clean.logprobs.cpu().tolist(), clean.keep.cpu().tolist(), _flags(clean)
    finally:
        L.vs_set_debug(0)
    assert not any(f & OUT_TIMEOUT for f in fl0)
    for rep in range(3):
        print(f"[timeout] later-barrier forced run, {case} rep {rep}", flush=True)
        out = ops.alloc_out(x.shape[0], dev)
        out.ids.fill_(-7)  # a result the kernel did not write shows as -7
        out.flags.fill_(0)
        t = _forced_later(lambda: ops.sample_rows(x, rows, out), debug)
        fl, ids = _flags(t), t.ids.cpu().tolist()
        lps, keep = t.logprobs.cpu().tolist(), t.keep.cpu().tolist()
        print(f"[timeout]   flagged rows {sum(bool(f & OUT_TIMEOUT) for f in fl)} of {len(fl)}", flush=True)
        for r in range(len(fl)):
            assert ids[r] != -7, f"row {r}: no result written"
            if not fl[r] & OUT_TIMEOUT:
                assert (ids[r], lps[r], keep[r]) == (ids0[r], lp0[r], k0[r]), f"row {r}: unflagged wrong result"
        L.vs_set_debug(debug)
        try:
            again = ops.sample_rows(x, rows)  # no reset: the forced run left the workspace zeroed
            assert again.ids.cpu().tolist() == ids0 and again.logprobs.cpu().tolist() == lp0
        finally:
            L.vs_set_debug(0)


def test_sampler_retry_after_a_later_barrier_timeout(dev):
    sp = Sampling(temperature=0.8, top_p=0.9)
    x = torch.randn(163840, generator=torch.Generator().manual_seed(2)).to(dev)
    a = Sampler(sp, vocab_valid=163840, request_id=3)
    b = Sampler(sp, vocab_valid=163840, request_id=3)
    b.rng = a.rng
    want = a.sample(x)
    got = _forced_later(lambda: b.sample(x))
    assert got == want and b.last_logprob == a.last_logprob and b.rng == a.rng


def test_device_state_after_a_later_barrier_timeout(dev):
    """The state entry point under later-barrier timeouts (C5 rows: value bins and gathers): a flagged row commits
    nothing, an unflagged row commits exactly the token an unforced step commits."""
    d = synth.CONFIGS["c5"](seed=6)
    B, V = d["logits"].shape
    x = torch.from_numpy(d["logits"]).to(dev)

    def fresh():
        ss = []
        for r, sp in enumerate(d["params"]):
            s = Sampler(sp, vocab_valid=V, request_id=r)
            s.rng = 0x7654321 ^ r
            ss.append(s)
        return DeviceSamplers(ss, V, hist_cap=64, device=dev)

    ref = fresh()
    want = ref.step(x).ids
    st_want = ref.host_state().copy()
    ds = fresh()
    st0 = ds.host_state().copy()
    out = _forced_later(lambda: ds.step(x, sync=False))
    fl, ids = _flags(out), out.ids.cpu().tolist()
    st1 = ds.host_state()
    print(f"[timeout] state rows flagged {sum(bool(f & OUT_TIMEOUT) for f in fl)} of {B}", flush=True)
    for r in range(B):
        if fl[r] & OUT_TIMEOUT:
            assert st1[r]["produced"] == st0[r]["produced"] and st1[r]["rng"] == st0[r]["rng"], r
            assert st1[r]["hist_len"] == st0[r]["hist_len"], r
        else:
            assert ids[r] == want[r], r
            assert st1[r]["rng"] == st_want[r]["rng"] and st1[r]["hist_len"] == st_want[r]["hist_len"], r



@pytest.mark.parametrize("later", [False, True])
def test_device_state_step_retries_timed_out_rows(dev, later):
    """DeviceSamplers.step (synchronous) repeats the rows that timed out under a cooperative launch: the tokens,
    logprobs and every slot's state equal an unforced step's, and no row comes back flagged."""
    d = synth.CONFIGS["c5"](seed=7)
    B, V = d["logits"].shape
    x = torch.from_numpy(d["logits"]).to(dev)

    def fresh():
        ss = []
        for r, sp in enumerate(d["params"]):
            s = Sampler(sp, vocab_valid=V, request_id=r)
            s.rng = 0x5151 ^ r
            ss.append(s)
        return DeviceSamplers(ss, V, hist_cap=64, device=dev)

    ref = fresh()
    want = ref.step(x)
    ds = fresh()
    print(f"[timeout] state step retry, later={later}", flush=True)
    got = _forced_later(lambda: ds.step(x)) if later else _forced(lambda: ds.step(x))
    assert got.ids == want.ids and got.logprobs == want.logprobs
    assert not any(f & OUT_TIMEOUT for f in got.flags)
    assert np.array_equal(ds.host_state(), ref.host_state())
    assert ds.history(3) == ref.history(3)

@pytest.mark.parametrize("coop", [0, 1])
def test_wait_time_bound(dev, coop):
    """The row barriers give up after a bound in wall time (the GPU's 100 MHz real-time counter): 200 us under a
    plain launch, 5 ms under a cooperative one. The testing flag VS_DEBUG_WAIT_CLOCK makes every barrier
    unreachable, so each FULL row waits out the bound at its first barrier and reports VS_OUT_TIMEOUT; the call's
    duration measures the bound. The workspace is left clean for the next ordinary call."""
    d = synth.CONFIGS["c5"](seed=4)
    x = torch.from_numpy(d["logits"]).to(dev)
    rows = ops.pack_rows(d["params"], d["u"], x.shape[1], d["hists"]).to(dev)
    clean = ops.sample_rows(x, rows)
    ids0 = clean.ids.cpu().tolist()
    L = _lib.load()
    prev = L.vs_set_cooperative(coop)
    L.vs_set_debug(_lib.DEBUG_WAIT_CLOCK)
    try:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        print(f"[timeout] wait-clock bound, cooperative={coop}", flush=True)
        e0.record()
        t = ops.sample_rows(x, rows)
        e1.record()
        torch.cuda.synchronize()
    finally:
        L.vs_set_debug(0)
        L.vs_set_cooperative(prev)
    us = e0.elapsed_time(e1) * 1000.0
    print(f"[timeout] wait-clock call: {us:.1f} us (cooperative={coop})", flush=True)
    assert all(f & OUT_TIMEOUT for f in _flags(t))
    lo, hi = (5000.0, 8000.0) if coop else (200.0, 1000.0)
    assert lo <= us <= hi, us
    again = ops.sample_rows(x, rows)
    assert again.ids.cpu().tolist() == ids0



def _debug(flags, fn):
    L = _lib.load()
    L.vs_set_debug(flags)
    try:
        r = fn()
        torch.cuda.synchronize()
    finally:
        L.vs_set_debug(0)
    return r


def test_xcd_split_guard_flags_every_row(dev):
    """The placement guard of the L2 exchange: with the testing flag that makes each row's last workgroup claim a
    neighbouring XCD, every row of a batch laid out one row per XCD group (GREEDY, TOPK and FULL rows of C3 plus
    greedy rows) reports VS_OUT_TIMEOUT rather than a result resolved from partials it cannot trust, commits
    nothing, and leaves the workspace zeroed: the next ordinary call is exact."""
    d = synth.CONFIGS["c3"](seed=2)
    d["params"][3] = Sampling(temperature=0.0)  # a GREEDY row beside the TOPK and FULL ones
    x = torch.from_numpy(d["logits"]).to(dev)
    V = x.shape[1]
    rows = ops.pack_rows(d["params"], d["u"], V, d["hists"]).to(dev)
    clean = ops.sample_rows(x, rows)
    ids0, lp0, fl0 = clean.ids.cpu().tolist(), clean.logprobs.cpu().tolist(), _flags(clean)
    assert not any(f & OUT_TIMEOUT for f in fl0)
    print("[xcd split] fake split, c3 seed 2", flush=True)
    t = _debug(_lib.DEBUG_FAKE_XCD_SPLIT, lambda: ops.sample_rows(x, rows))
    assert all(f & OUT_TIMEOUT for f in _flags(t)), _flags(t)
    again = ops.sample_rows(x, rows)
    assert again.ids.cpu().tolist() == ids0
    assert again.logprobs.cpu().tolist() == lp0
    assert _flags(again) == fl0


def test_xcd_split_recovers_with_the_coherent_exchange(dev):
    """The retry path under a (faked) split, on a 16-row batch laid out one row group per XCD: the plain and the
    cooperative launch both report every row, the retry switches the process to the device-coherent exchange and
    repeats the call, and the results equal an unforced call's."""
    from volundr_amd.sampler import _sample_checked
    d = synth.CONFIGS["c3"](seed=3)
    x = torch.from_numpy(d["logits"]).to(dev)
    n = x.shape[0]
    args = (d["params"], list(d["u"]), d["hists"], [0] * n, [()] * n)
    want = ops.sample_batch(x, *args)
    w = (want.ids.cpu().tolist(), want.logprobs.cpu().tolist())
    print("[xcd split] retry path with a fake split, c3 seed 3", flush=True)
    with pytest.warns(RuntimeWarning, match="device-coherent"):
        got, _ = _debug(_lib.DEBUG_FAKE_XCD_SPLIT, lambda: _sample_checked(x, *args))
    assert (got.ids.cpu().tolist(), got.logprobs.cpu().tolist()) == w
