"""GPU parity of the drop-in routes the scheduler takes (volundr-mlx/sampler.py:83-98, called per row by
scheduler.py:416-425): Sampler.choose, the batched sample_rows_for and the device-resident DeviceSamplers, against
the oracle driven as Sampler.choose drives Sampler.sample (oracle.sampler_ref.choose). Covers every branch of
choose: the reasoning budget's force and bias, argmax-only requests (mx.argmax over [:vocab_valid]), greedy
requests that need the sampler (argmax over the full row), stop masks that move a request between the two, and
sampled rows. The production vocabulary is used: V = 248320 logits of which vocab_valid = 248077 are real, with the
row maximum planted in the padding columns."""
import numpy as np
import pytest
import torch

from oracle import sampler_ref as S
from parity import LP_ATOL, LP_RTOL
from volundr_amd import DeviceSamplers, Sampler
from volundr_amd.sampler import sample_rows_for
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu

V, VV = 248320, 248077
THINK, UNTHINK = 1000, 1001
PAD_HOT = V - 5          # a padding column that holds the row maximum


class OracleRequest:
    """Sampler state for the oracle: rng, the produced tokens (forced ones included), the prompt."""

    def __init__(self, sp, prompt=(), think=(None, None)):
        self.sp, self.prompt, self.think = sp, list(prompt), think
        self.rng = S.seed_state(sp.seed)
        self.gen = []

    def step(self, x):
        nxt, u = S.xorshift64s_next(self.rng)
        r = S.choose(x, self.sp, VV, u, self.gen, self.prompt, self.think)
        return r, nxt

    def accept(self, tok, r, nxt):
        if r.kind == "sample":
            self.rng = nxt
        self.gen.append(int(tok))


def _requests():
    """(Sampling, prompt, think_ids) per request: every branch of Sampler.choose."""
    return [
        (Sampling(temperature=0.0, seed=1), (), (None, None)),                                  # argmax-only
        (Sampling(top_k=1, min_new_tokens=2, stop_token_ids=[PAD_HOT], seed=2), (), (None, None)),  # stop, then argmax
        (Sampling(temperature=0.0, repetition_penalty=1.2, seed=3), (), (None, None)),          # greedy, full row
        (Sampling(top_k=20, temperature=0.8, seed=4), (), (None, None)),                        # sampled top-k
        (Sampling(top_p=0.9, temperature=1.1, presence_penalty=0.4, frequency_penalty=0.1, seed=5), (), (None, None)),
        (Sampling(temperature=0.0, suppress_tokens=[VV + 2], seed=6), (), (None, None)),        # suppress >= vv
        (Sampling(temperature=0.0, reasoning_budget=3, seed=7), (5, THINK), (THINK, UNTHINK)),   # budget force
        (Sampling(top_k=50, reasoning_budget=5, reasoning_budget_soft_bias=30.0, seed=8), (THINK,), (THINK, UNTHINK)),
    ]


def _logits(rng, B):
    x = np.clip(rng.standard_normal((B, V)) * 2.0, -10.0, 10.0).astype(np.float32)
    x[:, PAD_HOT] = 14.0           # the largest logit sits in the padding: only [:vv] argmaxes must skip it
    x[:, 7] = 11.5                 # the largest valid logit
    return x


def _check(label, tok, lp, r):
    if r.kind == "sample" and (r.draw_boundary or r.topp_boundary) and tok != r.token:
        return
    assert tok == r.token, f"{label}: token {tok} != oracle {r.token} ({r.kind})"
    if r.kind != "force" and lp is not None:
        assert abs(lp - r.logprob) <= LP_RTOL * abs(r.logprob) + LP_ATOL, f"{label}: logprob {lp} vs {r.logprob}"


def test_choose_and_sample_rows_for(dev):
    rng = np.random.default_rng(2024)
    reqs = _requests()
    B = len(reqs)
    per_row = [Sampler(sp, prompt=pr, think_ids=th, vocab_valid=VV) for sp, pr, th in reqs]
    batched = [Sampler(sp, prompt=pr, think_ids=th, vocab_valid=VV) for sp, pr, th in reqs]
    oracle = [OracleRequest(sp, pr, th) for sp, pr, th in reqs]
    kinds = set()
    for step in range(8):
        x = _logits(rng, B)
        xt = torch.from_numpy(x).to(dev)
        print(f"[choose] step {step}", flush=True)
        toks_b = sample_rows_for(xt, batched)
        torch.cuda.synchronize()
        for r in range(B):
            tok_a = per_row[r].choose(xt[r])
            res, nxt = oracle[r].step(x[r])
            kinds.add(res.kind)
            lab = f"step {step} row {r}"
            _check("choose " + lab, tok_a, per_row[r].last_logprob if res.kind != "force" else None, res)
            _check("sample_rows_for " + lab, toks_b[r], batched[r].last_logprob if res.kind != "force" else None, res)
            oracle[r].accept(tok_a, res, nxt)
            assert tok_b_follow(toks_b[r], tok_a, res)
    assert kinds == {"argmax", "greedy", "sample", "force"}
    for r in range(B):
        for s in (per_row[r], batched[r]):
            assert s.rng == oracle[r].rng, f"row {r}: rng"
            assert s.produced == len(oracle[r].gen)
    # the routes the planted padding maximum separates
    assert oracle[0].gen == [7] * 8                        # argmax over [:vv]
    assert oracle[1].gen[:2] == [7, 7] and oracle[1].gen[2:] == [7] * 6   # stop-masked, then [:vv]
    assert oracle[2].gen[0] == PAD_HOT                     # the sampler's argmax sees the whole row
    assert oracle[6].gen[3] == UNTHINK                     # forced after 3 thinking tokens


def tok_b_follow(tok_b, tok_a, res):
    """The two host routes agree except on an excused boundary row."""
    return tok_b == tok_a or (res.kind == "sample" and (res.draw_boundary or res.topp_boundary))


def test_device_samplers_vocab_valid(dev):
    """DeviceSamplers keeps every request's state on the device and must reproduce Sampler.choose, including the
    argmax over [:vocab_valid] for requests that need no logits and the switch when a stop mask expires."""
    rng = np.random.default_rng(77)
    reqs = [q for q in _requests() if q[0].reasoning_budget is None]
    B = len(reqs)
    samplers = [Sampler(sp, vocab_valid=VV) for sp, _, _ in reqs]
    oracle = [OracleRequest(sp) for sp, _, _ in reqs]
    ds = DeviceSamplers(samplers, V, hist_cap=32, device=dev)
    for step in range(6):
        x = _logits(rng, B)
        print(f"[device vv] step {step}", flush=True)
        out = ds.step(torch.from_numpy(x).to(dev), sync=False)
        ids = out.ids.cpu().numpy()
        lps = out.logprobs.cpu().numpy().astype(np.float64)
        for r in range(B):
            res, nxt = oracle[r].step(x[r])
            _check(f"state step {step} row {r}", int(ids[r]), float(lps[r]), res)
            oracle[r].accept(ids[r], res, nxt)
    st = ds.host_state()
    for r in range(B):
        assert int(st[r]["rng"]) == oracle[r].rng and ds.history(r) == oracle[r].gen
    assert oracle[0].gen == [7] * 6 and oracle[2].gen[0] == PAD_HOT


@pytest.mark.parametrize("vv", [V // 3, 12289, 1])
def test_argmax_vv_far_below_v(dev, vv):
    """Argmax-only rows whose vocab_valid lies far below V, so that whole workgroups of the row hold no valid
    position: NaN, +inf and the global maximum planted past vocab_valid must not leak in; the result is
    np.argmax(x[:vv]) (sampler.py:96), for one row alone and for rows of a batch with other classes."""
    from volundr_amd import ops

    rng = np.random.default_rng(vv)
    B = 3
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    for r in range(B):
        x[r, vv:][rng.integers(0, V - vv, 5)] = np.nan
        x[r, V - 1] = np.inf
        x[r, (vv + V) // 2] = 50.0
    x[1, :vv] = -np.inf if vv == 1 else x[1, :vv]     # vv = 1: a single -inf entry, argmax 0
    x[2, vv - 1] = 30.0                               # the valid maximum at the last valid position
    sps = [Sampling(temperature=0.0), Sampling(top_k=1), Sampling(temperature=0.0)]
    print(f"[argmax vv] V={V} vv={vv}", flush=True)
    xt = torch.from_numpy(x).to(dev)
    rows = ops.pack_rows(sps, np.zeros(B), V, argmax_vv=[vv] * B).to(dev)
    o = ops.sample_rows(xt, rows)
    torch.cuda.synchronize()
    want = [int(np.argmax(x[r, :vv])) for r in range(B)]
    assert o.ids.cpu().tolist() == want
    # one argmax-only row inside a batch whose other row samples the full vocabulary
    sps2 = [Sampling(temperature=0.0), Sampling(top_k=20, temperature=0.9)]
    rows2 = ops.pack_rows(sps2, np.array([0.0, 0.3]), V, argmax_vv=[vv, None]).to(dev)
    o2 = ops.sample_rows(xt[:2], rows2)
    torch.cuda.synchronize()
    assert int(o2.ids[0].item()) == want[0]


def test_host_state_follows_the_device_pool(dev):
    """sample_rows_for keeps each request's state in a device pool: the host fields read back what the device
    advanced (rng, history, counts, produced); a host-side change (accept of a token, a new rng) is taken over by
    the next device step; a Sampler that is dropped frees its slot."""
    import gc

    from volundr_amd import sampler as SM

    rng = np.random.default_rng(99)
    sps = [Sampling(top_k=20, temperature=0.9, repetition_penalty=1.4, seed=61),
           Sampling(top_p=0.8, presence_penalty=0.7, seed=62)]
    ss = [Sampler(sp, vocab_valid=VV) for sp in sps]
    oracle = [OracleRequest(sp) for sp in sps]

    def run(nsteps, label):
        for step in range(nsteps):
            x = _logits(rng, len(ss))
            toks = sample_rows_for(torch.from_numpy(x).to(dev), ss)
            for r in range(len(ss)):
                res, nxt = oracle[r].step(x[r])
                _check(f"{label} step {step} row {r}", toks[r], ss[r].last_logprob, res)
                oracle[r].accept(toks[r], res, nxt)

    run(3, "first")
    for r, s in enumerate(ss):  # host reads pull the device state
        assert s.rng == oracle[r].rng and list(s.history) == oracle[r].gen and s.produced == 3
        assert sum(s.counts.values()) == 3
    # host-side changes: an accepted token and a new generator state
    ss[0].accept(7)
    oracle[0].gen.append(7)
    ss[1].rng = oracle[1].rng = 0xDEADBEEF1234567
    run(3, "after host changes")
    for r, s in enumerate(ss):
        assert s.rng == oracle[r].rng and list(s.history) == oracle[r].gen
    pool = ss[0]._vs[0]
    live = len(pool.order)
    s = None  # noqa: F841  (the loop variable held the last sampler)
    del ss[1]
    gc.collect()
    oracle.pop(1)
    run(1, "after a drop")
    assert len(pool.order) == live - 1
    assert SM._pools  # the pool is kept for later calls


def test_samplers_moving_between_pools(dev):
    """The same Samplers served from logits of two widths (two device pools) in turn: each move re-admits the
    request with its current state, and the batch's cached slots in the pool it left are not reused."""
    rng = np.random.default_rng(123)
    sps = [Sampling(top_k=30, repetition_penalty=1.3, seed=91), Sampling(top_p=0.9, frequency_penalty=0.3, seed=92)]
    ss = [Sampler(sp, vocab_valid=VV) for sp in sps]
    oracle = [OracleRequest(sp) for sp in sps]
    for step, width in enumerate((V, V, V - 8, V, V - 8, V - 8, V)):
        x = np.ascontiguousarray(_logits(rng, len(ss))[:, :width])
        toks = sample_rows_for(torch.from_numpy(x).to(dev), ss)
        for r in range(len(ss)):
            res, nxt = oracle[r].step(x[r])
            _check(f"step {step} width {width} row {r}", toks[r], ss[r].last_logprob, res)
            oracle[r].accept(toks[r], res, nxt)
    for r, s in enumerate(ss):
        assert s.rng == oracle[r].rng and list(s.history) == oracle[r].gen and s.produced == 7
