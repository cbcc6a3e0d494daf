"""Pins the NumPy oracle (oracle/) with checks that do not restate its formulas: hand-computed values, a brute-force
pure-Python sampler (tests/brute.py), special cases fixed by the definition, the reference's tie-order hand case
and the published xorshift64* recurrence. CPU only."""
import math

import numpy as np
import pytest

from brute import brute_sample, f32
from oracle import sampler_ref as S
from oracle import verify_ref as VR
from volundr_amd.session import Sampling


def P(**kw):
    return Sampling(**kw)


# ---------------------------------------------------------------- penalties (sampler.py:113-122), hand values
def test_repetition_penalty_hand_values():
    x = np.array([2.0, -2.0, 0.0, 5.0], np.float32)
    out = S.preprocess(x, P(repetition_penalty=1.25), {0: 1, 1: 3, 2: 1})
    assert out[0] == np.float32(1.6) and out[1] == np.float32(-2.5)
    assert out[2] == 0.0 and out[3] == 5.0          # zero: v*r = 0; untouched id unchanged


def test_frequency_presence_hand_values():
    x = np.array([1.0, 1.0, 1.0], np.float32)
    out = S.preprocess(x, P(frequency_penalty=0.5, presence_penalty=0.25), {0: 2, 2: 1})
    assert out[0] == np.float32(1.0 - (0.5 * 2 + 0.25)) and out[1] == 1.0 and out[2] == np.float32(0.25)


def test_penalty_float32_rounding_no_fma():
    # 0.1f*3 + 0.2f rounded twice in float32 (no fused multiply-add), then subtracted in float32
    x = np.array([1.0], np.float32)
    out = S.preprocess(x, P(frequency_penalty=0.1, presence_penalty=0.2), {0: 3})
    fc = f32(f32(0.1) * 3.0)
    assert out[0] == np.float32(f32(1.0 - f32(fc + f32(0.2))))


def test_ids_at_or_above_V_ignored():
    x = np.zeros(4, np.float32)
    out = S.preprocess(x, P(presence_penalty=1.0, logit_bias=[(7, 3.0)], suppress_tokens=[9]), {5: 1, 1: 1})
    assert out.tolist() == [0.0, -1.0, 0.0, 0.0]


def test_bias_then_suppress_then_stop():
    x = np.zeros(5, np.float32)
    sp = P(logit_bias=[(1, 2.0), (1, 0.5), (2, 1.0)], suppress_tokens=[2], stop_token_ids=[3], min_new_tokens=2)
    out = S.preprocess(x, sp, {}, produced=1)
    assert out[1] == 2.5 and out[2] == -np.inf and out[3] == -np.inf
    out = S.preprocess(x, sp, {}, produced=2)          # stop mask off once min_new_tokens reached
    assert out[3] == 0.0


# ---------------------------------------------------------------- special cases fixed by the definition
def test_u_zero_gives_top_token():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(300).astype(np.float32)
    assert S.sample(x, P(temperature=0.8), 0.0).token == int(np.argmax(x))


def test_u_near_one_gives_last_kept():
    x = np.array([3.0, 2.0, 1.0, 0.0], np.float32)
    r = S.sample(x, P(top_k=3), 1.0 - 1e-12)
    assert r.token == 2 and r.keep == 3


def test_top_k_one_is_argmax_and_greedy():
    x = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    assert S.sample(x, P(top_k=1), 0.7).token == 1 and S.sample(x, P(top_k=1), 0.7).kind == "greedy"
    assert S.sample(x, P(temperature=0.0), 0.3).token == 1


def test_tiny_top_p_keeps_top_token():
    x = np.array([0.0, 1.0, 0.5], np.float32)
    r = S.sample(x, P(top_p=1e-9), 0.99)
    assert r.token == 1 and r.keep == 1 and r.logprob == 0.0


def test_all_neg_inf_is_argmax_zero():
    x = np.full(8, -np.inf, np.float32)
    r = S.sample(x, P(), 0.5)
    assert r.token == 0 and r.kind == "nofinite"


def test_nan_wins_greedy_like_np_argmax():
    x = np.array([1.0, np.nan, 5.0, np.nan], np.float32)
    assert S.sample(x, P(top_k=1), 0.0).token == 1


def test_reference_tie_order_hand_case():
    # volundr-mlx/tests/test_volundr.py:159-161: [1,3,3,2,3,-inf,3,-1], k=3 -> {1,2,4}
    x = np.array([1, 3, 3, 2, 3, -np.inf, 3, -1], np.float32)
    r = S.sample(x, P(top_k=3, temperature=1.0), 0.999999)
    assert r.keep == 3 and r.topk_tie
    # the three kept tokens carry equal mass 1/3: draws at 0.2/0.5/0.8 hit 1, 2, 4 in index order
    assert [S.sample(x, P(top_k=3), u).token for u in (0.2, 0.5, 0.8)] == [1, 2, 4]


def test_exp40_filter_closed_form():
    # > 4096 finite tokens, no top-k: tokens with x/t < max/t - 40 are dropped (sampler.py:137-139)
    x = np.zeros(5000, np.float32)
    x[0] = 50.0
    x[1] = 10.0 + 1e-3       # kept: 10.001 >= 50 - 40
    x[2] = 9.999             # dropped
    r = S.sample(x, P(), 0.5)
    assert r.keep == 2       # token 0, token 1 (everything else sits at 0 < 10)


def test_logprob_closed_form():
    x = np.array([1.0, 0.0, -1.0], np.float32)
    r = S.sample(x, P(), 0.9)
    z = math.exp(1) + 1 + math.exp(-1)
    want = {0: 1 - math.log(z), 1: -math.log(z), 2: -1 - math.log(z)}[r.token]
    assert abs(r.logprob - want) < 1e-12


def test_min_p_cut():
    x = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    r = S.sample(x, P(min_p=0.5), 0.999)  # p/p0 = 1, .6, .3, .1 -> keep 2
    assert r.keep == 2 and r.token == 1


# ---------------------------------------------------------------- brute force on tiny vocabularies
@pytest.mark.parametrize("seed", range(40))
def test_oracle_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(2, 60))
    x = (rng.standard_normal(V) * rng.choice([0.1, 1, 4])).astype(np.float32)
    if rng.random() < 0.3:
        x[rng.integers(0, V, size=3)] = np.float32(rng.choice([-np.inf, 1.5]))  # ties / masked entries
    sp = P(temperature=float(rng.choice([0.5, 1.0, 1.7])), top_k=int(rng.choice([0, 1, 2, 5, 100])),
           top_p=float(rng.choice([1.0, 0.9, 0.5])), min_p=float(rng.choice([0.0, 0.1])),
           repetition_penalty=float(rng.choice([1.0, 1.3])), presence_penalty=float(rng.choice([0.0, 0.4])),
           frequency_penalty=float(rng.choice([0.0, 0.2])),
           logit_bias=[(int(rng.integers(0, V)), 0.7)] if rng.random() < 0.5 else [],
           suppress_tokens=[int(rng.integers(0, V))] if rng.random() < 0.3 else [])
    counts = S.counts_from_history(rng.integers(0, V, size=int(rng.integers(0, 10))))
    for u in rng.random(5):
        r = S.sample(x, sp, float(u), counts)
        if r.draw_boundary or r.topp_boundary:
            continue
        assert r.token == brute_sample(x, sp, float(u), counts)


# ---------------------------------------------------------------- xorshift64* (Vigna 2016)
@pytest.mark.parametrize("seed", range(10))
def test_plain_restatement_matches_oracle(seed):
    """sample_plain (the reference's argpartition form, timed by bench.py's CPU baseline) picks the oracle's token
    on random rows without ties at the k-th position, for every class of row."""
    from volundr_amd import synth

    d = synth.c3(seed=seed, V=20000, H=512) if seed % 2 else synth.c5(seed=seed, V=20000, B=4, H=2048)
    for i in range(d["logits"].shape[0]):
        c = S.counts_from_history(d["hists"][i])
        r = S.sample(d["logits"][i], d["params"][i], float(d["u"][i]), c)
        if r.topk_tie:
            continue
        assert S.sample_plain(d["logits"][i], d["params"][i], float(d["u"][i]), c) == r.token


def test_xorshift64star_known_sequence():
    # state recurrence x ^= x>>12; x ^= x<<25; x ^= x>>27; output x*0x2545F4914F6CDD1D; seed 1 -> first state
    st = S.seed_state(1)
    st, u = S.xorshift64s_next(st)
    x = 1
    x ^= x >> 12
    x ^= (x << 25) & S.MASK
    x ^= x >> 27
    assert st == x == 0x2000001
    assert u == (((0x2000001 * 0x2545F4914F6CDD1D) & S.MASK) >> 11) / 2.0**53
    # the seed is forced odd and masked to 64 bits
    assert S.seed_state(2) == 3 and S.seed_state(-1) == S.MASK


def test_sampler_shim_uniform_matches_oracle():
    from volundr_amd.sampler import Sampler

    s = Sampler(P(seed=12345))
    st = S.seed_state(12345)
    for _ in range(100):
        st, u = S.xorshift64s_next(st)
        assert s.uniform() == u


# ---------------------------------------------------------------- verify oracle
def test_verify_argmax_first_max_and_accept():
    x = np.zeros((1, 4, 6), np.float32)
    x[0, 0, [2, 4]] = 5.0         # exact tie: lower index
    x[0, 1, 1] = 3.0
    x[0, 2, 5] = 1.0
    x[0, 3, 0] = 2.0
    tok, acc, lp = VR.verify(x, np.array([[2, 1, 4]], np.int32), 6)
    assert tok.tolist() == [[2, 1, 5, 0]] and acc.tolist() == [2]
    tok, acc, _ = VR.verify(x, np.array([[2, 1, 5]], np.int32), 6)
    assert acc.tolist() == [3]                                      # all match -> T-1
    assert VR.verify(x, np.array([[0, 1, 5]], np.int32), 6)[1].tolist() == [0]  # first mismatch -> 0
    want = 5.0 - math.log(2 * math.exp(5.0) + 4)
    assert abs(lp[0, 0] - want) < 1e-12
    # vocab_valid excludes the tail
    tok, _, _ = VR.verify(x, np.array([[0, 0, 0]], np.int32), 4)
    assert tok[0, 0] == 2 and tok[0, 2] == 0


def test_verify_python_loop_brute():
    rng = np.random.default_rng(3)
    x = rng.integers(-3, 4, size=(2, 5, 40)).astype(np.float32)  # many ties
    tok, _, _ = VR.verify(x, np.zeros((2, 4), np.int32), 37)
    for b in range(2):
        for t in range(5):
            best = 0
            for i in range(37):
                if x[b, t, i] > x[b, t, best]:
                    best = i
            assert tok[b, t] == best


def test_emitted_hand_cases():
    """specdec.py:335-336 / scheduler.py:465-470: n = nacc + 1, emitted = inp[1:n] + [tok[n-1]], with inp[1:] the
    drafts. Hand cases for the oracle's and the product's emitted."""
    from volundr_amd.ops import emitted as em_product
    drafts = [11, 12, 13, 14]
    tok = [11, 12, 13, 14, 99]
    for em in (VR.emitted, em_product):
        assert em(drafts, tok, 4) == [11, 12, 13, 14, 99]           # all drafts accepted -> drafts + [tok[T-1]]
        assert em(drafts, [7, 12, 13, 14, 99], 0) == [7]            # first mismatch -> [tok[0]]
        assert em(drafts, [11, 12, 5, 14, 99], 2) == [11, 12, 5]    # nacc = k -> drafts[:k] + [tok[k]]
        assert em([], [42], 0) == [42]                              # T = 1: the bonus token only
        assert em(np.array(drafts, np.int32), np.array(tok, np.int32), 3) == [11, 12, 13, 14]


def test_emitted_is_the_argmax_prefix():
    """What the definition fixes: the nacc accepted drafts equal tok[:nacc], so the emitted tokens are exactly
    tok[:nacc+1] of the verify argmax; length nacc + 1. Checked on random blocks with planted accept lengths."""
    from volundr_amd.ops import emitted as em_product
    rng = np.random.default_rng(7)
    for trial in range(50):
        B, T, V = 3, int(rng.integers(1, 18)), 50
        x = rng.integers(-3, 4, size=(B, T, V)).astype(np.float32)
        tok, _, _ = VR.verify(x, np.zeros((B, T - 1), np.int32), V)
        drafts = tok[:, :-1].copy()
        for b in range(B):
            L = int(rng.integers(0, T))
            if L < T - 1:
                drafts[b, L] = (drafts[b, L] + 1) % V
        tok, acc, _ = VR.verify(x, drafts, V)
        for b in range(B):
            n = int(acc[b])
            want = [int(t) for t in tok[b, :n + 1]]
            assert VR.emitted(drafts[b], tok[b], n) == want
            assert em_product(drafts[b].tolist(), tok[b].tolist(), n) == want


def test_bf16_bits_roundtrip():
    from volundr_amd import synth

    x = np.array([1.0, -2.5, 3.1415926, 1e-3], np.float32)
    b = synth.f32_to_bf16_bits(x)
    assert np.allclose(synth.bf16_bits_to_f32(b), x, rtol=2**-8)
    assert VR.to_f32(b).tolist() == synth.bf16_bits_to_f32(b).tolist()


# ---------------------------------------------------------------- build-defined outputs the GPU tests rely on
def test_logsoftmax_greedy_closed_form():
    # greedy row: logprob = x[j] - log(sum exp(x)) over the finite entries
    x = np.array([1.0, 0.0, -1.0], np.float32)
    r = S.sample(x, P(top_k=1), 0.5)
    assert r.kind == "greedy" and r.token == 0
    assert abs(r.logprob - (1.0 - math.log(math.e + 1.0 + 1.0 / math.e))) < 1e-12
    # -inf entries carry no mass; a NaN-free row with infinities keeps the finite normaliser
    x = np.array([-np.inf, 2.0, -np.inf, 2.0, 0.0], np.float32)
    r = S.sample(x, P(temperature=0.0), 0.5)
    assert r.token == 1 and abs(r.logprob - (2.0 - math.log(2 * math.exp(2.0) + 1.0))) < 1e-12
    # a non-finite choice has logprob 0 (no finite logit at all, or +inf winning)
    assert S.sample(np.full(4, -np.inf, np.float32), P(), 0.5).logprob == 0.0
    assert S.sample(np.array([0.0, np.inf], np.float32), P(top_k=1), 0.5).logprob == 0.0


def _three_way():
    x = np.log(np.array([0.5, 0.3, 0.2])).astype(np.float32)
    xs = x - x[0]
    pr = np.exp(xs.astype(np.float64))
    return x, np.cumsum(pr / pr.sum())


@pytest.mark.parametrize("d,flag", [(1e-7, True), (-1e-7, True), (1e-5, False), (-1e-5, False)])
def test_draw_boundary_predicate(d, flag):
    # the draw u*z (z = 1 without top-p) placed next to the first CDF step cs[0]
    x, cs = _three_way()
    r = S.sample(x, P(), float(cs[0] + d))
    assert r.draw_boundary == flag
    assert r.token == (0 if d < 0 else 1)          # first cumsum >= u*z
    r = S.sample(x, P(), float(cs[1] + d))         # the second step
    assert r.draw_boundary == flag and r.token == (1 if d < 0 else 2)


@pytest.mark.parametrize("d,flag", [(1e-7, True), (-1e-7, True), (1e-5, False), (-1e-5, False)])
def test_topp_boundary_predicate(d, flag):
    x, cs = _three_way()
    r = S.sample(x, P(top_p=float(cs[1] + d)), 0.1)
    assert r.topp_boundary == flag
    assert r.keep == (2 if d < 0 else 3)           # first cumsum >= top_p, plus one
    assert not r.draw_boundary and r.token == 0


# ---------------------------------------------------------------- Sampler.choose and the reasoning budget
def _budget_replay(prompt, gen, n, soft, start, end):
    """Actions of the product Budget (a state machine) when driven as Sampler.choose drives it."""
    from volundr_amd.sampler import Budget

    b = Budget(n, soft, prompt, start, end)
    acts = []
    for j, tok in enumerate(gen):
        acts.append(b.act(j))
        if acts[-1][0] == "force":
            tok = end
        b.accept(j, tok)
    acts.append(b.act(len(gen)))
    return acts


def test_budget_hand_cases():
    S_, E_ = 7, 8
    # open in the prompt tail, n = 4: forced at output 4, then <think> masked for good
    acts = [S.budget_action([1, 2, S_], [0] * p, 4, 0.0, S_, E_) for p in range(4)]
    assert [a[0] for a in acts] == ["none"] * 4
    assert S.budget_action([1, 2, S_], [0, 0, 0, 0], 4, 0.0, S_, E_) == ("force", E_)
    assert S.budget_action([1, 2, S_], [0, 0, 0, 0, E_], 4, 0.0, S_, E_) == ("bias", [(S_, -np.inf)])
    # closed inside the prompt tail: idle until a generated <think>; soft bias from 80% of n on
    assert S.budget_action([S_, E_], [0] * 20, 10, 1.5, S_, E_) == ("none", None)
    # origin 1 (the token after the generated <think>): k zeros after it are k tokens spent
    assert S.budget_action([S_, E_], [S_] + [0] * 7, 10, 1.5, S_, E_) == ("none", None)         # 7 < 8
    assert S.budget_action([S_, E_], [S_] + [0] * 8, 10, 1.5, S_, E_) == ("bias", [(E_, 1.5)])  # 8 >= 0.8 * 10

    # closed by the model before the budget: nothing more, ever
    assert S.budget_action([S_], [0, E_, 0, 0, 0, 0, 0], 4, 1.0, S_, E_) == ("none", None)
    # a <think> older than 16 prompt tokens does not count
    assert S.budget_action([S_] + [0] * 16, [0] * 30, 4, 0.0, S_, E_) == ("none", None)


def test_budget_spot_values_of_the_state_machine():
    from volundr_amd.sampler import Budget

    b = Budget(10, 1.5, [7, 8], 7, 8)
    assert b.open is None and not b.closed and b.act(20) == ("none", None)
    b.accept(0, 7)
    assert b.open == 1 and b.act(5) == ("none", None) and b.act(9) == ("bias", [(8, 1.5)])
    assert b.act(11) == ("force", 8) and b.forced and b.closed and b.open is None


@pytest.mark.parametrize("seed", range(60))
def test_budget_state_machine_matches_record_derivation(seed):
    """The product's state-machine Budget and the oracle's whole-record derivation agree on every step of random
    token streams rich in <think>/<\\think> tokens."""
    rng = np.random.default_rng(seed)
    S_, E_ = 7, 8
    prompt = list(rng.choice([0, 1, S_, E_], size=int(rng.integers(0, 24)), p=[0.5, 0.2, 0.2, 0.1]))
    n = int(rng.integers(1, 12))
    soft = float(rng.choice([0.0, 2.0]))
    gen = []
    acts = []
    from volundr_amd.sampler import Budget

    b = Budget(n, soft, prompt, S_, E_)
    for j in range(40):
        a = b.act(j)
        want = S.budget_action(prompt, gen, n, soft, S_, E_)
        assert a == want, f"step {j}: {a} vs {want}"
        tok = E_ if a[0] == "force" else int(rng.choice([0, 1, S_, E_], p=[0.6, 0.2, 0.1, 0.1]))
        b.accept(j, tok)
        gen.append(tok)
        acts.append(a)


def test_choose_routes():
    V, vv = 12, 10
    x = np.zeros(V, np.float32)
    x[11] = 9.0                      # a padding column holds the row maximum
    x[3] = 2.0
    # needs no logits: argmax over [:vv] with its logprob over [:vv]
    r = S.choose(x, P(temperature=0.0), vv, 0.5, [])
    assert r.kind == "argmax" and r.token == 3
    assert abs(r.logprob - (2.0 - math.log(math.exp(2.0) + 9))) < 1e-12
    # greedy with a penalty needs the sampler: argmax over the full row (sampler.py:127-128 has no vv slice)
    r = S.choose(x, P(temperature=0.0, repetition_penalty=1.1), vv, 0.5, [])
    assert r.kind == "greedy" and r.token == 11
    # the stop mask makes an argmax-only request a sampler row while produced < min_new_tokens
    sp = P(top_k=1, min_new_tokens=2, stop_token_ids=[11])
    assert S.choose(x, sp, vv, 0.5, [0]).kind == "greedy" and S.choose(x, sp, vv, 0.5, [0]).token == 3
    assert S.choose(x, sp, vv, 0.5, [0, 0]).kind == "argmax"
    # budget force and bias
    sp = P(reasoning_budget=10, reasoning_budget_soft_bias=50.0, temperature=0.0)
    r = S.choose(x, sp, vv, 0.5, [5] + [0] * 10, prompt=[], think_ids=(5, 6))
    assert r.kind == "force" and r.token == 6
    r = S.choose(x, sp, vv, 0.5, [5] + [0] * 7, prompt=[], think_ids=(5, 6))    # 7 spent: no bias yet
    assert r.kind == "argmax" and r.token == 3
    r = S.choose(x, sp, vv, 0.5, [5] + [0] * 8, prompt=[], think_ids=(5, 6))    # 8 >= 0.8*10: +50 on <\think>
    assert r.kind == "greedy" and r.token == 6
