"""GPU parity of vs_sample_batch (through the C ABI via volundr_amd.ops) against the NumPy oracle."""
import numpy as np
import pytest
import torch

from oracle import sampler_ref as S
from parity import check_sample
from volundr_amd import sample_batch, synth
from volundr_amd._lib import OUT_COOP, OUT_GATHER, OUT_GREEDY, OUT_NOFINITE
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu


def run(dev, x, params, u, hists=None, produced=None, dtype=torch.float32, label="", max_excused=None, pairs=False):
    xt = torch.from_numpy(x).to(dev).to(dtype)
    xr = xt.float().cpu().numpy()  # the oracle sees exactly the widened values the kernel reads
    print(f"[{label}] B={x.shape[0]} V={x.shape[1]} dtype={dtype} pairs={pairs}", flush=True)
    out = sample_batch(xt, params, u, hists, produced, hist_pairs=pairs)
    torch.cuda.synchronize()
    refs = [S.sample(xr[i], params[i], float(u[i]), S.counts_from_history(hists[i]) if hists is not None else {},
                     0 if produced is None else produced[i]) for i in range(x.shape[0])]
    nb = check_sample(out, refs, label, max_excused)
    return out, refs, nb


def rand_params(rng, n, V):
    ps = []
    for _ in range(n):
        ps.append(Sampling(temperature=float(rng.choice([0.0, 0.5, 0.9, 1.0, 1.6])),
                           top_k=int(rng.choice([0, 1, 2, 7, 20, 50, 300])),
                           top_p=float(rng.choice([1.0, 0.95, 0.8, 0.3])),
                           min_p=float(rng.choice([0.0, 0.0, 0.05])),
                           repetition_penalty=float(rng.choice([1.0, 1.1, 1.3])),
                           presence_penalty=float(rng.choice([0.0, 0.3])),
                           frequency_penalty=float(rng.choice([0.0, 0.1]))))
    return ps


# 12 rows: 21 workgroups per row (top-k lists merged by heads); 24 rows: 10 (merged by rank)
@pytest.mark.parametrize("V", [1000, 5003, 40000])
@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("B", [12, 24])
def test_random_mix(dev, V, seed, B):
    rng = np.random.default_rng(100 + seed + B)
    x = (rng.standard_normal((B, V)) * rng.choice([0.2, 1.0, 3.0], size=(B, 1))).astype(np.float32)
    ps = rand_params(rng, B, V)
    hists = [rng.integers(0, V, size=int(rng.integers(0, 300))) for _ in range(B)]
    run(dev, x, ps, rng.random(B), hists, label=f"mix V{V} s{seed} B{B}")


@pytest.mark.parametrize("k", [50, 256])
def test_topk_concentrated_lists(dev, k):
    """The row's largest logits all sit in one workgroup's chunk: that list alone holds the top k, so the merge keeps
    many survivors (and for k=256 takes its radix-select path)."""
    rng = np.random.default_rng(41 + k)
    B, V = 16, 163840
    x = rng.standard_normal((B, V)).astype(np.float32)
    x[:, :600] += 20.0 + rng.random((B, 600)).astype(np.float32)
    x[1::2, V - 700:] += 19.0  # odd rows: a second dense block at the far end
    ps = [Sampling(temperature=1.0, top_k=k, top_p=float(rng.choice([1.0, 0.9]))) for _ in range(B)]
    run(dev, x, ps, rng.random(B), label=f"concentrated k{k}")


@pytest.mark.parametrize("nb,rest", [(60, -100.0), (1500, -100.0), (600, 0.0)])
@pytest.mark.parametrize("t", [0.7, 1.3, 0.31])
def test_exp40_filter_boundary(dev, nb, rest, t):
    """Whole-vocabulary rows (V > 4096, no top-k): many logits sit within a few ulps of the cut
    x / t >= max / t - 40 (sampler.py:137-139), so the kept set must be decided exactly as float32 division does."""
    V = 20000
    B = 4
    x = np.full((B, V), rest, np.float32)
    rng = np.random.default_rng(int(nb + 10 * t))
    if rest == 0.0:
        x += rng.standard_normal((B, V)).astype(np.float32)
    m = np.float32(10.0)
    cut = np.float32(m / np.float32(t) - np.float32(40.0)) * np.float32(t)
    for b in range(B):
        x[b, 7 + b] = m
        pos = rng.choice(np.arange(20, V), size=nb, replace=False)
        steps = np.arange(nb) - nb // 2
        x[b, pos] = (cut.view(np.int32) + np.sign(cut) * steps).astype(np.int32).view(np.float32)
    ps = [Sampling(temperature=t, top_k=0, top_p=1.0) for _ in range(B)]
    out, refs, _ = run(dev, x, ps, rng.random(B), label=f"exp40 nb{nb} t{t}")
    for r in refs:
        assert r.keep > 1


def test_exp40_near_misses_in_many_lanes(dev):
    """Hundreds of logits a few ulps below the exp(-40) cut in one chunk (many lanes pass the coarse lane bound)
    while only a few logits are kept: the small kept-set path must still gather every kept logit."""
    V, B, t = 20000, 4, 0.7
    x = np.full((B, V), -100.0, np.float32)
    m = np.float32(10.0)
    cut = np.float32(m / np.float32(t) - np.float32(40.0)) * np.float32(t)
    ci = cut.view(np.int32)
    rng = np.random.default_rng(5)
    for b in range(B):
        x[b, 3] = m
        below = (ci + np.sign(cut) * -rng.integers(1, 6, size=400)).astype(np.int32).view(np.float32)
        x[b, 20:420] = below
        x[b, 500 + 37 * np.arange(30)] = (ci + np.sign(cut) * rng.integers(0, 5, size=30)).astype(np.int32).view(np.float32)
    ps = [Sampling(temperature=t, top_k=0, top_p=float(p)) for p in (1.0, 0.9, 1.0, 0.5)]
    out, refs, _ = run(dev, x, ps, rng.random(B), label="exp40 near misses")
    assert refs[0].keep == 31 and refs[2].keep == 31
    assert all(int(f) & OUT_GATHER for f in out.flags.cpu().numpy())  # the small kept-set path


def test_bf16_rows(dev):
    rng = np.random.default_rng(7)
    B, V = 6, 30000
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    ps = rand_params(rng, B, V)
    run(dev, x, ps, rng.random(B), dtype=torch.bfloat16, label="bf16")  # many exact ties after rounding


@pytest.mark.parametrize("V", [30000, 163840])
def test_f16_rows(dev, V):
    rng = np.random.default_rng(8)
    B = 6
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    ps = rand_params(rng, B, V)
    hists = [rng.integers(0, V, size=int(rng.integers(0, 500))) for _ in range(B)]
    run(dev, x, ps, rng.random(B), hists, dtype=torch.float16, label=f"f16 V{V}")


def test_coop_path_near_flat(dev):
    rng = np.random.default_rng(11)
    B, V = 4, 50000
    x = (rng.standard_normal((B, V)) * 0.1).astype(np.float32)
    ps = [Sampling(top_p=0.95), Sampling(top_p=1.0), Sampling(top_p=0.5, min_p=0.9), Sampling(top_k=3000, top_p=0.9)]
    out, refs, _ = run(dev, x, ps, rng.random(B), label="coop")
    fl = out.flags.cpu().numpy()
    assert all(f & OUT_COOP for f in fl)


@pytest.mark.parametrize("sigma,top_p", [(2.0, 0.9), (4.0, 1.0), (1.0, 0.5), (6.0, 0.99)])
def test_binned_path_medium_sets(dev, sigma, top_p):
    # kept sets of a few hundred to a few thousand tokens: the two-level value-bin path
    rng = np.random.default_rng(int(sigma * 10) + int(top_p * 100))
    B, V = 4, 60000
    x = (rng.standard_normal((B, V)) * sigma).astype(np.float32)
    ps = [Sampling(top_p=top_p, temperature=float(tt)) for tt in (0.7, 1.0, 1.3, 2.0)]
    out, refs, _ = run(dev, x, ps, rng.random(B), label=f"binned s{sigma} p{top_p}")
    assert all(f & OUT_COOP for f in out.flags.cpu().numpy() if not f & OUT_GATHER)


def test_binned_path_many_draws(dev):
    # one row, many draws: exercises the speculative draw-bin ranges across the CDF
    rng = np.random.default_rng(21)
    V = 80000
    x = (rng.standard_normal((1, V)) * 0.3).astype(np.float32)
    xs = np.repeat(x, 16, axis=0)
    ps = [Sampling(top_p=0.9)] * 16
    run(dev, xs, ps, np.linspace(0.0, 0.999999, 16), label="binned draws")


def test_near_flat_full_size_extreme_draws(dev):
    """C5's shape at unit temperature (the dense value-bin instance without division) and at t = 0.8, with draws at
    both ends of the CDF: the draw's coarse bins are the top one (digit 255, beside the not-kept id 0xFFFF) and the
    last ones, with and without a top-p cut."""
    rng = np.random.default_rng(23)
    V = 163840
    x = (rng.standard_normal((1, V)) * 0.1).astype(np.float32)
    xs = np.repeat(x, 8, axis=0)
    ps = [Sampling(temperature=1.0, top_p=0.95)] * 3 + [Sampling(temperature=1.0, top_p=1.0)] * 3 + \
         [Sampling(temperature=0.8, top_p=0.95)] * 2
    us = [0.0, 1e-7, 0.9999999, 0.0, 0.5, 0.9999999, 1e-7, 0.9999999]
    run(dev, xs, ps, us, label="near-flat extremes")


def test_ties_fall_back_to_radix(dev):
    # bf16 near-flat logits: a few hundred distinct values for 100k tokens, so value bins hold long runs of ties
    rng = np.random.default_rng(22)
    B, V = 3, 100000
    x = (rng.standard_normal((B, V)) * 0.05).astype(np.float32)
    ps = [Sampling(top_p=0.95), Sampling(top_p=1.0), Sampling(top_p=0.3, temperature=0.5)]
    run(dev, x, ps, rng.random(B), dtype=torch.bfloat16, label="bf16 ties")


def test_gather_path(dev):
    rng = np.random.default_rng(12)
    B, V = 3, 20000
    x = (rng.standard_normal((B, V)) * 30).astype(np.float32)  # exp(-40) filter keeps a few dozen
    ps = [Sampling(top_k=0, top_p=p, temperature=1.0) for p in (1.0, 0.9, 0.5)]
    out, refs, _ = run(dev, x, ps, rng.random(B), label="gather")
    assert all(f & OUT_GATHER for f in out.flags.cpu().numpy())


def test_small_n_no_filter(dev):
    # <= 4096 finite tokens: no exp(-40) filter (sampler.py:137), kept = all finite (gather or coop)
    rng = np.random.default_rng(13)
    V = 4000
    x = (rng.standard_normal((2, V)) * 0.5).astype(np.float32)
    x[1, 1500:] = -np.inf
    run(dev, x, [Sampling(top_p=0.99), Sampling()], rng.random(2), label="n<=4096")


def test_edits(dev):
    rng = np.random.default_rng(14)
    B, V = 5, 9000
    x = (rng.standard_normal((B, V))).astype(np.float32)
    ps = [Sampling(logit_bias=[(5, 20.0), (5, 1.5), (V + 3, 1.0)], top_k=10),
          Sampling(suppress_tokens=[int(np.argmax(x[1]))], top_k=5, repetition_penalty=0.5),
          Sampling(stop_token_ids=[int(np.argmax(x[2]))], min_new_tokens=3, top_k=1),
          Sampling(logit_bias=[(-1, 30.0)], top_p=0.7),
          Sampling(frequency_penalty=0.7, presence_penalty=-0.2, repetition_penalty=1.4, top_k=0, top_p=0.9)]
    hists = [None, [int(np.argmax(x[1]))] * 3, [], [1, 2, 3], list(np.argsort(-x[4])[:40]) * 3]
    out, refs, _ = run(dev, x, ps, rng.random(B), hists, produced=[0, 0, 1, 0, 0], label="edits")
    assert out.ids[0].item() == 5 and out.ids[3].item() == V - 1


@pytest.mark.parametrize("V", [40000, 163840])
def test_topk_edits_move_lane_maxima(dev, V):
    """Top-k rows whose edits move the largest logits: heavy penalties on the row's top tokens (the bound taken
    before the edits is then too high and the kernel must redo it) and edits that raise logits (repetition penalty
    below 1, negative penalties, positive biases)."""
    rng = np.random.default_rng(V + 5)
    B = 8
    x = rng.standard_normal((B, V)).astype(np.float32) * 2.0
    order = np.argsort(-x, axis=1)
    ps, hists = [], []
    for b in range(B):
        k = [5, 20, 50, 200][b % 4]
        if b < 4:  # push the top tokens down hard
            ps.append(Sampling(top_k=k, repetition_penalty=3.0, frequency_penalty=2.0, presence_penalty=4.0))
            hists.append(list(order[b, :3 * k]) * 2)
        else:  # raise low tokens above the rest
            ps.append(Sampling(top_k=k, repetition_penalty=0.25, presence_penalty=-6.0, frequency_penalty=-1.0,
                               logit_bias=[(int(order[b, -1 - j]), 40.0) for j in range(3)]))
            hists.append(list(order[b, V // 2:V // 2 + k]) + list(rng.integers(0, V, size=50)))
    run(dev, x, ps, rng.random(B), hists, label=f"topk edits V{V}")


def test_long_and_unaligned_histories(dev):
    # histories beyond the in-register prefetch (32768 tokens) and rows whose history starts unaligned
    rng = np.random.default_rng(23)
    B, V = 3, 20000
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    ps = [Sampling(top_k=30, repetition_penalty=1.3, frequency_penalty=0.05, presence_penalty=0.2)] * B
    hists = [rng.integers(0, V, size=40001), rng.integers(0, 300, size=7), rng.integers(0, V, size=32771)]
    run(dev, x, ps, rng.random(B), hists, label="long histories")


def test_nonfinite_rows(dev):
    V = 3000
    x = np.zeros((5, V), np.float32)
    x[0, :] = -np.inf
    x[1, :] = -np.inf
    x[1, 7] = np.inf
    x[2, 100] = np.nan
    x[2, 50] = 4.0
    x[3, :] = np.nan
    x[4, :] = -np.inf
    x[4, 2999] = 1.0
    ps = [Sampling(), Sampling(top_k=5), Sampling(top_k=1), Sampling(top_k=0), Sampling(top_p=0.5)]
    out, refs, _ = run(dev, x, ps, [0.3] * 5, label="nonfinite")
    fl = out.flags.cpu().numpy()
    assert fl[0] & OUT_NOFINITE and fl[1] & OUT_NOFINITE and fl[2] & OUT_GREEDY
    assert out.ids.cpu().tolist() == [0, 7, 100, 0, 2999]


def test_full_rows_with_masked_logits(dev):
    """FULL-class rows over the whole vocabulary with -inf scattered through every workgroup's chunk (masked
    tokens): lanes holding a non-finite logit take the exact statistics loop, the others the three-input one."""
    V = 163840
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((3, V)) * 2).astype(np.float32)
    x[0, ::7] = -np.inf
    x[1, 100000:] = -np.inf
    x[2, 1::3] = -np.inf
    x[2, 5] = np.inf
    ps = [Sampling(temperature=0.8, top_p=0.9), Sampling(top_p=0.95), Sampling(temperature=1.0, top_p=0.7)]
    run(dev, x, ps, [0.25, 0.6, 0.9], label="masked full rows")


def test_signed_zero_and_ties(dev):
    V = 600
    x = np.zeros((3, V), np.float32)
    x[:, 10] = -0.0
    x[0, 20:30] = 2.0
    x[1, ::2] = -0.0
    ps = [Sampling(top_k=1), Sampling(top_k=4), Sampling(top_k=7, temperature=0.5)]
    out, refs, nb = run(dev, x, ps, [0.1, 0.99, 0.5], label="ties", max_excused=0)
    # every row of zeros is one tie: the kept sets are the lowest indices, the draws land on fixed positions
    assert refs[1].topk_tie and refs[2].topk_tie
    assert out.ids.cpu().tolist() == [20, 3, 3] and out.keep.cpu().tolist()[1:] == [4, 7]


@pytest.mark.parametrize("V", [8, 163840])
def test_reference_tie_hand_case(dev, V):
    """volundr-mlx/tests/test_volundr.py:159-161: [1,3,3,2,3,-inf,3,-1] with k=3 keeps {1,2,4} (ties to the lower
    index); the three kept tokens carry equal mass, so draws 0.2/0.5/0.8 land on 1, 2 and 4. At V=163840 the
    pattern sits at the start of a row of -inf and again inside a row of far lower finite logits."""
    pat = np.array([1, 3, 3, 2, 3, -np.inf, 3, -1], np.float32)
    rows = []
    for fill in ([-np.inf] if V == 8 else [-np.inf, -30.0]):
        r = np.full(V, fill, np.float32)
        r[:8] = pat
        rows += [r] * 3
    x = np.stack(rows)
    us = [0.2, 0.5, 0.8] * (len(rows) // 3)
    out, refs, _ = run(dev, x, [Sampling(top_k=3)] * len(rows), us, label=f"tie hand case V{V}", max_excused=0)
    assert out.ids.cpu().tolist() == [1, 2, 4] * (len(rows) // 3)
    assert out.keep.cpu().tolist() == [3] * len(rows)
    assert np.allclose(out.logprobs.cpu().numpy(), -np.log(3.0), rtol=1e-6)


def test_strided_rows_and_many_launches(dev):
    rng = np.random.default_rng(15)
    B, V = 100, 2500
    big = torch.from_numpy((rng.standard_normal((B, V + 13)) * 2).astype(np.float32)).to(dev)
    xt = big[:, :V]  # ld = V + 13: scalar-load path
    ps = rand_params(rng, B, V)
    u = rng.random(B)
    out = sample_batch(xt, ps, u)
    xr = xt.cpu().numpy()
    refs = [S.sample(xr[i], ps[i], float(u[i])) for i in range(B)]
    check_sample(out, refs, "strided B100")


def test_deterministic(dev):
    d = synth.c5(seed=3, B=4, H=1000)
    xt = torch.from_numpy(d["logits"][:4]).to(dev)
    a = sample_batch(xt, d["params"][:4], d["u"][:4], d["hists"][:4])
    b = sample_batch(xt, d["params"][:4], d["u"][:4], d["hists"][:4])
    assert torch.equal(a.ids, b.ids) and torch.equal(a.keep, b.keep)


@pytest.mark.parametrize("B", [1, 2, 16])
def test_repeated_calls_identical(dev, B):
    """Every workgroup order the hardware picks gives the same bits: FULL rows through the value-bin and gather
    paths (B = 1 uses 64 workgroups per row, B = 16 uses 16), repeated 25 times against the first call."""
    g = np.random.default_rng(40 + B)
    x = torch.from_numpy((g.standard_normal((B, 163840)) * np.where(np.arange(B) % 2, 1.0, 0.1)[:, None])
                         .astype(np.float32)).to(dev)
    ps = [Sampling(temperature=0.8 if r % 3 else 1.0, top_p=(0.9, 0.95, 1.0)[r % 3]) for r in range(B)]
    u = g.random(B)
    first = sample_batch(x, ps, u)
    want = (first.ids.cpu(), first.logprobs.cpu(), first.keep.cpu(), first.flags.cpu())
    for rep in range(25):
        o = sample_batch(x, ps, u)
        got = (o.ids.cpu(), o.logprobs.cpu(), o.keep.cpu(), o.flags.cpu())
        assert all(torch.equal(a, b) for a, b in zip(got, want)), f"call {rep + 2} differs"


@pytest.mark.parametrize("name,pairs", [("c1", False), ("c3", False), ("c5", False), ("c3", True), ("c5", True)])
def test_configs_full_size(dev, name, pairs):
    d = synth.CONFIGS[name](seed=0)
    out, refs, nb = run(dev, d["logits"], d["params"], d["u"], d["hists"], label=name, max_excused=1, pairs=pairs)
    print(f"{name}: {len(refs)} rows, {nb} CDF-boundary rows", flush=True)


@pytest.mark.parametrize("V", [5003, 40000, 163840])
def test_hist_pairs_equal_raw_histories(dev, V):
    """Penalty counts as a sorted (id, count) table (VS_ROW_HIST_PAIRS) give bit-identical results to the raw
    histories they count, and match the oracle: random rows with every penalty kind, ids at and above V, tables of
    one entry, tables whose ids all lie in one workgroup's range, Zipf-dense and uniform histories."""
    rng = np.random.default_rng(V)
    B = 16
    x = (rng.standard_normal((B, V)) * rng.choice([0.2, 1.0, 3.0], size=(B, 1))).astype(np.float32)
    ps = rand_params(rng, B, V)
    ps = [Sampling(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p, min_p=p.min_p,
                   repetition_penalty=float(rng.choice([1.1, 1.3, 0.8])), presence_penalty=0.3,
                   frequency_penalty=float(rng.choice([0.0, 0.1]))) for p in ps]
    hists = []
    for r in range(B):
        kind = r % 5
        if kind == 0:
            h = rng.integers(0, V, size=int(rng.integers(1, 4000)))
        elif kind == 1:
            h = (rng.zipf(1.1, size=3000) - 1) % V
        elif kind == 2:
            h = np.array([int(rng.integers(0, V))] * 3)      # one entry, count 3
        elif kind == 3:
            h = rng.integers(V // 2, V // 2 + 300, size=500)  # one workgroup's range
        else:
            h = np.concatenate([rng.integers(0, V, 200), np.array([V, V + 5, V + 5])])  # ids at and above V
        hists.append(h)
    u = rng.random(B)
    a, refs, _ = run(dev, x, ps, u, hists, label=f"raw V{V}")
    b, _, _ = run(dev, x, ps, u, hists, label=f"pairs V{V}", pairs=True)
    for f in ("ids", "logprobs", "keep", "flags"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f


def test_hist_pairs_long_table(dev):
    """A table of more entries than two probe rounds resolve (V = 248320, ~200k distinct ids): the search narrows
    over further rounds."""
    rng = np.random.default_rng(3)
    B, V = 2, 248320
    x = (rng.standard_normal((B, V)) * 0.5).astype(np.float32)
    ps = [Sampling(top_p=0.9, repetition_penalty=1.5, frequency_penalty=0.05), Sampling(top_k=30, repetition_penalty=1.2)]
    hists = [rng.integers(0, V, size=400000), rng.integers(0, V, size=300000)]
    run(dev, x, ps, rng.random(B), hists, label="long pairs", pairs=True, max_excused=1)


def test_sampler_shim_sequence(dev):
    from volundr_amd.sampler import Sampler

    rng = np.random.default_rng(16)
    V = 7000
    sp = Sampling(temperature=0.9, top_k=40, top_p=0.9, repetition_penalty=1.2, presence_penalty=0.3, seed=99)
    smp = Sampler(sp, vocab_valid=V)
    counts, st, produced = {}, S.seed_state(99), 0
    for step in range(12):
        x = (rng.standard_normal(V) * 2).astype(np.float32)
        tok = smp.choose(torch.from_numpy(x).to(dev))
        st, u = S.xorshift64s_next(st)
        ref = S.sample(x, sp, u, counts, produced)
        assert tok == ref.token or ref.draw_boundary
        counts[ref.token] = counts.get(ref.token, 0) + 1
        produced += 1
    assert smp.counts == counts


@pytest.mark.parametrize("B,V,radix", [(16, 163840, False), (16, 163840, True), (24, 40000, False), (8, 65536, True),
                                       (32, 20000, False)])
def test_xcd_exchange_identical(dev, B, V, radix):
    """Batches whose rows each sit on one XCD exchange their data through that XCD's L2; the same calls with
    VS_DEBUG_NO_XCD_EXCHANGE use the device-coherent level. Every class (greedy, top-k, whole-row value bins, the
    gather and the radix fallback) returns the same bits both ways, and matches the oracle."""
    from volundr_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(B * 7 + V + radix)
    x = (rng.standard_normal((B, V)) * rng.choice([0.1, 1.0, 3.0], size=(B, 1))).astype(np.float32)
    ps = rand_params(rng, B, V)
    hists = [rng.integers(0, V, size=int(rng.integers(0, 500))) for _ in range(B)]
    u = rng.random(B)
    base = _lib.DEBUG_FORCE_RADIX if radix else 0
    try:
        L.vs_set_debug(base)
        a, _, _ = run(dev, x, ps, u, hists, label=f"xcd B{B} V{V} radix={radix}")
        a = tuple(t.cpu() for t in (a.ids, a.logprobs, a.keep, a.flags))
        L.vs_set_debug(base | _lib.DEBUG_NO_XCD_EXCHANGE)
        b, _, _ = run(dev, x, ps, u, hists, label=f"coherent B{B} V{V} radix={radix}")
        b = tuple(t.cpu() for t in (b.ids, b.logprobs, b.keep, b.flags))
    finally:
        L.vs_set_debug(0)
    assert all(torch.equal(p, q) for p, q in zip(a, b))


def test_xcd_placement(dev):
    """The placement the L2 exchange relies on: workgroups b and b + 8 of a grid run on the same XCD (the dispatcher
    deals workgroups to the 8 XCDs in turn), for grids of the sampling kernel's sizes."""
    from volundr_amd import _lib
    L = _lib.load()
    for nb in (8, 160, 240, 256, 1024):
        out = torch.full((nb,), 99, dtype=torch.int32, device=dev)
        assert L.vs_xcd_ids(out.data_ptr(), nb, 512, torch.cuda.current_stream(dev).cuda_stream) == 0
        ids = out.cpu().numpy()
        assert (ids < 8).all(), ids
        assert (ids == ids[np.arange(nb) % 8]).all(), f"grid {nb}: {ids[:32]}"
        print(f"grid {nb}: XCDs of workgroups 0-7 {ids[:8].tolist()}", flush=True)


def test_xcd_and_coherent_launches_alternate(dev):
    """One workspace shared by launches that alternate between the L2 exchange (16 rows: every row on one XCD) and
    the device-coherent one (12 rows): the rows' control blocks carry their call count across both kinds, so the
    flag barriers of a later call never pass on flags an earlier call left, and every call matches the oracle."""
    rng = np.random.default_rng(77)
    V = 163840
    for rep, B in enumerate([16, 12, 16, 12, 16]):
        x = (rng.standard_normal((B, V)) * rng.choice([0.1, 1.0], size=(B, 1))).astype(np.float32)
        ps = [Sampling(temperature=float(rng.choice([1.0, 0.8])), top_p=float(rng.choice([0.9, 0.95, 1.0])),
                       top_k=int(rng.choice([0, 0, 20]))) for _ in range(B)]
        run(dev, x, ps, rng.random(B), label=f"alternate {rep} B{B}", max_excused=1)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_xcd_exchange_half_precision(dev, dtype):
    """16 rows of 163840 half-precision logits (one row per XCD group, the L2 exchange) with every class, penalties
    and near-flat rows: oracle parity, and the same bits with the device-coherent exchange."""
    from volundr_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(91 + (dtype == torch.float16))
    B, V = 16, 163840
    x = (rng.standard_normal((B, V)) * rng.choice([0.1, 1.0, 3.0], size=(B, 1))).astype(np.float32)
    ps = rand_params(rng, B, V)
    hists = [rng.integers(0, V, size=int(rng.integers(0, 800))) for _ in range(B)]
    u = rng.random(B)
    a, _, _ = run(dev, x, ps, u, hists, dtype=dtype, label=f"xcd {dtype}", max_excused=1)
    try:
        L.vs_set_debug(_lib.DEBUG_NO_XCD_EXCHANGE)
        b, _, _ = run(dev, x, ps, u, hists, dtype=dtype, label=f"coherent {dtype}", max_excused=1)
    finally:
        L.vs_set_debug(0)
    assert all(torch.equal(p.cpu(), q.cpu()) for p, q in zip((a.ids, a.logprobs, a.keep, a.flags),
                                                             (b.ids, b.logprobs, b.keep, b.flags)))


@pytest.mark.parametrize("span,radix", [(0.5, False), (3.9, False), (4.2, False), (1.0, True)])
def test_narrow_rows(dev, span, radix):
    """Unit-temperature whole-vocabulary rows whose kept values span about `span` (the narrow value-bin pass at 2^31
    fixed point up to 4, the general one above), with top-p cuts, min-p (its radix select computes the same masses)
    and the radix fallback forced: oracle parity."""
    from volundr_amd import _lib
    L = _lib.load()
    rng = np.random.default_rng(int(span * 10) + radix)
    B, V = 16, 163840
    x = rng.uniform(-span / 2, span / 2, size=(B, V)).astype(np.float32)
    ps = [Sampling(temperature=1.0, top_p=float(rng.choice([0.5, 0.9, 0.95, 1.0])),
                   min_p=float(rng.choice([0.0, 0.0, 0.3]))) for _ in range(B)]
    try:
        L.vs_set_debug(_lib.DEBUG_FORCE_RADIX if radix else 0)
        run(dev, x, ps, rng.random(B), label=f"narrow span {span} radix {radix}", max_excused=1)
    finally:
        L.vs_set_debug(0)
