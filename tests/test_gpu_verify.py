"""GPU parity of vs_verify_greedy against the NumPy oracle: argmax and accept bit-exact, logprob within 1e-5."""
import numpy as np
import pytest
import torch

from oracle import verify_ref as VR
from volundr_amd import emitted, synth, verify_greedy

pytestmark = pytest.mark.gpu


def check(dev, bits_or_f32, drafts, vv, dtype, label):
    B, T, V = bits_or_f32.shape
    if bits_or_f32.dtype == np.uint16:
        xt = torch.from_numpy(bits_or_f32.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(bits_or_f32).to(dev).to(dtype)
    print(f"[{label}] B={B} T={T} V={V} vv={vv} {xt.dtype}", flush=True)
    ref_in = xt.float().cpu().numpy()
    dt = torch.from_numpy(drafts).to(dev) if T > 1 else None
    o = verify_greedy(xt, dt, vv)
    torch.cuda.synchronize()
    tok, acc, lp = VR.verify(ref_in, drafts, vv)
    assert np.array_equal(o.argmax.cpu().numpy(), tok), label
    assert np.array_equal(o.accept.cpu().numpy(), acc), label
    g = o.logprobs.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(g - lp) <= 1e-5 * np.abs(lp) + 1e-10), (label, np.max(np.abs(g - lp)))
    return o


@pytest.mark.parametrize("name", ["c2", "c4"])
def test_configs(dev, name):
    d = synth.CONFIGS[name](seed=0, tie_frac=0.2)
    o = check(dev, d["logits_bf16"], d["drafts"], 163840, torch.bfloat16, name)
    assert np.array_equal(o.accept.cpu().numpy(), d["accept"])
    # the emitted tokens of each request (specdec.py:335-336, scheduler.py:465-470) from the device outputs
    tok, acc, _ = VR.verify(d["logits_bf16"], d["drafts"], 163840)
    am, ac = o.argmax.cpu().tolist(), o.accept.cpu().tolist()
    for b in range(len(ac)):
        got = emitted(d["drafts"][b].tolist(), am[b], ac[b])
        assert got == VR.emitted(d["drafts"][b], tok[b], int(acc[b])), (name, b)
        assert len(got) == ac[b] + 1


def test_ties_and_vocab_valid(dev):
    rng = np.random.default_rng(5)
    x = rng.integers(-4, 5, size=(3, 6, 5000)).astype(np.float32)  # heavy ties: first max must win
    drafts = np.argmax(x[..., :4990], -1)[:, :5].astype(np.int32)
    drafts[1, 2] += 1
    check(dev, x, drafts, 4990, torch.float32, "ties f32")
    check(dev, x, drafts, 4990, torch.bfloat16, "ties bf16")
    check(dev, x, drafts, 4990, torch.float16, "ties f16")


def test_single_position_and_odd_sizes(dev):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((5, 1, 12345)).astype(np.float32)
    check(dev, x, np.zeros((5, 0), np.int32), 12345, torch.float32, "T=1")
    x = rng.standard_normal((2, 9, 777)).astype(np.float32)
    d = np.argmax(x, -1)[:, :8].astype(np.int32)
    check(dev, x, d, 777, torch.float32, "odd")


def test_nonfinite(dev):
    x = np.zeros((1, 3, 300), np.float32)
    x[0, 0, 5] = np.nan
    x[0, 1, :] = -np.inf
    x[0, 2, 9] = np.inf
    x[0, 2, 10] = np.inf
    o = verify_greedy(torch.from_numpy(x).to(dev), torch.tensor([[5, 0]], dtype=torch.int32, device=dev), 300)
    assert o.argmax.cpu().tolist() == [[5, 0, 9]] and o.accept.item() == 2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_nonfinite_across_workgroups(dev, dtype):
    """NaN ranks first (np.argmax), +inf beats every finite value, all -inf gives index 0, signed zeros tie (first
    index wins), and the maximum may sit in the row's last element: positions spread over several workgroups."""
    V, T = 40000, 8
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((1, T, V)) - 10.0).astype(np.float32)
    x[0, 0, 100] = 3.0
    x[0, 0, 30000] = np.nan
    x[0, 1, 25000] = np.nan
    x[0, 1, 39000] = np.nan
    x[0, 2, 35000] = np.inf
    x[0, 2, 12000] = np.inf
    x[0, 3, :] = -np.inf
    x[0, 4, :] = -np.inf
    x[0, 4, 20000] = 1.5
    x[0, 5, 500] = -0.0
    x[0, 5, 300] = 0.0
    x[0, 6, 200] = -0.0
    x[0, 6, 800] = 0.0
    x[0, 7, V - 1] = 6.0
    xt = torch.from_numpy(x).to(dev).to(dtype)
    ref_in = xt.float().cpu().numpy()
    want = np.argmax(ref_in, axis=-1).astype(np.int32)
    assert want[0].tolist() == [30000, 25000, 12000, 0, 20000, 300, 200, V - 1]
    drafts = want[:, :-1].copy()
    print(f"[nonfinite] V={V} T={T} {dtype}", flush=True)
    o = verify_greedy(xt, torch.from_numpy(drafts).to(dev), V)
    torch.cuda.synchronize()
    assert np.array_equal(o.argmax.cpu().numpy(), want)
    assert o.accept.item() == T - 1
    _, _, lp = VR.verify(ref_in, drafts, V)
    g = o.logprobs.cpu().numpy().astype(np.float64)
    fin = [4, 5, 6, 7]  # finite maximum and no NaN or +inf in the position
    assert np.all(np.abs(g[0, fin] - lp[0, fin]) <= 1e-5 * np.abs(lp[0, fin]) + 1e-10), (g[0, fin], lp[0, fin])


@pytest.mark.parametrize("T", [2, 32, 33, 34, 40, 65, 70])
def test_accept_lengths_around_the_packed_limit(dev, T):
    """Blocks of up to 33 positions carry the accept information in one packed word, longer ones take the
    counter-and-reload path: every accept length 0..T-1 on both sides of the limit."""
    rng = np.random.default_rng(T)
    B, V = T, 3000  # request b gets its first mismatch at position b (b = T-1: all drafts accepted)
    x = rng.standard_normal((B, T, V)).astype(np.float32)
    tok = np.argmax(x, -1)
    drafts = tok[:, :-1].astype(np.int32).copy()
    for b in range(B):
        if b < T - 1:
            drafts[b, b] = (drafts[b, b] + 1) % V
    o = check(dev, x, drafts, V, torch.float32, f"T={T}")
    assert o.accept.cpu().tolist() == list(range(T))


def test_more_rows_than_one_launch_holds(dev):
    """2040 positions: more workgroups than the device keeps resident at once, so the call runs as several
    launches, and requests whose rows straddle two launches read the earlier launch's tokens."""
    rng = np.random.default_rng(21)
    B, T, V = 120, 17, 5000
    x = rng.standard_normal((B, T, V)).astype(np.float32)
    tok = np.argmax(x, -1)
    drafts = tok[:, :-1].astype(np.int32).copy()
    for b in range(B):
        j = b % T
        if j < T - 1:
            drafts[b, j] = (drafts[b, j] + 1) % V
    o = check(dev, x, drafts, V, torch.float32, "B120 T17")
    assert o.accept.cpu().tolist() == [b % T for b in range(B)]


def test_repeated_calls_on_one_workspace(dev):
    """Calls of different shapes back to back on one workspace: the words a call reads carry its own tag, so a
    call never takes what an earlier one left."""
    rng = np.random.default_rng(22)
    for rep, (B, T, V) in enumerate([(4, 17, 7000), (1, 17, 7000), (3, 5, 9000), (4, 17, 7000), (2, 33, 4000)]):
        x = rng.standard_normal((B, T, V)).astype(np.float32)
        drafts = np.argmax(x, -1)[:, :-1].astype(np.int32).copy()
        drafts[0, rep % (T - 1)] += 1
        check(dev, x, drafts, V, torch.float32, f"shape {B}x{T}x{V}")


def test_long_blocks_accept_lengths(dev):
    """Blocks of 130 positions: the request's finisher reads its tokens 64 per ballot over three rounds, all of them
    (also past the first mismatch, whose round decides the accept length); a second call on the same workspace."""
    rng = np.random.default_rng(31)
    T, V = 130, 2000
    want_acc = [0, 63, 64, 100, 129]
    B = len(want_acc)
    for rep in range(2):
        x = rng.standard_normal((B, T, V)).astype(np.float32)
        tok = np.argmax(x, -1)
        drafts = tok[:, :-1].astype(np.int32).copy()
        for b, a in enumerate(want_acc):
            if a < T - 1:
                drafts[b, a] = (drafts[b, a] + 1) % V
        o = check(dev, x, drafts, V, torch.float32, f"T={T} rep {rep}")
        assert o.accept.cpu().tolist() == want_acc


def _check_f32_floor(dev, x, drafts, vv, dtype, label):
    """As check, with the logprob's absolute floor at 2^-22 instead of 1e-10: the kernel sums exp(x - max) in
    float32 per lane, so a row where one token holds nearly all the mass (logprob near 0) carries the float32
    rounding of a sum near 1 (the reference's own float32 log-softmax does too)."""
    B, T, V = x.shape
    xt = torch.from_numpy(x).to(dev).to(dtype)
    ref_in = xt.float().cpu().numpy()
    o = verify_greedy(xt, torch.from_numpy(drafts).to(dev) if T > 1 else None, vv)
    torch.cuda.synchronize()
    tok, acc, lp = VR.verify(ref_in, drafts, vv)
    assert np.array_equal(o.argmax.cpu().numpy(), tok), label
    assert np.array_equal(o.accept.cpu().numpy(), acc), label
    g = o.logprobs.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(g - lp) <= 1e-5 * np.abs(lp) + 2.0 ** -22), (label, np.max(np.abs(g - lp)))


def test_random_shapes_one_workspace(dev):
    """60 seeded calls of random shape (B 1-8, T 1-40, V 100-20000, vocab_valid from V/2 to V) and dtype on one
    workspace, each against the oracle: the exchange slots' epochs keep every call apart from the earlier ones.
    Some rows are dominated by one token, hence the float32 floor of _check_f32_floor."""
    rng = np.random.default_rng(123)
    for it in range(60):
        B, T, V = int(rng.integers(1, 9)), int(rng.integers(1, 41)), int(rng.integers(100, 20000))
        vv = int(rng.integers(max(1, V // 2), V + 1))
        dt = [torch.float32, torch.bfloat16, torch.float16][it % 3]
        x = (rng.standard_normal((B, T, V)) * rng.uniform(0.5, 4)).astype(np.float32)
        xt = torch.from_numpy(x).to(dev).to(dt)
        ref = xt.float().cpu().numpy()
        drafts = np.argmax(ref[..., :vv], -1)[:, :-1].astype(np.int32).copy() if T > 1 else np.zeros((B, 0), np.int32)
        for b in range(B):
            if T > 1 and rng.random() < 0.7:
                j = int(rng.integers(0, T - 1))
                drafts[b, j] = (drafts[b, j] + 1) % vv
        _check_f32_floor(dev, ref, drafts, vv, dt, f"random {it}: B={B} T={T} V={V} vv={vv}")
