"""GPU parity of vs_lmhead_sample (the bf16 lm_head with Sampler.sample fused after it) through the C ABI.

The head's bf16 logits are taken from vs_lmhead_verify_greedy with return_logits on the same h and W: the two
kernels share the MFMA loop, tile mapping and accumulation order, so the logits are the same bits (test_gpu_lmhead.py
pins them against the exact products). On those logits the fused result must equal vs_sample_batch bit for bit (ids,
logprobs, flags, kept sizes), and the oracle (sampler.py:100-156 restated) to the parity bar."""
import numpy as np
import pytest
import torch

from oracle import sampler_ref as S
from parity import check_sample
from volundr_amd import lmhead_sample, lmhead_verify_greedy, ops
from volundr_amd._lib import OUT_UNSUPPORTED
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu


def _head(dev, R, N, K, seed, scale=1.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    h = (torch.randn(R, K, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g, device=dev) * (scale * 4.0 / K ** 0.5)).to(torch.bfloat16)
    return h, W


def _logits(h, W):
    _, lg = lmhead_verify_greedy(h.unsqueeze(0), W, torch.zeros(1, h.shape[0] - 1, dtype=torch.int32,
                                                                device=h.device), return_logits=True)
    return lg[0]  # bf16 [R, N]


def _compare(dev, h, W, sps, u, label, argmax_vv=None, max_excused=None):
    R, N = h.shape[0], W.shape[0]
    print(f"[lmhead_sample] {label}: R={R} N={N} K={h.shape[1]}", flush=True)
    got = lmhead_sample(h, W, sps, u, argmax_vv=argmax_vv)
    lg = _logits(h, W)
    rows = ops.pack_rows(sps, u, N, None, argmax_vv=argmax_vv).to(dev)
    want = ops.sample_rows(lg.float().contiguous(), rows)
    torch.cuda.synchronize()
    for f in ("ids", "flags", "keep"):
        assert torch.equal(getattr(got, f), getattr(want, f)), f"{label}: {f} {getattr(got, f)} vs {getattr(want, f)}"
    # sampled rows draw from the same sorted keys: identical logprobs; a greedy row's log-softmax sums its
    # exponentials in another grouping (a few float32 roundings apart)
    greedy = torch.tensor([sp.greedy for sp in sps], device=dev)
    gl, wl = got.logprobs.double(), want.logprobs.double()
    assert torch.equal(gl[~greedy], wl[~greedy]), label
    assert torch.all((gl - wl).abs() <= 1e-5 * wl.abs() + 1e-10), label
    x = lg.float().cpu().numpy()
    refs = []
    for i, sp in enumerate(sps):
        if argmax_vv is not None and argmax_vv[i] is not None:
            continue
        refs.append((i, S.sample(x[i], sp, float(u[i]), {}, 0)))
    sub = ops.SampleOut(*(getattr(got, f)[[i for i, _ in refs]] for f in ("ids", "logprobs", "flags", "keep")))
    check_sample(sub, [r for _, r in refs], label, max_excused)
    return got, x


def _mixed(rng, R):
    ks = [1, 2, 5, 20, 20, 50, 64, 3, 40, 64, 8, 30, 20, 16, 64, 10]
    sps = []
    for i in range(R):
        if i % 7 == 6:
            sps.append(Sampling(temperature=0.0))  # greedy: argmax over the whole row
        else:
            sps.append(Sampling(top_k=ks[i % len(ks)], temperature=float(rng.choice([0.5, 0.8, 1.0, 1.4])),
                                top_p=float(rng.choice([1.0, 0.95, 0.8, 0.3])),
                                min_p=float(rng.choice([0.0, 0.0, 0.1]))))
    return sps


@pytest.mark.parametrize("R,N,K", [(16, 40000, 512), (5, 12345, 768), (1, 3000, 256), (16, 163840, 1024)])
def test_fused_equals_logits_path(dev, R, N, K):
    rng = np.random.default_rng(R + N)
    h, W = _head(dev, R, N, K, seed=N)
    _compare(dev, h, W, _mixed(rng, R), rng.random(R), f"mix R{R}", max_excused=1)


def test_ties_and_argmax_vv(dev):
    """bf16 logits tie often: a head whose weight rows repeat (equal logits at many ids) must still give the lower
    id first among equal values; argmax-only rows skip the columns at and above vocab_valid, where the maximum sits."""
    R, N, K = 8, 20000, 512
    h, W = _head(dev, R, N, K, seed=3)
    W[1000:1200] = W[5]      # 201 equal logits per row, among the largest when row 5 is large
    W[N - 50:] = W[7] * 4    # the padding columns hold each row's largest logits
    sps = [Sampling(top_k=20), Sampling(top_k=64, top_p=0.9), Sampling(temperature=0.0), Sampling(top_k=1),
           Sampling(temperature=0.0), Sampling(top_k=5, temperature=0.7), Sampling(temperature=0.0),
           Sampling(top_k=64)]
    avv = [None, None, N - 50, None, None, None, 123, None]
    rng = np.random.default_rng(4)
    _, x = _compare(dev, h, W, sps, rng.random(R), "ties", argmax_vv=avv)
    got = lmhead_sample(h, W, sps, rng.random(R), argmax_vv=avv)
    assert int(got.ids[2]) == int(np.argmax(x[2, :N - 50])) and int(got.ids[6]) == int(np.argmax(x[6, :123]))


def test_nonfinite_logits(dev):
    """A weight row of infinities makes that id's logit +inf or -inf (or NaN with mixed signs): top-k keeps finite
    logits only (sampler.py:130-136), greedy rows follow np.argmax (NaN first)."""
    R, N, K = 4, 5000, 256
    h, W = _head(dev, R, N, K, seed=9)
    W[17] = float("inf")
    sps = [Sampling(top_k=10), Sampling(temperature=0.0), Sampling(top_k=64, temperature=0.6), Sampling(top_k=3)]
    _compare(dev, h, W, sps, np.random.default_rng(5).random(R), "nonfinite")


def test_unsupported_rows(dev):
    """Rows that need their logits: the C ABI flags them VS_OUT_UNSUPPORTED; the Python call takes the unfused path
    for the whole batch and equals vs_sample_batch on the head's logits."""
    from volundr_amd import _lib

    R, N, K = 4, 6000, 256
    h, W = _head(dev, R, N, K, seed=11)
    sps = [Sampling(top_k=20), Sampling(top_p=0.9), Sampling(top_k=20, logit_bias=[(5, 2.0)]), Sampling(top_k=200)]
    u = np.random.default_rng(6).random(R)
    rows = ops.pack_rows(sps, u, N, None).to(dev)
    out = ops.alloc_out(R, dev)
    L = _lib.load()
    ws = ops.workspace(dev, L.vs_lmhead_sample_workspace_bytes(R), "lmsample")
    _lib.check(L.vs_lmhead_sample(h.data_ptr(), K, W.data_ptr(), K, N, K, R, rows.params.data_ptr(), out.ids.data_ptr(),
                                  out.logprobs.data_ptr(), out.flags.data_ptr(), out.keep.data_ptr(), ws.data_ptr(),
                                  ws.numel(), ops._stream_handle(dev)), "vs_lmhead_sample")
    fl = [int(f) & 0xFFFFFFFF for f in out.flags.cpu().tolist()]
    assert [bool(f & OUT_UNSUPPORTED) for f in fl] == [False, True, True, True]
    got = lmhead_sample(h, W, sps, u)
    want = ops.sample_rows((h @ W.t()).contiguous(), rows)
    assert torch.equal(got.ids, want.ids) and torch.equal(got.logprobs, want.logprobs)


def test_full_size_head(dev):
    """The production head: 248320 x 5120 bf16, 16 decode rows."""
    R, N, K = 16, 248320, 5120
    h, W = _head(dev, R, N, K, seed=21)
    rng = np.random.default_rng(22)
    _compare(dev, h, W, _mixed(rng, R), rng.random(R), "full head", max_excused=1)
