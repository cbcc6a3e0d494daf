"""GPU parity of vs_lmhead_verify_greedy (the bf16 lm_head with greedy verify fused in; volundr-mlx/volundr.py:958-968
-> spec/specdec.py:326-327) against oracle/lmhead_ref.py:
  * logits: equal to the correctly rounded bf16 values except where the exact value lies within the float32
    accumulation bound of a bf16 rounding boundary (`ambiguous`), where one ulp either way is allowed;
  * argmax, accept: bit-exact to verify on the kernel's own logits (the epilogue), and to the oracle wherever no
    ambiguous logit is within reach of the maximum; logprob within 1e-5 relative."""
import numpy as np
import pytest
import torch

from oracle import lmhead_ref as L
from oracle import verify_ref as VR
from volundr_amd import lmhead_verify_greedy, verify_greedy

pytestmark = pytest.mark.gpu


def _bits_tensor(bits, dev):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(dev)


def _case(seed, B, T, K, N, scale=1.0, plant=True):
    rng = np.random.default_rng(seed)
    h = L.bf16_rne(rng.standard_normal((B * T, K)).astype(np.float32))
    w = L.bf16_rne((rng.standard_normal((N, K)) * scale / np.sqrt(K)).astype(np.float32))
    drafts = rng.integers(0, N, (B, max(T - 1, 0))).astype(np.int32)
    if plant:
        # make some drafts right so accept lengths vary
        ex = L.logits_exact(h, w)
        tok = ex.reshape(B, T, N).argmax(-1)
        for b in range(B):
            n = int(rng.integers(0, T))
            drafts[b, :n] = tok[b, :n]
    return h, w, drafts


def _run(dev, h, w, drafts, B, T, vv):
    K = h.shape[1]
    o, lg = lmhead_verify_greedy(_bits_tensor(h, dev).reshape(B, T, K), _bits_tensor(w, dev),
                                 torch.from_numpy(drafts).to(dev) if T > 1 else None, vocab_valid=vv,
                                 return_logits=True)
    torch.cuda.synchronize()
    return o, lg.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B * T, -1)


def _check(o, got, h, w, drafts, B, T, vv):
    want, amb = L.logits_bf16(h, w)
    bad = (got != want) & ~amb
    assert not bad.any(), f"{int(bad.sum())} logits differ outside the ambiguity band, first at {np.argwhere(bad)[0]}"
    # every logit lies between the bf16 roundings of (exact - bound) and (exact + bound)
    ex, eb = L.logits_exact(h, w), L.fp32_error_bound(h, w)
    gf = L.bf16_to_f32(got).astype(np.float64)
    lo = L.bf16_to_f32(L.bf16_rne((ex - eb).astype(np.float32)))
    hi = L.bf16_to_f32(L.bf16_rne((ex + eb).astype(np.float32)))
    assert ((gf >= lo) & (gf <= hi)).all()
    # the epilogue, bit-exact on the kernel's own logits
    tok, acc, lp = VR.verify(got.reshape(B, T, -1), drafts, vv)
    np.testing.assert_array_equal(o.argmax.cpu().numpy(), tok)
    np.testing.assert_array_equal(o.accept.cpu().numpy(), acc)
    np.testing.assert_allclose(o.logprobs.cpu().numpy(), lp, rtol=1e-5, atol=1e-6)
    # and equal to the oracle's argmax where rounding cannot move it
    wt, _, _ = VR.verify(want.reshape(B, T, -1), drafts, vv)
    wf = L.bf16_to_f32(want).reshape(B, T, -1)[..., :vv]
    for b in range(B):
        for t in range(T):
            mx = wf[b, t].max()
            close = np.abs(wf[b, t] - mx) <= 2.0 ** -6 * max(abs(mx), 1e-30)
            if not (amb.reshape(B, T, -1)[b, t, :vv] & close).any() and close.sum() == 1:
                assert tok[b, t] == wt[b, t], (b, t)


@pytest.mark.parametrize("B,T", [(1, 1), (1, 16), (1, 17), (2, 16), (1, 33), (3, 16), (4, 16), (4, 17), (5, 16)])
def test_lmhead_verify_shapes(dev, B, T):
    K, N = 1024, 5003
    vv = N - 37
    h, w, drafts = _case(B * 100 + T, B, T, K, N, scale=4.0)
    o, got = _run(dev, h, w, drafts, B, T, vv)
    _check(o, got, h, w, drafts, B, T, vv)


@pytest.mark.parametrize("B,T,N", [(4, 17, 900), (1, 17, 200), (1, 17, 600), (1, 17, 5003)])
def test_lmhead_fewer_workgroups_than_positions(dev, B, T, N):
    """A vocabulary of fewer 16-row tiles than positions gives fewer workgroups than positions, so a second launch
    merges the partials instead of one workgroup per position (N = 900 at 68 positions, N = 200 at 17); N = 600
    merges in the launch with 38 workgroups, between calls with 256 on the same workspace (every partial slot
    belongs to one position and one workgroup, whatever the grid)."""
    K = 1024
    vv = N - 7
    h, w, drafts = _case(B * 1000 + N, B, T, K, N, scale=4.0)
    o, got = _run(dev, h, w, drafts, B, T, vv)
    _check(o, got, h, w, drafts, B, T, vv)


def test_lmhead_hidden_5120_and_exact_ties(dev):
    B, T, K, N = 1, 17, 5120, 20000
    h, w, drafts = _case(7, B, T, K, N, scale=4.0)
    ex = L.logits_exact(h, w)
    # duplicate the winning row of position 3 at a higher and a lower id: the lowest id wins the exact tie
    win = int(ex[3].argmax())
    w[N - 5] = w[win]
    w[11] = w[win]
    o, got = _run(dev, h, w, drafts, B, T, N)
    _check(o, got, h, w, drafts, B, T, N)
    assert int(o.argmax[0, 3]) == min(11, win)


def test_lmhead_matches_verify_kernel_on_its_logits(dev):
    """The fused epilogue equals vs_verify_greedy run on the logits the fused kernel reports."""
    B, T, K, N = 2, 17, 2048, 40000
    h, w, drafts = _case(11, B, T, K, N, scale=3.0)
    o, got = _run(dev, h, w, drafts, B, T, N - 100)
    lg = _bits_tensor(got, dev).reshape(B, T, N)
    ov = verify_greedy(lg, torch.from_numpy(drafts).to(dev), N - 100)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o.argmax.cpu().numpy(), ov.argmax.cpu().numpy())
    np.testing.assert_array_equal(o.accept.cpu().numpy(), ov.accept.cpu().numpy())
    np.testing.assert_allclose(o.logprobs.cpu().numpy(), ov.logprobs.cpu().numpy(), rtol=1e-5, atol=1e-6)


def test_lmhead_nonfinite_outputs(dev):
    """Head outputs with infinities and NaN (an infinite hidden entry times weights of both signs gives +-inf rows;
    two of opposite signs give NaN where the weights agree in sign) and a zero hidden row (every logit 0, one tie
    over the vocabulary): the epilogue's exact per-value path, against np.argmax on the kernel's own logits and
    against vs_verify_greedy run on them."""
    B, T, K, N = 1, 17, 1024, 30000
    h, w, drafts = _case(31, B, T, K, N, plant=False)
    h = h.copy()
    h[2, 5] = 0x7F80  # +inf
    h[4, 5] = 0x7F80
    h[4, 9] = 0xFF80  # -inf
    h[6, :] = 0
    o, got = _run(dev, h, w, drafts, B, T, N)
    tok, acc, _ = VR.verify(got.reshape(B, T, -1), drafts, N)
    gf = L.bf16_to_f32(got).reshape(B, T, -1)
    assert np.isposinf(gf[0, 2]).any() and np.isnan(gf[0, 4]).any() and (gf[0, 6] == 0).all()
    np.testing.assert_array_equal(o.argmax.cpu().numpy(), tok)
    np.testing.assert_array_equal(o.accept.cpu().numpy(), acc)
    assert int(o.argmax[0, 6]) == 0
    ov = verify_greedy(_bits_tensor(got, dev).reshape(B, T, N), torch.from_numpy(drafts).to(dev), N)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o.argmax.cpu().numpy(), ov.argmax.cpu().numpy())
    fin = np.isfinite(gf).all(axis=-1)[0]  # positions without any non-finite logit
    np.testing.assert_allclose(o.logprobs.cpu().numpy()[0, fin], ov.logprobs.cpu().numpy()[0, fin], rtol=1e-5,
                               atol=1e-6)


def test_lmhead_full_size_against_torch(dev):
    """vocab 248320 x hidden 5120 (the model's head), B=1, T=17: logits against torch's float32 matmul of the same
    bf16 operands (a plain PyTorch float32 reference), rounded to bf16; argmax/accept/logprob against the verify
    oracle on the kernel's logits."""
    B, T, K, N, vv = 1, 17, 5120, 248320, 248077
    g = torch.Generator(device=dev).manual_seed(3)
    h = torch.randn(B * T, K, generator=g, device=dev).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g, device=dev) / 16).to(torch.bfloat16)
    ref = (h.float() @ W.float().T)
    tok_ref = ref.to(torch.bfloat16).float()[:, :vv].argmax(-1)
    drafts = tok_ref[:16].reshape(1, 16).to(torch.int32).clone()
    drafts[0, 9] = (drafts[0, 9] + 1) % vv  # accept length 9
    o, lg = lmhead_verify_greedy(h.reshape(B, T, K), W, drafts, vocab_valid=vv, return_logits=True)
    torch.cuda.synchronize()
    d = (lg.reshape(B * T, N).float() - ref).abs()
    bound = K * 2.0 ** -24 * (h.float().abs() @ W.float().abs().T) + ref.abs() * 2.0 ** -8
    assert bool((d <= bound).all())
    got = lg.view(torch.int16).cpu().numpy().view(np.uint16).reshape(B, T, N)
    tok, acc, lp = VR.verify(got, drafts.cpu().numpy(), vv)
    np.testing.assert_array_equal(o.argmax.cpu().numpy(), tok)
    np.testing.assert_array_equal(o.accept.cpu().numpy(), acc)
    np.testing.assert_allclose(o.logprobs.cpu().numpy(), lp, rtol=1e-5, atol=1e-6)
    assert int(o.accept[0]) <= 9


@pytest.mark.parametrize("B,T,K", [(1, 17, 768), (1, 1, 1280), (2, 16, 256), (4, 17, 768)])
def test_lmhead_hidden_sizes(dev, B, T, K):
    """Any hidden size that is a multiple of 256 (the 512-wide k chunks are used only where K allows them)."""
    N = 3001
    h, w, drafts = _case(K + B * T, B, T, K, N, scale=4.0)
    o, got = _run(dev, h, w, drafts, B, T, N)
    _check(o, got, h, w, drafts, B, T, N)
