"""CPU pinning of oracle/lmhead_ref.py (bf16 lm_head + greedy verify, volundr-mlx/volundr.py:958-968,
spec/specdec.py:326-327) against torch's bf16 conversion and pure-Python sums."""
import math

import numpy as np
import torch

from oracle import lmhead_ref as L


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0, 3.4e38, 1e-40], np.float32)])
    # exact halfway cases: bit 15 set, lower bits zero, both parities of bit 16
    hw = (rng.integers(0, 1 << 15, 200).astype(np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, hw])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(L.bf16_rne(x), want)
    assert np.isnan(L.bf16_to_f32(L.bf16_rne(np.array([np.nan], np.float32))))[0]


def test_logits_exact_against_fsum():
    rng = np.random.default_rng(1)
    h = L.bf16_rne(rng.standard_normal((3, 64)).astype(np.float32))
    w = L.bf16_rne(rng.standard_normal((20, 64)).astype(np.float32))
    ex = L.logits_exact(h, w)
    hf, wf = L.bf16_to_f32(h), L.bf16_to_f32(w)
    for r in range(3):
        for n in range(20):
            want = math.fsum(float(hf[r, k]) * float(wf[n, k]) for k in range(64))
            assert abs(ex[r, n] - want) <= 1e-12 * (1 + abs(want))
    b, amb = L.logits_bf16(h, w)
    # the correctly rounded value: torch's float64 -> bf16 conversion
    want = torch.from_numpy(ex).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(b, want)


def test_ambiguity_flag():
    # a value exactly between two bf16 neighbours is ambiguous under any positive error bound; a bf16 value itself is
    # not (for a small bound)
    h = L.bf16_rne(np.array([[1.0, 1.0]], np.float32))
    one_plus = L.bf16_to_f32(np.array([0x3F80 + 1], np.uint16))[0]  # 1 + 2^-7
    w = L.bf16_rne(np.array([[1.0, 2.0 ** -8], [1.0, 0.0], [one_plus, 0.0]], np.float32))
    b, amb = L.logits_bf16(h, w)
    assert amb[0, 0] and not amb[0, 1] and not amb[0, 2]
    assert L.bf16_to_f32(b[0, 1]) == 1.0 and L.bf16_to_f32(b[0, 2]) == one_plus


def test_verify_on_planted_argmax():
    rng = np.random.default_rng(2)
    R, K, N = 5, 32, 50
    h = L.bf16_rne(rng.standard_normal((R, K)).astype(np.float32))
    w = L.bf16_rne(rng.standard_normal((N, K)).astype(np.float32) * 0.1)
    w[7] = L.bf16_rne(L.bf16_to_f32(h[0]) * 4)  # row 7 aligns with position 0: its logit is the largest there
    w[9] = w[7]      # an exact tie: the lower id wins
    drafts = np.array([[7, 3, 3, 3]], np.int32)
    b, amb, tok, acc, lp = L.verify(h, w, drafts, N, 1, R)
    assert tok[0, 0] == 7 and acc[0] == 1 and lp.shape == (1, R)
    assert int(np.argmax(L.logits_exact(h, w)[0])) in (7, 9)
