"""The cooperative radix select of the FULL class (top-p and the draw by a mass-weighted radix select on the 64-bit
keys), forced for every large kept set with the VS_DEBUG_FORCE_RADIX testing flag: otherwise it only runs with
min-p or when value bins are too full to refine, so its top-p and draw answers get little coverage from the other
tests. Checked against the oracle with the ordinary parity rules."""
import numpy as np
import pytest
import torch

from oracle import sampler_ref as S
from parity import check_sample
from volundr_amd import _lib, sample_batch
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu


def _forced(fn):
    L = _lib.load()
    L.vs_set_debug(_lib.DEBUG_FORCE_RADIX)
    try:
        r = fn()
        torch.cuda.synchronize()
    finally:
        L.vs_set_debug(0)
    return r


@pytest.mark.parametrize("V,B", [(40000, 12), (163840, 8)])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_forced_radix_matches_oracle(dev, V, B, seed):
    rng = np.random.default_rng(500 + seed + V)
    x = (rng.standard_normal((B, V)) * rng.choice([0.1, 0.5, 1.0, 2.0], size=(B, 1))).astype(np.float32)
    ps = [Sampling(temperature=float(rng.choice([0.7, 1.0, 1.3])), top_k=0,
                   top_p=float(rng.choice([1.0, 0.95, 0.8, 0.3])), min_p=float(rng.choice([0.0, 0.0, 0.05])),
                   repetition_penalty=float(rng.choice([1.0, 1.3])), frequency_penalty=float(rng.choice([0.0, 0.1])))
          for _ in range(B)]
    hists = [rng.integers(0, V, size=int(rng.integers(0, 300))) for _ in range(B)]
    u = rng.random(B)
    xt = torch.from_numpy(x).to(dev)
    print(f"[radix] V={V} B={B} seed={seed}", flush=True)
    out = _forced(lambda: sample_batch(xt, ps, u, hists))
    refs = [S.sample(x[i], ps[i], float(u[i]), S.counts_from_history(hists[i])) for i in range(B)]
    check_sample(out, refs, f"radix V{V} s{seed}", max_excused=1)
