"""vs_sample_batch_noalloc (the allocation-free entry point, workspace in a fixed device array) against
vs_sample_batch on the same inputs, both through the C ABI: results must be identical, call after call, with the
second call smaller than the first (the array keeps the last call's contents, which the kernels leave zeroed)."""
import numpy as np
import pytest
import torch

from volundr_amd import _lib, synth
from volundr_amd.ops import _DTYPES, alloc_out, pack_rows, workspace
from volundr_amd.session import Sampling

pytestmark = pytest.mark.gpu


def _call(fn_name, x, rows, out, dev):
    L = _lib.load()
    ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
    B, V = x.shape
    head = (x.data_ptr(), _DTYPES[x.dtype], B, V, x.stride(0), rows.params.data_ptr(), ptr(rows.hist),
            ptr(rows.bias_ids), ptr(rows.bias_vals), ptr(rows.mask_ids), out.ids.data_ptr(), out.logprobs.data_ptr(),
            out.flags.data_ptr(), out.keep.data_ptr())
    stream = torch.cuda.current_stream(dev).cuda_stream
    if fn_name == "noalloc":
        rc = L.vs_sample_batch_noalloc(*head, stream)
    else:
        ws = workspace(dev, L.vs_sample_workspace_bytes(B, V))
        rc = L.vs_sample_batch(*head, ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, fn_name)
    return out


def _compare(dev, x, samplings, u, hists, label):
    print(f"[noalloc] {label}: B={x.shape[0]} V={x.shape[1]}", flush=True)
    rows = pack_rows(samplings, u, x.shape[1], hists).to(dev)
    a = _call("ws", x, rows, alloc_out(x.shape[0], dev), dev)
    b = _call("noalloc", x, rows, alloc_out(x.shape[0], dev), dev)
    torch.cuda.synchronize()
    for f in ("ids", "logprobs", "flags", "keep"):
        assert torch.equal(getattr(a, f), getattr(b, f)), f"{label}: {f} differs"
    return a


def test_noalloc_matches_workspace_entry(dev):
    L = _lib.load()
    assert L.vs_sample_noalloc_scratch_bytes() == L.vs_sample_workspace_bytes(16, 163840)  # 16 rows, ~5.6 MB
    # first call: the C5 shape (FULL rows: row barriers, histogram slots, gathers all use the array)
    d = synth.c5(seed=1)
    x = torch.from_numpy(d["logits"]).to(dev)
    _compare(dev, x, d["params"], d["u"], d["hists"], "c5")
    # second call, smaller: a mix of classes on 5 rows of V = 40000
    rng = np.random.default_rng(3)
    V = 40000
    xs = torch.from_numpy((rng.standard_normal((5, V)) * 2).astype(np.float32)).to(dev)
    ps = [Sampling(top_k=20), Sampling(top_p=0.9), Sampling(temperature=0.0), Sampling(top_k=300, top_p=0.95),
          Sampling(top_p=0.5, repetition_penalty=1.3)]
    hists = [rng.integers(0, V, size=50) for _ in range(5)]
    _compare(dev, xs, ps, rng.random(5), hists, "mix B5")
    # and the C3 shape once more after the small call
    d = synth.c3(seed=2)
    _compare(dev, torch.from_numpy(d["logits"]).to(dev), d["params"], d["u"], d["hists"], "c3")


def test_noalloc_timeout_leaves_the_array_zeroed(dev):
    """Rows that give up at a row barrier (forced from the host with a one-poll spin limit, so every kernel exits
    normally) report VS_OUT_TIMEOUT and leave the shared array zeroed: the next ordinary call through the
    allocation-free entry point equals vs_sample_batch, with no reset (its callers have none)."""
    L = _lib.load()
    d = synth.c5(seed=4)
    x = torch.from_numpy(d["logits"]).to(dev)
    rows = pack_rows(d["params"], d["u"], x.shape[1], d["hists"]).to(dev)
    print("[noalloc] forced timeout, c5 seed 4", flush=True)
    L.vs_set_spin_limit(1)
    try:
        t = _call("noalloc", x, rows, alloc_out(x.shape[0], dev), dev)
        torch.cuda.synchronize()
    finally:
        L.vs_set_spin_limit(0)
    flags = [int(f) & 0xFFFFFFFF for f in t.flags.cpu().tolist()]
    assert any(f & _lib.OUT_TIMEOUT for f in flags)
    _compare(dev, x, d["params"], d["u"], d["hists"], "c5 after timeout")


def test_noalloc_rejects_bad_arguments(dev):
    L = _lib.load()
    assert L.vs_sample_batch_noalloc(0, 0, -1, 10, 10, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) == _lib.VS_EINVAL
    assert L.vs_sample_batch_noalloc(0, 0, 0, 10, 10, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) == _lib.VS_OK
