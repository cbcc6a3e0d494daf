"""The sampling and verify entry points captured in a HIP graph (torch.cuda.CUDAGraph on a side stream whose
workspace was zeroed before the capture, so that only kernels are recorded): every replay, with eager work of the
same library between replays, returns exactly the eager results, since the kernels leave their workspaces zeroed."""
import numpy as np
import pytest
import torch

from volundr_amd import ops, synth

pytestmark = pytest.mark.gpu


def _capture(make_call, n=3):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call = make_call()
        call(0)  # eager, on the side stream: binds it and zeroes its workspace outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for _ in range(n):
            call(0)
    return g, call


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_sample_graph_replays(dev, name):
    d = synth.CONFIGS[name](seed=4)
    x = torch.from_numpy(d["logits"]).to(dev)
    rows = ops.pack_rows(d["params"], d["u"], x.shape[1], d["hists"]).to(dev)
    eager = ops.PreparedSample([x], rows)
    e = eager(0)
    torch.cuda.synchronize()
    want = (e.ids.cpu().numpy().copy(), e.logprobs.cpu().numpy().copy(), e.flags.cpu().numpy().copy())
    print(f"[graph] capture {name}", flush=True)
    g, call = _capture(lambda: ops.PreparedSample([x], rows))
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        got = (call.out.ids.cpu().numpy(), call.out.logprobs.cpu().numpy(), call.out.flags.cpu().numpy())
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b, err_msg=f"replay {r}")
        eager(0)  # the program's own eager work between replays
        torch.cuda.synchronize()
        np.testing.assert_array_equal(eager.out.ids.cpu().numpy(), want[0])


def test_verify_graph_replays(dev):
    d = synth.CONFIGS["c4"](seed=2)
    x = torch.from_numpy(d["logits_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
    drafts = torch.from_numpy(d["drafts"]).to(dev)
    eager = ops.PreparedVerify([x], drafts)
    e = eager(0)
    torch.cuda.synchronize()
    want = (e.argmax.cpu().numpy().copy(), e.accept.cpu().numpy().copy(), e.logprobs.cpu().numpy().copy())
    print("[graph] capture c4 verify", flush=True)
    g, call = _capture(lambda: ops.PreparedVerify([x], drafts))
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        got = (call.out.argmax.cpu().numpy(), call.out.accept.cpu().numpy(), call.out.logprobs.cpu().numpy())
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b, err_msg=f"replay {r}")
        eager(0)
        torch.cuda.synchronize()
