"""The sampling and verify entry points captured in a HIP graph (torch.cuda.CUDAGraph on a side stream whose
workspace was zeroed before the capture, so that only kernels are recorded): every replay, with eager work of the
same library between replays, returns exactly the eager results: the kernels leave their workspaces ready for the
next call."""
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


def _replay_alternating(g, buf, inputs, wants, got_fn, label):
    """Replays with the captured input buffer refilled between replays (eager copies on the current stream): each
    replay must match the eager results for the input it ran on."""
    for r in range(6):
        j = r % len(inputs)
        buf.copy_(inputs[j])
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(got_fn(), wants[j]):
            np.testing.assert_array_equal(a, b, err_msg=f"{label} replay {r} (input {j})")


def test_verify_graph_replays_new_inputs(dev):
    """The tags of the verify kernel's exchanged words come from epochs in the workspace, so replays of a captured
    call (three calls per replay here) on new logits never take words an earlier replay left."""
    xs, wants = [], []
    d0 = synth.CONFIGS["c2"](seed=5)
    drafts = torch.from_numpy(d0["drafts"]).to(dev)
    for seed in (5, 6):
        d = synth.CONFIGS["c2"](seed=seed)
        x = torch.from_numpy(d["logits_bf16"].view(np.int16)).to(dev).view(torch.bfloat16)
        e = ops.PreparedVerify([x], drafts)(0)
        torch.cuda.synchronize()
        xs.append(x)
        wants.append((e.argmax.cpu().numpy().copy(), e.accept.cpu().numpy().copy(), e.logprobs.cpu().numpy().copy()))
    assert not np.array_equal(wants[0][0], wants[1][0])
    buf = xs[0].clone()
    print("[graph] capture c2 verify, refilled input", flush=True)
    g, call = _capture(lambda: ops.PreparedVerify([buf], drafts))
    _replay_alternating(g, buf, xs, wants, lambda: (call.out.argmax.cpu().numpy(), call.out.accept.cpu().numpy(),
                                                    call.out.logprobs.cpu().numpy()), "verify")


def test_lmhead_graph_replays_new_inputs(dev):
    """The fused head's in-launch merge (tagged partials, per-position epochs in the workspace) under graph replays
    with new hidden states between replays."""
    B, T, K, N = 1, 17, 1024, 5003
    gen = torch.Generator(device=dev).manual_seed(9)
    W = (torch.randn(N, K, generator=gen, device=dev) / 8).to(torch.bfloat16)
    hs = [torch.randn(B, T, K, generator=gen, device=dev).to(torch.bfloat16) for _ in range(2)]
    drafts = torch.randint(0, N, (B, T - 1), generator=gen, device=dev, dtype=torch.int32)
    wants = []
    for h in hs:
        o = ops.lmhead_verify_greedy(h, W, drafts)
        torch.cuda.synchronize()
        wants.append((o.argmax.cpu().numpy().copy(), o.accept.cpu().numpy().copy(), o.logprobs.cpu().numpy().copy()))
    assert not np.array_equal(wants[0][0], wants[1][0])
    buf = hs[0].clone()
    out = ops.VerifyOut(torch.empty(B, T, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev),
                        torch.empty(B, T, dtype=torch.float32, device=dev))
    print("[graph] capture lm_head verify, refilled hidden states", flush=True)
    g, _ = _capture(lambda: (lambda i: ops.lmhead_verify_greedy(buf, W, drafts, out=out)))
    _replay_alternating(g, buf, hs, wants, lambda: (out.argmax.cpu().numpy(), out.accept.cpu().numpy(),
                                                    out.logprobs.cpu().numpy()), "lm_head")
