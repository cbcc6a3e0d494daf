"""CPU checks of the boundary: the C-ABI library loads and exports every symbol the header declares; host packing
follows sampler.py's parameter semantics. No device calls."""
import re
from pathlib import Path

import numpy as np
import pytest

from volundr_amd import _lib, pack_rows
from volundr_amd.session import Sampling

ROOT = Path(__file__).resolve().parent.parent


def test_header_symbols_exported():
    L = _lib.load()
    hdr = (ROOT / "include" / "volundr_sampling.h").read_text()
    names = set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(vs_\w+)\s*\(", hdr, re.M))
    assert names == set(_lib.EXPORTS)
    for n in names:
        assert hasattr(L, n)
    assert L.vs_version() == _lib.ABI_VERSION
    assert L.vs_sample_workspace_bytes(16, 163840) > 0


def test_row_struct_size_matches_header():
    hdr = (ROOT / "include" / "volundr_sampling.h").read_text()
    assert "96 bytes" in hdr and _lib.ROW_DTYPE.itemsize == 96
    assert "48 bytes" in hdr and _lib.STATE_DTYPE.itemsize == 48
    assert f"increments on any signature or struct change): {_lib.ABI_VERSION}." in hdr


def test_errors_without_device_calls():
    L = _lib.load()
    assert L.vs_sample_batch(0, 0, -1, 10, 10, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) == _lib.VS_EINVAL
    assert b"B < 0" in L.vs_last_error()
    assert L.vs_sample_batch(0, 0, 0, 10, 10, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) == _lib.VS_OK
    assert L.vs_verify_greedy(0, 0, 1, 0, 10, 10, 10, 0, 0, 0, 0, 0, 0, 0) == _lib.VS_EINVAL
    assert L.vs_sample_batch_state(0, 0, 1, 10, 10, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0) == _lib.VS_EINVAL
    assert b"null state" in L.vs_last_error()


def test_pack_rows_semantics():
    sps = [Sampling(top_k=None, temperature=0.7, logit_bias=[(3, 1.0), (1, 2.0), (3, 0.5), (99, 1.0)],
                    suppress_tokens=[4, 4, 50, -1], stop_token_ids=[2], min_new_tokens=1),
           Sampling(top_k=-3, temperature=1e-7)]
    p = pack_rows(sps, [0.25, 0.5], V=10, histories=[[1, 1, 2], None], produced=[0, 5], extras=[[(3, -1.0)], None])
    r0, r1 = p.params
    assert r0["top_k"] == 0 and r0["flags"] == 0 and r0["temperature"] == np.float32(0.7)
    assert r1["top_k"] == 1 and r1["flags"] == _lib.VS_ROW_GREEDY  # temperature < 1e-6 -> greedy
    # biases sorted by id, equal ids in application order (extra first), ids >= V dropped
    b = slice(r0["bias_begin"], r0["bias_end"])
    assert p.bias_ids[b].tolist() == [1, 3, 3, 3] and p.bias_vals[b].tolist() == [2.0, -1.0, 1.0, 0.5]
    assert p.mask_ids[r0["supp_begin"]:r0["supp_end"]].tolist() == [4, 9]   # -1 wraps to V-1
    assert p.mask_ids[r0["stop_begin"]:r0["stop_end"]].tolist() == [2]
    assert r1["stop_end"] == r1["stop_begin"]
    assert p.hist[r0["hist_begin"]:r0["hist_end"]].tolist() == [1, 1, 2] and r1["hist_end"] == r1["hist_begin"]
    with pytest.raises(ValueError):
        pack_rows([Sampling()], [0.1, 0.2], V=10)


def test_no_cpu_fallback():
    import torch

    from volundr_amd import sample_batch, verify_greedy

    with pytest.raises(ValueError):
        sample_batch(torch.zeros(1, 10), [Sampling()], [0.5])
    with pytest.raises(ValueError):
        verify_greedy(torch.zeros(1, 2, 10), torch.zeros(1, 1, dtype=torch.int32))


def test_budget_logic():
    from volundr_amd.sampler import Budget

    b = Budget(4, 0.0, [1, 2, 7], 7, 8)   # <think>=7 open in the prompt tail
    assert b.open == 0
    assert [b.act(i)[0] for i in range(4)] == ["none"] * 4
    assert b.act(4) == ("force", 8)
    assert b.act(5) == ("bias", [(7, -np.inf)])
    b = Budget(10, 1.5, [7, 8], 7, 8)     # closed in the prompt: never opens
    assert b.open is None and b.act(20) == ("none", None)
    b = Budget(10, 1.5, [], 7, 8)
    b.accept(0, 7)
    assert b.open == 1 and b.act(9) == ("bias", [(8, 1.5)]) and b.act(5) == ("none", None)


def test_draft_entry_points_reject_bad_shapes_without_device_calls():
    L = _lib.load()
    # more than 8 slots, more than 16 candidates, rank not a multiple of 16: rejected before any launch
    assert L.vs_draft_walk(1, 1, 16, 1, 4, 4, 10, 256, 1, 1, 9, 16, 1, 0) == _lib.VS_EINVAL
    assert L.vs_draft_walk(1, 1, 17, 1, 4, 4, 10, 256, 1, 1, 7, 17, 1, 0) == _lib.VS_EINVAL
    assert L.vs_draft_walk(1, 1, 16, 1, 4, 4, 10, 250, 1, 1, 7, 16, 1, 0) == _lib.VS_EINVAL
    assert L.vs_draft_walk(0, 1, 16, 1, 4, 4, 10, 256, 1, 1, 7, 16, 1, 0) == _lib.VS_EINVAL
    assert L.vs_draft_walk(1, 1, 16, 1, 4, 4, 10, 256, 1, 0, 7, 16, 1, 0) == _lib.VS_OK  # n = 0: nothing to do
    assert L.vs_topk_batch(1, 0, 1, 10, 10, 0, 1, 1, 1, 1 << 20, 0) == _lib.VS_EINVAL  # k < 1
    assert L.vs_draft_workspace_bytes(2, 7, 163840) > L.vs_sample_workspace_bytes(14, 163840)
    assert L.vs_draft_propose(1, 0, 1, 7, 10, 10, 1, 4, 4, 10, 256, 1, 1, 0, 0, 0) == _lib.VS_EINVAL  # null ws


def test_token_history_is_list_like_and_packs_like_a_list():
    from volundr_amd.sampler import TokenHistory

    rng = np.random.default_rng(5)
    lists = [rng.integers(0, 1000, n).tolist() for n in (0, 1, 63, 64, 65, 300)]
    hs = []
    for lst in lists:
        h = TokenHistory()
        for t in lst:
            h.append(t)
        assert len(h) == len(lst) and list(h) == lst and h == lst and np.asarray(h).tolist() == lst
        if lst:
            assert h[0] == lst[0] and h[-1] == lst[-1] and h[1:4] == lst[1:4]
        hs.append(h)
    assert TokenHistory(lists[-1]) == lists[-1]
    with pytest.raises(ValueError):
        TokenHistory().append(-1)
    with pytest.raises(ValueError):
        TokenHistory().append(2**31)
    sps = [Sampling(temperature=float(rng.uniform(0.1, 2)), top_k=int(rng.integers(-2, 50)),
                    top_p=float(rng.uniform(0.1, 1)), repetition_penalty=1.1,
                    logit_bias=[(int(rng.integers(0, 1000)), 0.5)], suppress_tokens=[7] * (i % 2))
           for i in range(len(lists))]
    u = rng.random(len(lists))
    a = pack_rows(sps, u, V=1000, histories=lists)
    b = pack_rows(sps, u, V=1000, histories=hs)
    assert a.params.tobytes() == b.params.tobytes()
    for f in ("hist", "bias_ids", "bias_vals", "mask_ids"):
        assert np.array_equal(getattr(a, f), getattr(b, f))
    assert pack_rows([], [], V=10).params.size == 0


def test_cooperative_setting_is_per_thread_and_restorable():
    import threading

    L = _lib.load()
    assert L.vs_set_cooperative(1) == 0
    seen = []
    th = threading.Thread(target=lambda: seen.append(L.vs_set_cooperative(0)))
    th.start()
    th.join()
    assert seen == [0]  # the other thread's own setting was still the default
    assert L.vs_set_cooperative(0) == 1  # this thread's setting survived the other thread's call


def test_pack_rows_hist_pairs():
    """The (id, count) table form: ids ascending and unique, counts from the raw history or a counts dict (the same
    table either way), the flag set, the range at an even word."""
    from volundr_amd._lib import VS_ROW_HIST_PAIRS

    hist = [5, 3, 5, 9, 3, 5, 200]
    counts = {}
    for t in hist:
        counts[t] = counts.get(t, 0) + 1
    sps = [Sampling(repetition_penalty=1.2), Sampling(repetition_penalty=1.2)]
    a = pack_rows(sps, [0.1, 0.2], 100, [[1, 2, 3], hist], hist_pairs=True)
    b = pack_rows(sps, [0.1, 0.2], 100, [{1: 1, 2: 1, 3: 1}, counts])
    for p in (a, b):
        r = p.params[1]
        assert int(r["flags"]) & VS_ROW_HIST_PAIRS and int(r["hist_begin"]) % 2 == 0
        assert p.hist[r["hist_begin"]:r["hist_end"]].tolist() == [3, 2, 5, 3, 9, 1, 200, 1]
    assert np.array_equal(a.hist, b.hist) and np.array_equal(a.params, b.params)
    c = pack_rows(sps[:1], [0.1], 100, [[]], hist_pairs=True)
    assert not int(c.params[0]["flags"]) & VS_ROW_HIST_PAIRS and c.params[0]["hist_end"] == c.params[0]["hist_begin"]
