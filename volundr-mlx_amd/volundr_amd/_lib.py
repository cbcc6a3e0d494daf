"""ctypes binding of libvolundr_sampling.so (declarations: include/volundr_sampling.h).

There is no fallback: if the library is missing or fails to load, every call raises. Build it with
`python volundr-mlx_amd/volundr_amd/build.py` (or `__graft_entry__.build()`).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libvolundr_sampling.so"

VS_OK, VS_EINVAL, VS_EWORKSPACE, VS_EHIP = 0, -1, -2, -3
VS_F32, VS_BF16, VS_F16 = 0, 1, 2
VS_ROW_GREEDY = 1
VS_ROW_ARGMAX_VV = 2
VS_ROW_FORCE = 4
VS_ROW_HIST_PAIRS = 8
OUT_DRAW_BOUNDARY = 1 << 0
OUT_TOPP_BOUNDARY = 1 << 1
OUT_GREEDY = 1 << 3
OUT_NOFINITE = 1 << 4
OUT_COOP = 1 << 5
OUT_GATHER = 1 << 6
OUT_HIST_FULL = 1 << 7
OUT_FORCED = 1 << 8
OUT_UNSUPPORTED = 1 << 9
OUT_TIMEOUT = 1 << 31
DEBUG_FORCE_RADIX = 1
DEBUG_SPIN_LATER_BARRIERS = 2
DEBUG_WAIT_CLOCK = 4
DEBUG_NO_XCD_EXCHANGE = 8
DEBUG_FAKE_XCD_SPLIT = 16

# vs_row_params, 96 bytes (layout fixed by the C header)
ROW_DTYPE = np.dtype([
    ("temperature", "<f4"), ("repetition_penalty", "<f4"), ("frequency_penalty", "<f4"),
    ("presence_penalty", "<f4"), ("top_k", "<i4"), ("flags", "<u4"),
    ("top_p", "<f8"), ("min_p", "<f8"), ("u", "<f8"), ("hist_begin", "<i8"), ("hist_end", "<i8"),
    ("bias_begin", "<i4"), ("bias_end", "<i4"), ("supp_begin", "<i4"), ("supp_end", "<i4"),
    ("stop_begin", "<i4"), ("stop_end", "<i4"), ("vocab_valid", "<i4"), ("force_token", "<i4"),
])
assert ROW_DTYPE.itemsize == 96

# vs_row_state, 48 bytes: the per-request sampler state of vs_sample_batch_state
STATE_DTYPE = np.dtype([("rng", "<u8"), ("hist_off", "<i8"), ("hist_len", "<i4"), ("hist_cap", "<i4"),
                        ("produced", "<i4"), ("min_new_tokens", "<i4"), ("tab_off", "<i8"), ("tab_len", "<i4"),
                        ("hist_base", "<i4")])
assert STATE_DTYPE.itemsize == 48

ABI_VERSION = 10
EXPORTS = ("vs_sample_batch", "vs_sample_batch_state", "vs_state_fold", "vs_sample_workspace_bytes", "vs_verify_greedy",
           "vs_verify_workspace_bytes", "vs_topk_batch", "vs_draft_walk", "vs_draft_propose",
           "vs_draft_workspace_bytes", "vs_lmhead_verify_greedy", "vs_lmhead_workspace_bytes", "vs_lmhead_sample",
           "vs_lmhead_sample_workspace_bytes", "vs_set_spin_limit", "vs_workspace_init", "vs_last_error", "vs_version",
           "vs_sample_batch_noalloc", "vs_sample_noalloc_scratch_bytes", "vs_launch_floor", "vs_stream_read", "vs_xcd_ids", "vs_set_cooperative", "vs_set_debug")

_lib = None


class VsError(RuntimeError):
    pass


def load():
    """Load the library once; raise VsError if it is not there."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise VsError(f"{LIB_PATH} is missing: build it with volundr-mlx_amd/volundr_amd/build.py")
    L = ctypes.CDLL(str(LIB_PATH))
    vp, i32, i64, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_size_t
    L.vs_sample_batch.argtypes = [vp, i32, i32, i32, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    L.vs_sample_batch.restype = i32
    L.vs_sample_batch_noalloc.argtypes = [vp, i32, i32, i32, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    L.vs_sample_batch_noalloc.restype = i32
    L.vs_sample_noalloc_scratch_bytes.argtypes = []
    L.vs_sample_noalloc_scratch_bytes.restype = sz
    L.vs_sample_batch_state.argtypes = [vp, i32, i32, i32, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz,
                                        vp]
    L.vs_state_fold.argtypes = [vp, vp, vp, i64, vp, i32, vp]
    L.vs_state_fold.restype = i32
    L.vs_sample_batch_state.restype = i32
    L.vs_lmhead_verify_greedy.argtypes = [vp, i64, vp, i64, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, i64, vp, sz,
                                          vp]
    L.vs_lmhead_verify_greedy.restype = i32
    L.vs_stream_read.argtypes = [vp, sz, i32, vp, vp]
    L.vs_stream_read.restype = i32
    L.vs_lmhead_sample.argtypes = [vp, i64, vp, i64, i32, i32, i32, vp, vp, vp, vp, vp, vp, sz, vp]
    L.vs_lmhead_sample.restype = i32
    L.vs_lmhead_sample_workspace_bytes.argtypes = [i32]
    L.vs_lmhead_sample_workspace_bytes.restype = sz
    L.vs_lmhead_workspace_bytes.argtypes = [i32, i32]
    L.vs_lmhead_workspace_bytes.restype = sz
    L.vs_launch_floor.argtypes = [i32, i32, sz, i32, vp]
    L.vs_launch_floor.restype = i32
    L.vs_xcd_ids.argtypes = [vp, i32, i32, vp]
    L.vs_xcd_ids.restype = i32
    L.vs_set_debug.argtypes = [ctypes.c_uint]
    L.vs_set_debug.restype = i32
    L.vs_set_cooperative.argtypes = [i32]
    L.vs_set_cooperative.restype = i32
    L.vs_set_spin_limit.argtypes = [ctypes.c_uint]
    L.vs_set_spin_limit.restype = i32
    L.vs_topk_batch.argtypes = [vp, i32, i32, i32, i64, i32, vp, vp, vp, sz, vp]
    L.vs_topk_batch.restype = i32
    L.vs_draft_walk.argtypes = [vp, vp, i32, vp, vp, vp, i32, i32, vp, i32, i32, i32, vp, vp]
    L.vs_draft_walk.restype = i32
    L.vs_draft_propose.argtypes = [vp, i32, i32, i32, i32, i64, vp, vp, vp, i32, i32, vp, vp, vp, sz, vp]
    L.vs_draft_propose.restype = i32
    L.vs_draft_workspace_bytes.argtypes = [i32, i32, i32]
    L.vs_draft_workspace_bytes.restype = sz
    L.vs_sample_workspace_bytes.argtypes = [i32, i32]
    L.vs_sample_workspace_bytes.restype = sz
    L.vs_verify_greedy.argtypes = [vp, i32, i32, i32, i32, i64, i32, vp, vp, vp, vp, vp, sz, vp]
    L.vs_verify_greedy.restype = i32
    L.vs_verify_workspace_bytes.argtypes = [i32, i32, i32]
    L.vs_verify_workspace_bytes.restype = sz
    L.vs_workspace_init.argtypes = [vp, sz, vp]
    L.vs_workspace_init.restype = i32
    L.vs_last_error.argtypes = []
    L.vs_last_error.restype = ctypes.c_char_p
    L.vs_version.argtypes = []
    L.vs_version.restype = i32
    _lib = L
    return L


def check(rc: int, what: str):
    if rc != VS_OK:
        msg = load().vs_last_error().decode(errors="replace")
        raise VsError(f"{what} failed ({rc}): {msg}")
