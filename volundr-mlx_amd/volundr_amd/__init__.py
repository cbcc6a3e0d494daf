"""volundr_amd - MI355X-native token selection for volundr-mlx (sampler.py path, greedy speculative verify, DFlash2 candidate walk).

    from volundr_amd import Sampling, Sampler, sample_batch, verify_greedy

Sampling / Sampler / Budget keep the reference's call surface (volundr-mlx/session.py:439-478,
volundr-mlx/sampler.py:18-156); sample_batch / verify_greedy are the batched device entry points. The arithmetic
runs in libvolundr_sampling.so (hand-written HIP for gfx950, C ABI in include/volundr_sampling.h).
"""
from .session import Sampling
from .sampler import Budget, Sampler, sample_rows_for
from .ops import (DeviceRows, PackedRows, SampleOut, VerifyOut, draft_propose, draft_walk, emitted, lmhead_sample, lmhead_verify_greedy,
                  pack_rows,
                  sample_batch, sample_rows, topk_batch, verify_greedy)
from .state import DeviceSamplers
from ._lib import LIB_PATH, VsError

__all__ = ["Sampling", "Sampler", "Budget", "sample_rows_for", "sample_batch", "sample_rows", "pack_rows",
           "PackedRows", "DeviceRows", "SampleOut", "VerifyOut", "verify_greedy", "emitted", "DeviceSamplers", "topk_batch", "draft_walk", "draft_propose", "lmhead_verify_greedy", "lmhead_sample",
           "LIB_PATH", "VsError"]
