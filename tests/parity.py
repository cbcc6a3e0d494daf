"""Parity rules shared by the GPU tests (the contract of the task):
  * token ids identical, except where the draw lies within 1e-6 of a CDF boundary, the top-p cut lies within 1e-6
    of a cumulative boundary, or the top-k cut splits a run of tied logits (argpartition is implementation-defined
    there); such rows are counted and reported;
  * logprobs within 1e-5 relative, with an absolute floor of 1e-10 (values below 1e-5 in magnitude are limited by
    float64 cancellation in the reference formula itself, e.g. log(p) for p = 1 - 1e-12);
  * keep counts identical unless the top-p cut is a boundary case.
"""
import numpy as np

from volundr_amd._lib import OUT_DRAW_BOUNDARY, OUT_TIMEOUT, OUT_TOPP_BOUNDARY

LP_RTOL = 1e-5
LP_ATOL = 1e-10


def check_sample(out, refs, label=""):
    ids = out.ids.cpu().numpy()
    lps = out.logprobs.cpu().numpy().astype(np.float64)
    fl = out.flags.cpu().numpy().astype(np.int64) & 0xFFFFFFFF
    keep = out.keep.cpu().numpy()
    boundary = 0
    for r, ref in enumerate(refs):
        assert not (fl[r] & OUT_TIMEOUT), f"{label} row {r}: timeout flag"
        soft = ref.kind == "sample" and (ref.draw_boundary or ref.topp_boundary or ref.topk_tie
                                         or fl[r] & (OUT_DRAW_BOUNDARY | OUT_TOPP_BOUNDARY))
        if ids[r] != ref.token:
            assert soft, f"{label} row {r}: token {ids[r]} != oracle {ref.token} (keep {keep[r]} vs {ref.keep})"
            boundary += 1
            continue
        if ref.kind == "sample" and not (ref.topp_boundary or fl[r] & OUT_TOPP_BOUNDARY or ref.topk_tie):
            assert keep[r] == ref.keep, f"{label} row {r}: keep {keep[r]} != oracle {ref.keep}"
        if ref.kind == "sample" and (ref.topp_boundary or ref.topk_tie):
            continue
        tol = LP_RTOL * abs(ref.logprob) + LP_ATOL
        assert abs(lps[r] - ref.logprob) <= tol, f"{label} row {r}: logprob {lps[r]} vs {ref.logprob}"
    return boundary
