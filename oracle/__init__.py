"""CPU oracle for the token-selection hot path. TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference's sampling and greedy-verify arithmetic so that the HIP path can be
checked against it on the same inputs. Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg
may import it, and only as the checker (or the timed CPU baseline), never as the product path: the product path in
`volundr-mlx_amd/volundr_amd` calls the HIP library and fails loudly when it is missing.

Modules:
  sampler_ref  - `Sampler.sample` / `uniform` / `accept` (volundr-mlx/sampler.py:58-156) with the uniform draw
                 supplied as an argument, plus the build-defined logprob and CDF-boundary diagnostics.
  verify_ref   - greedy verify: first-max argmax over [:vocab_valid], accept prefix, chosen-token logprob
                 (volundr-mlx/spec/specdec.py:326-336, volundr-mlx/scheduler.py:462-470,
                 volundr-mlx/spec/check_verify.py:27-30).

Pinning (what checks each function independently of its own formula) is listed in each module's header.
"""
