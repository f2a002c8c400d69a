"""CPU oracle for the qwen3_5 MTP speculative-decode step -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithms of the reference path
(giapnguyen74/lollm `src/qwen3_5/*.py`, `src/generate.py`, `src/attention.py`) so
that the HIP product in `lollm_amd` can be checked against it on identical inputs.

Rules that bind this package:
  * Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
    may import it, and only as the checker or the timed CPU baseline.  The product
    (`lollm_amd`) never imports it and has no CPU fallback.
  * `qwen3_5_ref.py` is a torch-on-CPU restatement of the reference's float math.
  * `sampler_ref.c` (built by `oracle/Makefile` into `oracle/_build/`) is the exact
    integer/IEEE restatement of the build's rejection sampler and Philox stream; the
    GPU sampler must match it bit for bit.

How each function is pinned (golden vectors, closed forms, invariants) is listed in
the header of each module.
"""
