"""CPU oracle for the packed-ternary MoE decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, what the reference (maple-run) computes on the
hot path. The HIP kernels are compared against it, and it is the CPU
baseline ``bench.py`` times. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it; the shipped package never
does, and fails loudly when its HIP library is missing instead of falling back
here.

Modules
-------
``pack``     -- 2-bit / 4-bit packing, RTN quantisation, ternarisation
               (reference ``src/maple_run/pack.py:17-149``).
``kernels``  -- dequantised float64 closed forms of every hot-path kernel:
               ternary GEMV, router top-k, expert SwiGLU / GEMV / down-sum,
               MoE combine, RTN4 GEMV / embedding, RMSNorm, dispatch.
``decoder``  -- the synthetic decoder step (RoPE, decode GQA attention,
               decoder layer, lm_head) used for the full-model parity check.

How each function is pinned (against what fails if it is wrong) is listed in
the docstring of each function and tested in ``tests/test_oracle_*.py``.
"""
