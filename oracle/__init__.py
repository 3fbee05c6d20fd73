"""CPU oracle for the FP8 decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the arithmetic of the reference's torch golden paths
for block-scaled FP8 linears, the MoE expert layer and the DSA lightning indexer + top-k.
It is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it. ``tilert_amd`` never imports it and
fails loudly when its HIP library is missing.

Modules
-------
fp8        OCP e4m3fn codec restated from the format definition (numpy); pins torch's cast.
reference  torch-CPU restatement of the reference goldens (act_quant, weight_dequant,
           fp8_gemm, linear, MoE gate/up+SwiGLU and down+weighted sum, indexer scores,
           top-k). Each function cites the reference file:line it follows.
brute      fp64 brute-force evaluations on tiny inputs (pure numpy loops), used to pin
           ``reference`` against what the mathematics fixes.

Parity pins (what checks each function): see the docstring of every function and the
tests under ``tests/test_oracle_*.py``.  Every function here has at least one check that
is independent of its own formula (exhaustive codec comparison, closed forms, fp64 brute
force, invariants); none is "parity unpinned".
"""
