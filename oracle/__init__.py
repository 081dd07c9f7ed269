"""CPU oracle for the GRBeam shared-prefix decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU, the arithmetic of the
reference GRBeam path (Greek-Guardian/Kadllm) and of the third-party
Qwen3.5 layer math that path depends on.  It exists to check the HIP
implementation in ``kadllm_amd``; it is never the thing measured or shipped.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package must not import, call or
fall back to anything here.

Modules
-------
ops_ref     gated delta (recurrent and chunked), causal conv1d, prefix attention
grbeam_ref  fixed-depth beam search selection and an exhaustive brute force
qwen35_ref  Qwen3.5 hybrid text model: full forward, prefill snapshot, suffix decode

Every function cites the reference file:line it follows.  Pinning of each
function (golden vectors, library routines, closed forms) lives in
``tests/test_oracle_*.py``.
"""
