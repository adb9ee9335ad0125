"""CPU oracle for the bound-propagation hot path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU with plain PyTorch
fp32/fp64 arithmetic, the reference algorithms that the HIP backend replaces
(IBP forward trace, CROWN backward, ReLU relaxation, concretization,
alpha/alpha-beta optimisation, BaB node-batch evaluation). Each function cites
the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker or as the CPU
baseline being timed -- never as the product path. ``boundflow_amd`` never
imports it.

Pinning: every function here is checked by ``tests/test_oracle_*.py`` against
golden vectors written by ``tests/golden/make_golden.py`` from the reference
implementation itself (imported in the build container only), against the
fixtures the reference's own tests hold, and against closed forms /
brute-force checks on tiny inputs.
"""
