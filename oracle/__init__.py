"""CPU oracle for the MI355X PJRT plugin's hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference (Lazarus-931/mccl-jax)
computes for the one-GPU jitted-StableHLO path, so the HIP kernels can be
checked against it.  It is a checker, never a product path: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it.  The plugin and the kernel library never call into it, and they fail
loudly when their HIP build is missing instead of falling back here.

The reference's numerical oracle is JAX's XLA:CPU backend running the same
jitted StableHLO (docs/ops.md:7-10).  JAX/jaxlib are a third-party dependency
that is absent from /root/reference and from this image, with no version
pinned anywhere in the reference, so the functions here restate
the published semantics of the StableHLO ops (and JAX's lowering of the
config functions) in numpy: fp64 for floating-point truth, exact integer /
bit arithmetic for bf16 rounding, argmax and indexing, and strictly
sequential fp32 accumulation for scatter-add.  The reference holds no golden
vectors or known-answer tests for this path (its only KATs are the
out-of-scope collective smokes), so every function is pinned instead by the
closed forms, invariants and brute-force checks in tests/test_oracle_pins.py.

Modules
  bf16     exact bf16 / f16 encode-decode (round to nearest even)
  ops      restatements of the config functions and of each StableHLO op
  inputs   seeded input generators (numpy PCG64), byte-identical to the GPU
  native   ctypes bridge to the C restatement in oracle/c (sequential
           scatter-add, bit-exact argmax) for full-size checks
"""

from . import bf16, inputs, ops  # noqa: F401
