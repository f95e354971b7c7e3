"""CPU oracle for the decode hot path: a numpy restatement of the reference's algorithms.

TEST INFRASTRUCTURE ONLY. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only as the checker (or, for `cpu_baseline`, as the timed
CPU path). The product package (`kernels.*`) never imports it and has no CPU fallback.

Modules and the reference code each one restates (paths relative to the reference repository):

- `oracle.quant`     int4 format and RTN quantizer, `kernels/quant.py:17-54`.
- `oracle.reference` dequantize / W4A16 matmul / RMSNorm / SwiGLU references,
                     `kernels/reference.py:9-45`, plus the byte formulas of
                     `kernels/rmsnorm.py:71-74` and `kernels/swiglu.py:64-65`.
- `oracle.fp8`       OCP e4m3 encode/decode, per-channel FP8 quantizer and W8A16 reference,
                     `kernels/fp8.py:21-39` and `tests/test_fp8.py:20`.
- `oracle.torch_cpu` the same references as torch ops on CPU tensors (the reference's own CPU
                     path, timed on all host cores by `bench.py`'s `cpu_baseline`), pinned
                     against the numpy modules above.

Every function is pinned by checks in `tests/test_oracle_*.py` that do not retype its formula:
the reference tests' known-answer values (`tests/test_quant.py:15-18,34-35`), hand-derived
known answers, invariants from the mathematics (round trips, error bounds, tie rounding,
clamping), float64 brute force on small shapes, and library routines that the reference itself
calls (torch's `float8_e4m3fn` cast, IEEE fp16 rounding). No function is left unpinned.
"""
