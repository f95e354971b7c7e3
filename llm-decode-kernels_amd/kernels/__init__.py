"""MI355X (gfx950) decode hot path of llm-decode-kernels: W4A16 and FP8 weight-only matmuls,
fused RMSNorm(+residual) and fused SwiGLU, as hand-written HIP kernels behind a C ABI.

The modules keep the reference's names and call signatures (`kernels.quant`, `kernels.w4a16`,
`kernels.fp8`, `kernels.rmsnorm`, `kernels.swiglu`), so callers written against the reference
import them unchanged. All ops run on the GPU only; see `kernels._lib`.
"""
