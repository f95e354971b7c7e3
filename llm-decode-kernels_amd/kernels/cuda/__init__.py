"""The native W4A16 decode entry point under the reference's import path (`kernels.cuda`).

The reference keeps its hand-written CUDA decode kernel here (kernels/cuda/w4a16_cuda.py); callers
import `kernels.cuda.w4a16_cuda.w4a16_decode_cuda`. On MI355X the same name runs this build's
gfx950 HIP entry `ldk_w4a16_decode`; the package name is kept so such callers need no change.
"""
