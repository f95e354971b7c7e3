"""`w4a16_decode_cuda`: the native W4A16 decode entry (`ldk_w4a16_decode`, M <= 16 rows).

Drop-in for the reference's kernels/cuda/w4a16_cuda.py:45-56 (the name and module path are the
reference's; the kernel is this build's gfx950 HIP code). Contract: same arguments as
`w4a16_matmul`, at most 16 rows, RuntimeError for more (the reference's TORCH_CHECK, tested at
tests/test_w4a16_cuda.py:43-45). `split_k` is the number of workgroups splitting K per column
tile; None (or 0) takes the library's table, which needs no timing at first call, where the
reference times each factor once per shape (w4a16_cuda.py:29-42). Split partials meet in the
library workspace, inside the one launch, instead of a zero-filled fp32 buffer and a cast launch.
"""

from __future__ import annotations

import torch

from kernels import _lib

_split_choice: dict[tuple, int] = {}  # (row bucket, N, K, bias) -> split_k asked for


def w4a16_decode_cuda(x, qweight, scales, zeros, group_size=128, bias=None, split_k=None):
    """y = x @ dequant(W).T for M <= 16 rows. Same contract as kernels.w4a16.w4a16_matmul."""
    K = x.shape[-1]
    N = qweight.shape[1]
    dev = _lib.require_gpu(x, qweight, scales, zeros, bias, what="w4a16_decode_cuda")
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    b = None if bias is None else bias.to(torch.float16).contiguous()
    qw, s, z = qweight.contiguous(), scales.contiguous(), zeros.contiguous()
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w4a16_decode(
            _lib.ptr(x2), x2.stride(0), _lib.ptr(qw), _lib.ptr(s), _lib.ptr(z), _lib.ptr(b),
            _lib.ptr(out), out.stride(0), M, N, K, group_size, int(split_k or 0), ws, ws_bytes,
            _lib.stream(dev))
    if st == _lib.ERR_UNSUPPORTED:
        raise RuntimeError(_lib.load().ldk_last_error().decode())
    _lib.check(st, "w4a16_decode_cuda")
    if split_k:
        _split_choice[(min(1 << (M - 1).bit_length(), 16), N, K, bias is not None)] = int(split_k)
    return out.view(*x.shape[:-1], N)


# The reference's choice export for this entry (w4a16_cuda.py:59-72): keys "m,N,K,bias".
def split_choices() -> dict:
    return {str(k): v for k, v in _split_choice.items()}


def export_choices() -> dict:
    return {",".join(map(str, k)): v for k, v in _split_choice.items()}


def import_choices(choices: dict) -> None:
    for key, split in choices.items():
        m, n, k, b = key.split(",")
        _split_choice[(int(m), int(n), int(k), b == "True")] = int(split)
