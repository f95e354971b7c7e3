"""ctypes binding of kernels/bench/libldk_probe.so, the calibration kernels of the roofline
measurements (kernels/bench/probe.hip): an empty kernel, a contiguous read and the W4A16 M = 1
kernel's tile pattern as loads only, and K pieces with their cross-workgroup reductions. Used by
kernels.bench.profile_cases."""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

from kernels import _lib  # noqa: F401  (torch's HIP runtime first, as for the product library)

LIB_PATH = Path(__file__).with_name("libldk_probe.so")
_vp, _i64, _i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
_lib_probe = None


def _load():
    global _lib_probe
    if _lib_probe is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} not found: build it first (llm-decode-kernels_amd/build.py)")
        lib = ctypes.CDLL(str(LIB_PATH))
        lib.ldk_probe_empty.argtypes = [_i32, _i32, _vp]
        lib.ldk_probe_stream.argtypes = [_vp, _i64, _i32, _vp, _vp]
        lib.ldk_probe_tile.argtypes = [_vp, _i32, _i32, _vp, _vp]
        lib.ldk_probe_piece.argtypes = [_i32, _i32, _vp, _i32, _i32, _vp, _vp, _vp]
        _lib_probe = lib
    return _lib_probe


def _stream():
    return _vp(torch.cuda.current_stream().cuda_stream)


def _ok(st: int, what: str):
    if st:
        raise RuntimeError(f"{what}: status {st}")


def empty(workgroups: int = 1, threads: int = 64):
    _ok(_load().ldk_probe_empty(workgroups, threads, _stream()), "probe_empty")


def stream(src: torch.Tensor, sink: torch.Tensor, loads: int = 1):
    assert src.is_cuda and src.is_contiguous() and src.nbytes % 16 == 0
    grid = -(-src.nbytes // (16 * 256 * loads))
    assert sink.dtype == torch.int32 and sink.numel() >= grid
    _ok(_load().ldk_probe_stream(_vp(src.data_ptr()), src.nbytes, loads, _vp(sink.data_ptr()),
                                 _stream()), "probe_stream")


def tile(qweight: torch.Tensor, sink: torch.Tensor):
    R, N = qweight.shape
    assert qweight.dtype == torch.int32 and qweight.is_contiguous() and R % 192 == 0 and N % 32 == 0
    assert sink.dtype == torch.int32 and sink.numel() >= N // 32 * 384
    _ok(_load().ldk_probe_tile(_vp(qweight.data_ptr()), R, N, _vp(sink.data_ptr()), _stream()),
        "probe_tile")


PIECE_SHAPES = {"whole32x192": 0, "piece64x64": 1, "piece256x16": 2, "piece256x4": 3}
PIECE_REDUCTIONS = {"none": 0, "store": 1, "fixed_atomic": 2, "f32_atomic": 3}


def piece(shape: str, red: str, qweight: torch.Tensor, ws: torch.Tensor, out: torch.Tensor):
    """qweight [R, N] int32 read as `shape` pieces, partials met by `red` (probe.hip)."""
    R, N = qweight.shape
    assert qweight.dtype == torch.int32 and qweight.is_contiguous()
    assert ws.nbytes >= N * 8 + 64 * N * 4 and out.dtype == torch.float16 and out.numel() >= N
    _ok(_load().ldk_probe_piece(PIECE_SHAPES[shape], PIECE_REDUCTIONS[red], _vp(qweight.data_ptr()), R, N,
                                _vp(ws.data_ptr()), _vp(out.data_ptr()), _stream()), "probe_piece")
