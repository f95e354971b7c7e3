"""ctypes binding of libldk_amd.so, the gfx950 HIP kernel library (C ABI in include/ldk.h).

Every public op of this package calls into this library with raw device pointers and the torch
current stream. There is no CPU path: if the library is missing or the tensors are not on a
ROCm GPU, the ops raise.

The library links the HIP runtime by soname (libamdhip64.so.7). torch is imported first so that
the runtime torch already loaded satisfies that soname: one HIP runtime per process, so streams
and device pointers are shared with torch.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).with_name("libldk_amd.so")

# Status codes (enum ldk_status).
OK, ERR_INVALID, ERR_ALIGN, ERR_UNSUPPORTED, ERR_LAUNCH = 0, 1, 2, 3, 4
# dtype codes (enum ldk_dtype).
F16, BF16, F32 = 0, 1, 2
# flags (enum ldk_flags).
FACTORED, EXACT, PATH_VALU, PATH_MFMA, PATH_GEMM = 1, 2, 4, 8, 64
CPW_FLAGS = {1: 16, 2: 32, 4: 48}  # chunks of loads per wave and round (LDK_CPW_*)
CPW_MASK = 48

_DTYPE_CODE = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}

_vp, _i64, _i32, _f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
_ip = ctypes.POINTER(ctypes.c_int)

# name -> argtypes, mirroring include/ldk.h.
SIGNATURES = {
    "ldk_abi_version": [],
    "ldk_last_error": [],
    "ldk_int4_pack": [_vp, _vp, _i64, _i64, _vp],
    "ldk_int4_unpack": [_vp, _vp, _i64, _i64, _vp],
    "ldk_quantize_rtn": [_vp, _i32, _vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "ldk_w4a16_dequant": [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp],
    "ldk_workspace_bytes": [],
    "ldk_w4a16_matmul": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32,
                         _i32, _i32, _i32, _vp, _i64, _vp],
    "ldk_w4a16_decode": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32,
                         _vp, _i64, _vp],
    "ldk_w4a16_config": [_i64, _i64, _i64, _i32, _ip, _ip, _ip],
    "ldk_w4a16_kernel_name": [_i64, _i64, _i64, _i32, ctypes.c_char_p, _i64],
    "ldk_w4a16_matmul_noalloc": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32,
                                 _i32, _i32, _i32, _vp],
    "ldk_w4a16_rmsnorm_matmul": [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _i64, _i64,
                                 _i32, _vp, _i64, _vp],
    "ldk_w4a16_swiglu_matmul": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _vp, _i64, _vp],
    "ldk_fp8_quantize": [_vp, _i32, _vp, _vp, _i64, _i64, _vp],
    "ldk_fp8_dequant": [_vp, _vp, _i32, _vp, _i64, _i64, _vp],
    "ldk_w8a16_swiglu_matmul": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp],
    "ldk_w4a16_row_stats_count": [_i64, _i64, _i32],
    "ldk_w4a16_matmul_residual_stats": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i32,
                                        _vp, _i64, _vp],
    "ldk_w4a16_rmsnorm_stats_matmul": [_vp, _vp, _i32, _vp, _f32, _vp, _vp, _vp, _vp, _vp, _i64,
                                       _i64, _i32, _vp, _i64, _vp],
    "ldk_w8a16_rmsnorm_matmul": [_vp, _vp, _vp, _vp, _f32, _vp, _vp, _vp, _vp, _i64, _i64, _vp,
                                 _i64, _vp],
    "ldk_w8a16_matmul": [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _i32, _i32,
                         _vp, _i64, _vp],
    "ldk_w8a16_config": [_i64, _i64, _i64, _ip, _ip, _ip],
    "ldk_rmsnorm": [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _f32, _vp],
    "ldk_swiglu": [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _vp],
    "ldk_greedy_step": [_vp, _i32, _i64, _vp, _vp, _i64, _vp, _vp],
    "ldk_f16_gemv": [_vp, _vp, _i64, _vp, _i64, _i64, _i32, _vp],
    "ldk_f16_rmsnorm_gemv": [_vp, _vp, _vp, _f32, _vp, _i64, _vp, _i64, _i64, _i32, _vp],
    "ldk_decode_attention": [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _f32, _vp, _vp, _i32,
                             _vp],
    "ldk_decode_attention_ranges": [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _i64, _i64, _f32, _vp, _vp,
                                    _i32, _vp],
    "ldk_prefill_attention": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64,
                              _f32, _vp],
    "ldk_w4a16_attn_matmul_residual_stats": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                             _i64, _i64, _i32, _vp, _i64, _vp],
    "ldk_w8a16_attn_matmul": [_vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp],
    "ldk_w4a16_matmul_swiglu_applies": [_i64, _i64, _i64, _i32],
    "ldk_w4a16_matmul_swiglu": [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i32, _vp, _i64,
                                _vp],
    "ldk_w8a16_matmul_swiglu_applies": [_i64, _i64, _i64],
    "ldk_w8a16_matmul_swiglu": [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp],
}

_lock = threading.Lock()
_lib = None


class NativeLibraryMissing(RuntimeError):
    """libldk_amd.so has not been built (run `python -c "import __graft_entry__ as g; g.build()"`
    or `python llm-decode-kernels_amd/build.py`)."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library with argument/return types set."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryMissing(f"{LIB_PATH} not found: build it first")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = {"ldk_last_error": ctypes.c_char_p,
                              "ldk_workspace_bytes": ctypes.c_int64,
                              "ldk_w4a16_row_stats_count": ctypes.c_int64}.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Raise for a non-zero status: ValueError for bad arguments, RuntimeError otherwise (the
    reference's native extension raises RuntimeError from TORCH_CHECK)."""
    if status == OK:
        return
    msg = (load().ldk_last_error() or b"").decode(errors="replace")
    if status in (ERR_INVALID, ERR_ALIGN):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


class _TensorPtr(ctypes.c_void_p):
    """A device pointer argument that keeps its tensor alive. ctypes holds the argument objects
    until the foreign call returns, so a temporary such as `ptr(t.contiguous())` cannot go back
    to torch's caching allocator (and be handed to the next temporary of the same call) before
    the launch is enqueued; after that, the allocator's stream ordering protects it."""

    __slots__ = ("tensor",)


def ptr(t: torch.Tensor | None):
    if t is None:
        return None
    p = _TensorPtr(t.data_ptr())
    p.tensor = t
    return p


def stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float16, bfloat16 or float32") from None


# Most byte ranges one launch warms (csrc/warm.h, kWarmMax).
WARM_MAX_RANGES = 8


def warm_list(warm, what: str) -> list:
    """The non-empty tensors of a launch's warm ranges, checked: at most WARM_MAX_RANGES, each
    contiguous."""
    warm = [t for t in warm if t.numel()]
    if len(warm) > WARM_MAX_RANGES:
        raise ValueError(f"{what}: at most {WARM_MAX_RANGES} warm ranges")
    for t in warm:
        if not t.is_contiguous():
            raise ValueError(f"{what}: warm tensors must be contiguous")
    return warm


def warm_arrays(warm: list):
    """The C arrays of the warm tensors' device addresses and byte sizes."""
    wp = (ctypes.c_void_p * max(1, len(warm)))(*[t.data_ptr() for t in warm])
    wb = (ctypes.c_int64 * max(1, len(warm)))(*[t.numel() * t.element_size() for t in warm])
    return wp, wb


def require_gpu(*tensors: torch.Tensor | None, what: str) -> torch.device:
    """All given tensors must live on one ROCm GPU. There is no CPU implementation."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(f"{what}: tensors must be on a ROCm GPU (got {t.device}); "
                               "this library has no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"{what}: tensors on different devices ({dev} and {t.device})")
    if dev is None:
        raise RuntimeError(f"{what}: no tensor given")
    return dev


def on_gpu(*tensors: torch.Tensor | None, what: str):
    """For the weight-format routines, which the reference writes as device-agnostic torch code
    (kernels/quant.py:20-49, kernels/fp8.py:25-35) and its tests call on CPU tensors: returns
    (run_device, home_device, tensors on run_device). Tensors on a GPU stay there; CPU tensors are
    copied to the current ROCm GPU, where the HIP kernel runs, and the caller moves its results
    back to `home_device`. Without a visible GPU this raises: there is no CPU implementation."""
    given = [t for t in tensors if t is not None]
    if not given:
        raise RuntimeError(f"{what}: no tensor given")
    home = given[0].device
    if any(t.device != home for t in given):
        raise RuntimeError(f"{what}: tensors on different devices")
    if home.type == "cuda":
        return home, home, list(tensors)
    if home.type != "cpu" or not torch.cuda.is_available():
        raise RuntimeError(f"{what}: needs a ROCm GPU to run its HIP kernel (got {home} tensors "
                           "and no visible GPU); this library has no CPU path")
    run = torch.device("cuda", torch.cuda.current_device())
    return run, home, [None if t is None else t.to(run) for t in tensors]


_workspaces: dict[int, torch.Tensor] = {}


def workspace(dev: torch.device):
    """(pointer, bytes) of this device's split-K workspace: allocated zero-filled on first use and
    kept for the life of the process. Its counters are reset by the kernels themselves, so it is
    valid for every later call, including calls replayed from a captured graph. Make the first
    call (which allocates) outside graph capture. Calls sharing it must be stream-ordered."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _workspaces.get(idx)
    if ws is None:
        # Allocated under capture, the buffer would come from the graph's private memory pool and
        # outlive the graph it belongs to (and its zero fill would be a node of that graph).
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                f"the split-K workspace of cuda:{idx} is allocated by the first library call on that "
                "device, which must not be under graph capture: run the op once before capturing "
                "(as a warm-up), or call kernels._lib.workspace(device) first")
        nbytes = int(load().ldk_workspace_bytes())
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=torch.device("cuda", idx))
        _workspaces[idx] = ws
    return ctypes.c_void_p(ws.data_ptr()), ws.numel()


class device_guard:
    """Make `dev` current for the duration of a launch when it is not already."""

    def __init__(self, dev: torch.device):
        self.dev = dev
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.dev.index is not None and self.dev.index != cur:
            self.prev = cur
            torch.cuda.set_device(self.dev.index)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False
