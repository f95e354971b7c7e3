"""ldk_w4a16_matmul_noalloc (the allocation-free W4A16 entry, split-K partials in a library-owned
device array) against ldk_w4a16_matmul with a caller-provided workspace, through the C ABI:
bit-identical outputs on consecutive calls that share the array (the second with a smaller
input), and an explicit split whose partials exceed the array rejected with a clear error."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from kernels import _lib
from kernels.bench import cases
from oracle import quant as oq

pytestmark = pytest.mark.gpu

SCRATCH = int(re.search(r"#define LDK_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)",
                        (Path(__file__).resolve().parents[1] / "include" / "ldk.h").read_text())
              .group(1)) << 20


def _case(M, N, K, seed):
    w, x = cases.w4a16_case(M, N, K, seed)
    qw, s, z = oq.quantize_rtn(w.numpy(), 128)
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (x.numpy(), qw, s, z)]


def _call(entry, x, qw, s, z, split_k=0, flags=0):
    M, K = x.shape
    N = qw.shape[1]
    out = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    lib = _lib.load()
    st_ptr = _lib.stream(x.device)
    args = (_lib.ptr(x), K, _lib.ptr(qw), _lib.ptr(s), _lib.ptr(z), None, _lib.ptr(out), N, M, N, K,
            128, 0, split_k, flags)
    if entry == "noalloc":
        st = lib.ldk_w4a16_matmul_noalloc(*args, st_ptr)
    else:
        ws, ws_bytes = _lib.workspace(x.device)
        st = lib.ldk_w4a16_matmul(*args, ws, ws_bytes, st_ptr)
    msg = (lib.ldk_last_error() or b"").decode()
    return st, msg, out


# (M, N, K, split_k): the headline gate_up (hybrid grid, split remainder tiles), down (split 5),
# MFMA down at 16 rows (split 8: the largest default use of the array), q/o at 4 rows (no split)
CASES = [(1, 17920, 1536, 0), (1, 1536, 8960, 0), (16, 1536, 8960, 0), (4, 1536, 1536, 0),
         (1, 512, 8960, 7)]


@pytest.mark.parametrize("big,small", [(2, 0), (2, 1), (0, 4), (2, 3)])
def test_noalloc_matches_workspace_entry_on_consecutive_calls(big, small):
    print(f"[no_alloc] {CASES[big]} then {CASES[small]}", flush=True)
    for idx in (big, small):
        M, N, K, split = CASES[idx]
        x, qw, s, z = _case(M, N, K, seed=idx)
        st_ref, msg_ref, ref = _call("workspace", x, qw, s, z, split)
        st, msg, out = _call("noalloc", x, qw, s, z, split)
        torch.cuda.synchronize()
        assert st_ref == 0, msg_ref
        assert st == 0, msg
        assert torch.equal(out, ref), (CASES[idx], float((out.float() - ref.float()).abs().max()))


def test_noalloc_repeated_calls_stay_clean():
    """The kernels re-zero the words and slots they use: many calls in a row keep agreeing."""
    x, qw, s, z = _case(1, 1536, 8960, seed=9)
    _, _, ref = _call("workspace", x, qw, s, z, 7)
    for _ in range(10):
        st, msg, out = _call("noalloc", x, qw, s, z, 7)
        assert st == 0, msg
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_noalloc_rejects_a_split_beyond_its_array():
    """16 rows of N = 4096 split 32 ways need 65536 words of 136 bytes (8.9 MB) > the array."""
    assert SCRATCH == 4 << 20
    x, qw, s, z = _case(16, 4096, 4096, seed=3)
    st, msg, out = _call("noalloc", x, qw, s, z, split_k=32, flags=_lib.PATH_MFMA)
    assert st == _lib.ERR_INVALID and "needs" in msg and str(SCRATCH) in msg, msg
    st_ref, msg_ref, ref = _call("workspace", x, qw, s, z, split_k=32, flags=_lib.PATH_MFMA)
    assert st_ref == 0, msg_ref  # the 32 MiB caller workspace holds it
