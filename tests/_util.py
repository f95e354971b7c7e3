"""Shared helpers of the GPU parity tests: host/device conversion and the tolerance metrics."""

from __future__ import annotations

import numpy as np
import torch


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def dev(a, device="cuda") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def bits16(a) -> np.ndarray:
    a = a if isinstance(a, np.ndarray) else to_np(a)
    return np.ascontiguousarray(a).view(np.uint16)


def err_stats(out, ref) -> dict:
    """max-abs and relative-L2 error of an fp16 output against an fp32/fp64 reference."""
    o = (out if isinstance(out, np.ndarray) else to_np(out)).astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    d = o - r
    return {"max_abs": float(np.abs(d).max()),
            "rel_l2": float(np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30))}


def assert_north_star(out, ref, max_abs=2e-2, rel_l2=1e-3):
    """The acceptance bar for fp16 matmul outputs: max-abs <= 2e-2 AND rel-L2 <= 1e-3 against
    the fp32-accumulated dequantize-then-matmul reference."""
    e = err_stats(out, ref)
    assert e["max_abs"] <= max_abs and e["rel_l2"] <= rel_l2, e
    return e


def ulp_diff_fp16(a, b) -> np.ndarray:
    """Distance between two fp16 arrays in units in the last place: the bit patterns are mapped
    to a monotone integer line (negative values mirrored, +0 and -0 both at 0)."""
    def ordered(x):
        u = bits16(x).astype(np.int32)
        mag = u & 0x7FFF
        return np.where(u & 0x8000, -mag, mag)
    return np.abs(ordered(a) - ordered(b))


def within_one_ulp_of_intermediate(out, inter, other) -> np.ndarray:
    """True where the fp16 output equals fp16(other * i') for some i' within one fp16 ulp of the
    reference's rounded fp16 intermediate `inter` (the product itself rounded once). This is the
    fp16 1-ulp tolerance stated on the one rounding step whose input depends on a transcendental
    or a reduction order (rsqrt of the mean square, exp in silu)."""
    o = bits16(out)
    inter = np.asarray(inter, dtype=np.float16)
    other = np.asarray(other, dtype=np.float16)
    ok = np.zeros(o.shape, dtype=bool)
    for cand in (np.nextafter(inter, np.float16(-np.inf)), inter, np.nextafter(inter, np.float16(np.inf))):
        prod = (other.astype(np.float32) * cand.astype(np.float32)).astype(np.float16)
        ok |= bits16(prod) == o
        ok |= (bits16(prod) & 0x7FFF) + (o & 0x7FFF) == 0  # +0 / -0
    return ok
