"""Builds libldk_amd.so, the gfx950 HIP kernel library behind the C ABI in include/ldk.h.

Each csrc/*.hip file is compiled with hipcc for gfx950 only, in parallel, then linked into
`kernels/libldk_amd.so` inside this package (in-tree, so it travels with the repository snapshot).

    python llm-decode-kernels_amd/build.py [-j N] [--save-temps DIR]
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = REPO / "include"
OBJ = PKG / "_build"
LIB = PKG / "kernels" / "libldk_amd.so"
ARCH = "gfx950"

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

CFLAGS = [
    "-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC",
    # Packed FP32 instructions are kept out of the device code entirely.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE-exact float division and sqrt: the quantizers must reproduce torch's bits.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, save_temps: Path | None) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", str(src), "-o", str(obj)]
    if save_temps is not None:
        cmd.append(f"-save-temps={save_temps}")
    res = subprocess.run(cmd, capture_output=True, text=True,
                         cwd=str(save_temps) if save_temps else None)
    errs = [ln for ln in res.stderr.splitlines()
            if "packed-fp32-ops" not in ln and ln.strip() and "warning: feature flag" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(errs[-60:]))
    return obj


def build(jobs: int | None = None, save_temps: str | None = None, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link kernels/libldk_amd.so. Returns its path."""
    OBJ.mkdir(exist_ok=True)
    st = Path(save_temps).resolve() if save_temps else None
    if st:
        st.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, st), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stderr[-4000:])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--save-temps", default=None)
    args = ap.parse_args()
    try:
        build(args.j, args.save_temps, verbose=True)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
