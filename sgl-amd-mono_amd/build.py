"""Build recipe of libmono_amd.so: every HIP source of ``csrc/`` compiled for gfx950 by
hipcc into one shared library with the C ABI of ``include/mono_amd.h``.

Run ``python -m sgl_amd_mono_amd.build`` (or ``__graft_entry__.build()``). The library
lands next to this file, where ``_lib.py`` loads it from.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB = PKG / "libmono_amd.so"
ARCH = "gfx950"

# CDNA4 only. Packed-FP32 VALU ops are disabled: some of their forms have given wrong
# results on these machines, and the kernels are memory bound anyway.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the monokernels build with ROCm's hipcc for gfx950")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass warns that it does not know the packed-fp32 feature: harmless
    err = "\n".join(
        ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln and ln.strip()
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err:
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int = 0) -> Path:
    """Compile every ``csrc/*.hip`` into ``libmono_amd.so`` (always recompiles): each
    source to an object of its own, in parallel, then one link."""
    import tempfile
    from concurrent.futures import ThreadPoolExecutor

    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 16)
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(prefix="mono_build_") as tmpdir:
        objs = [Path(tmpdir) / (src.stem + ".o") for src in srcs]
        cmds = [[hipcc(), *flags, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
                for src, obj in zip(srcs, objs)]
        with ThreadPoolExecutor(jobs) as pool:
            list(pool.map(lambda c: _run(c, verbose), cmds))
        tmp = LIB.with_suffix(".so.tmp")
        _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o",
              str(tmp)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
