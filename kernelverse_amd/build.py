"""Build libkvv.so (the HIP verdict library) in-tree for gfx950.

    python -m kernelverse_amd.build

The scan kernels are instantiated once per element type from
csrc/kvv_scan_inst.hip (-DKVV_DT=<code>), so the fifteen dtypes compile in
parallel next to csrc/kvv.hip (API, reduce, select, finalize); the objects are
linked into kernelverse_amd/libkvv.so, which travels with the repository.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libkvv.so"
N_DTYPES = 15

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # every float operation of the elementwise test is rounded on its own, as torch-CPU does
    "-ffp-contract=off",
    # packed fp32 ops stay off (they have given silent wrong results on this hardware)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the verdict library needs ROCm's hipcc to build")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd[-3:])}")


def build(verbose: bool = False, jobs: int = None) -> Path:
    cc = hipcc()
    inc = [f"-I{ROOT / 'include'}", f"-I{CSRC}"]
    jobs = jobs or min(os.cpu_count() or 4, 16)
    with tempfile.TemporaryDirectory(prefix="kvv_build_") as tmp:
        tmp = Path(tmp)
        units = [(CSRC / "kvv.hip", [], tmp / "kvv.o")]
        units += [(CSRC / "kvv_scan_inst.hip", [f"-DKVV_DT={dt}"], tmp / f"kvv_scan_{dt}.o") for dt in range(N_DTYPES)]
        cmds = [[cc, *HIPCC_FLAGS, *inc, *defs, "-c", str(src), "-o", str(obj)] for src, defs, obj in units]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        tmp_out = OUT.with_suffix(".so.tmp")
        _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", *[str(o) for _, _, o in units], "-o", str(tmp_out)],
             verbose)
        os.replace(tmp_out, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
