"""Build ``libcatopt_hip.so`` from ``catopt_amd/csrc/*.hip`` for gfx950.

Each translation unit is compiled with ``hipcc -c`` in parallel, then the
objects are linked into one shared library next to this file (in-tree, so
the library travels with the repository snapshot).  Compile flags:

* ``--offload-arch=gfx950`` only — the kernels are written for CDNA4;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` disables packed
  fp32 instruction selection (the host pass warns it does not know the
  feature; that warning is harmless);
* ``-O3 -std=c++17 -fPIC``;
* per-source extras in ``SOURCE_FLAGS``: the retention scan keeps its MFMA
  accumulators in VGPRs (``-amdgpu-mfma-vgpr-form``) because its loop scales
  and converts them on the VALU every chunk, and AGPR-resident accumulators
  would cost a copy in and out for each of those operations; the dense
  affine scan feeds each step's accumulators back as the next step's MFMA
  B operands, which read VGPRs only (AGPR-resident accumulators cost 16
  ``v_accvgpr_read`` per step, each waiting on its MFMA).

Run ``python -m catopt_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "libcatopt_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# every kernel is this library's own: no vendor library is linked
LINK_LIBS: list[str] = []

SOURCE_FLAGS = {
    "retention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "scan_dense.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build")
    return exe


def _compile(src: Path, obj: Path, extra: list[str]) -> tuple[Path, str]:
    cmd = [_hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o",
           str(obj)]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{p.stdout}\n{p.stderr}")
    return obj, p.stderr


def build(verbose: bool = False, jobs: int | None = None, extra: list[str] | None = None) -> Path:
    """Compile every kernel source and link the shared library; return its path."""
    BUILD.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    extra = list(extra or [])
    objs: list[Path] = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, BUILD / (s.stem + ".o"), extra) for s in srcs]
        for f in futs:
            obj, log = f.result()
            objs.append(obj)
            if verbose and log.strip():
                print(log, file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), *LINK_LIBS]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stdout}\n{p.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
