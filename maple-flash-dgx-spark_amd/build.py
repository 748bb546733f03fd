"""Build ``libmaple_amd.so`` from ``csrc/*.hip`` for gfx950 with hipcc.

Objects go to ``_build/`` next to this file; the shared library is written
in-tree (``libmaple_amd.so``) so it travels with the source tree.  Every call
recompiles all sources (the build check must always compile).  A second
library, ``libmaple_amd_stamps.so``, links the same objects with the
one-launch MoE layer built with ``-DMA_PHASE_STAMPS`` (per-phase real-time
stamps in its workspace, for timelines; ``ma_moe_phase_stamps``).

    python maple-flash-dgx-spark_amd/build.py
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libmaple_amd.so"
OUT_STAMPS = PKG / "libmaple_amd_stamps.so"
STAMPED_SOURCES = ("moe_xcd.hip",)
OBJ = PKG / "_build"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast",
    "-munsafe-fp-atomics",
    # Kernel arguments arrive preloaded in SGPRs (saves a dependent load at
    # the head of every kernel; decode kernels are latency-bound).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    # Keep the compiler from forming packed-FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _compile(src: Path, stamps: bool = False) -> Path:
    obj = OBJ / (src.stem + ("_stamps.o" if stamps else ".o"))
    cmd = [HIPCC, *FLAGS, *(["-DMA_PHASE_STAMPS"] if stamps else []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def _link(objs, out: Path) -> None:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = True) -> Path:
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; cannot build the maple_amd HIP library")
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources), max(1, (os.cpu_count() or 4)))
    stamped = [src for src in sources if src.name in STAMPED_SOURCES]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs_f = [ex.submit(_compile, src) for src in sources]
        stamped_f = {src.name: ex.submit(_compile, src, True) for src in stamped}
        objs = [f.result() for f in objs_f]
        stamped_objs = {name: f.result() for name, f in stamped_f.items()}
    _link(objs, OUT)
    _link([stamped_objs.get(src.name, obj) for src, obj in zip(sources, objs)], OUT_STAMPS)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources (and {OUT_STAMPS.name})")
    return OUT


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
