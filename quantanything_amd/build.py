"""Builds ``libqa_hip.so`` (gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in ``csrc/_build`` (in
parallel) and linked into ``quantanything_amd/libqa_hip.so``. Only symbols
marked ``QA_API`` are exported (``-fvisibility=hidden``).

Usage: ``python -m quantanything_amd.build`` (also called by
``__graft_entry__.build()``).
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = CSRC / "_build"
LIB = PKG / "libqa_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed FP32 VALU instructions are disabled for every HIP source.
# Leading scalar kernel arguments (up to 16 dwords) arrive preloaded in
# SGPRs: a kernel can issue its first loads without a scalar load round
# trip of its arguments.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-mllvm", "-amdgpu-kernarg-preload-count=16"]
COMMON = ["-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
          f"--offload-arch={ARCH}", "-Wno-unused-command-line-argument"]


def _compile(src):
    out = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *COMMON, *DEVICE_FLAGS, "-c", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in proc.stderr.splitlines()
                     if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{errs}")
    return out


def build(verbose=True):
    """Compiles and links the library; returns its path."""
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol (e.g. a kernel whose launch stub the
    # host pass did not emit) fails the link instead of the first load
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC",
           "-Wl,-z,defs", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("link failed:\n" + proc.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
