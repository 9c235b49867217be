"""Build libsaeflow_hip.so in-tree from saeflow_amd/csrc/*.hip for gfx950.

    python -m saeflow_amd.build [-v]

Each source is compiled to an object under saeflow_amd/_build/ (in parallel), then
linked into saeflow_amd/libsaeflow_hip.so, which exports exactly the entry points of
include/saeflow_hip.h. Always recompiles: callers that only need a library load it with
saeflow_amd._lib.
"""

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsaeflow_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # packed fp32 VALU ops stay off (only scalar fp32 VALU in these kernels)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",  # only the SF_API entry points of include/saeflow_hip.h are exported
    "-Wno-unused-command-line-argument",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (needs ROCm: /opt/rocm/bin/hipcc)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build(verbose=False, jobs=None):
    """Compile every csrc/*.hip and link libsaeflow_hip.so; returns the library path."""
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD / (s.stem + ".o") for s in sources]
    jobs = jobs or min(len(sources), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(lambda so: _run([cc, *HIPCC_FLAGS, "-I", str(PKG.parent / "include"), "-c", str(so[0]),
                                     "-o", str(so[1])], verbose), zip(sources, objs)))
    tmp = LIB.with_name(LIB.name + ".tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    p = argparse.ArgumentParser()
    p.add_argument("-v", "--verbose", action="store_true")
    print(build(verbose=p.parse_args().verbose))
    sys.exit(0)
