"""Builds libwptv.so, the HIP library of the verify step, for gfx950 only.

    python -m wpt_amd.build        compile every source under wpt_amd/csrc

The library lands in wpt_amd/lib/ (in the tree, so that it travels with the
repository to a GPU machine); it links the HIP runtime by its soname, which
resolves to the runtime PyTorch has already loaded when it is imported after
torch.
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
SOURCES = PACKAGE / "csrc"
LIBRARY = PACKAGE / "lib" / "libwptv.so"
ARCH = "gfx950"

# Every HIP source is compiled with packed FP32 arithmetic off (the packed
# forms are left to no code in this library), and with the first 16 dwords
# of each kernel's arguments preloaded into SGPRs at wave launch (gfx950's
# kernarg preload; the code keeps the loads as a fallback prologue).
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16", "-Wall", "-Wno-unused-function",
             "-Wno-unused-variable", "-Wno-unused-but-set-variable"]


def hipcc():
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc is not installed: the HIP library cannot be built")
    return found


def _compile(source, objects):
    target = objects / (source.name + ".o")
    command = [hipcc(), *HIP_FLAGS, "-c", str(source), "-o", str(target)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source.name} failed:\n{' '.join(command)}\n{result.stderr}")
    return target


def build(verbose=False):
    """Compiles every source and links the library; returns its path."""
    sources = sorted(SOURCES.glob("*.hip")) + sorted(SOURCES.glob("*.cpp"))
    objects = PACKAGE / "lib" / "obj"
    objects.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        built = list(pool.map(lambda source: _compile(source, objects), sources))
    partial = LIBRARY.with_suffix(".so.tmp")
    command = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(partial), *map(str, built)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking libwptv.so failed:\n{' '.join(command)}\n{result.stderr}")
    os.replace(partial, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
