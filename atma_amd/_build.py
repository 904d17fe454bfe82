"""Build libatma_hip.so from atma_amd/csrc/*.hip for gfx950 (hipcc, in-tree).

Usage: ``python -m atma_amd._build [--jobs N]``.  The library lands next to this
file (``atma_amd/libatma_hip.so``) so it travels with the source tree; objects go
to ``atma_amd/_build/``.
"""

import argparse
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
OBJDIR = PKG / "_build"
LIB = PKG / "libatma_hip.so"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for all device code (they have produced wrong
# results on this hardware pool); hipcc's host pass warns that it does not know
# the feature, which is harmless.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                # keep MFMA accumulators in VGPRs: the softmax touches them with VALU ops,
                # and AGPR residency costs a v_accvgpr move per element per key block
                "-mllvm", "-amdgpu-mfma-vgpr-form"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-munsafe-fp-atomics",
                "-Wno-unused-command-line-argument", "-Wno-unknown-warning-option"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{proc.stdout}")
    return obj


def build(jobs: int = 0, verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link libatma_hip.so.  Always rebuilds."""
    OBJDIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources in {CSRC}")
    jobs = jobs or min(len(sources), max(1, min(os.cpu_count() or 1, 16)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{proc.stdout}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=0)
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True)


if __name__ == "__main__":
    sys.exit(main())
