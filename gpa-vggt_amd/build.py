"""Build recipe for the gfx950 shared library behind the `merging` package.

    python gpa-vggt_amd/build.py            # compile + link
    python gpa-vggt_amd/build.py --report   # also print per-kernel VGPR/spill usage

Each `csrc/*.hip` file is compiled by hipcc for gfx950 only and the objects are
linked into `merging/_lib/libgpa_mi355x.so`.  The library is loaded with
ctypes after `import torch`, so it binds to the HIP runtime torch already
loaded (same SONAME, libamdhip64.so.7).
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
OBJ_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "merging" / "_lib"
LIB_NAME = "libgpa_mi355x.so"
LIB_PATH = LIB_DIR / LIB_NAME

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    # Code object v5: loadable by the HIP runtime torch bundles (ROCm 7.0)
    # as well as by the system ROCm 7.2 runtime.
    "-mcode-object-version=5",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-source extra flags.  The attention kernel keeps its MFMA accumulators
# in VGPRs with the VGPR form of MFMA selected (195 VGPRs, no AGPR copies or
# spills at two waves per SIMD).
FILE_FLAGS = {
    "attn_keybias.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the gfx950 library)")


def _compile(src: Path, report: bool) -> tuple[Path, str]:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if report:
        cmd.insert(1, "-Rpass-analysis=kernel-resource-usage")
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj, res.stderr


def build(report: bool = False, verbose: bool = True) -> Path:
    """Compile every csrc/*.hip for gfx950 and link the shared library."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        results = list(pool.map(lambda s: _compile(s, report), sources))
    if report:
        for _, log in results:
            for line in log.splitlines():
                if "remark" in line and any(
                    key in line for key in ("Function Name", "VGPRs:", "AGPRs", "Spill", "LDS Size", "Occupancy")
                ):
                    print(line.split("remark: ")[-1])
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for o, _ in results]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH.relative_to(REPO_DIR)}")
    return LIB_PATH


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--report", action="store_true", help="print kernel resource usage")
    args = ap.parse_args(argv)
    build(report=args.report)
    return 0


if __name__ == "__main__":
    sys.exit(main())
