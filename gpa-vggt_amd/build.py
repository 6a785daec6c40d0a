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
# in VGPRs with the VGPR form of MFMA selected (256 VGPRs at two waves per
# SIMD, no AGPR copies, no VGPR or SGPR spills, no scratch).
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


def resource_usage(sources=None) -> dict:
    """Per-kernel register and scratch use as hipcc reports it for the
    library's own flags: {source name: {kernel: {"vgprs", "sgpr_spill",
    "vgpr_spill", "scratch", "occupancy"}}}.  Compiles to a temporary
    object; nothing under the package is touched."""
    import re
    import tempfile
    keys = {"VGPRs": "vgprs", "SGPRs Spill": "sgpr_spill", "VGPRs Spill": "vgpr_spill",
            "ScratchSize [bytes/lane]": "scratch", "Occupancy [waves/SIMD]": "occupancy"}
    srcs = sorted(CSRC.glob("*.hip")) if sources is None else [CSRC / s for s in sources]

    def one(src: Path):
        with tempfile.TemporaryDirectory() as tmp:
            cmd = [_hipcc(), "-Rpass-analysis=kernel-resource-usage", *HIPCC_FLAGS,
                   *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(Path(tmp) / "k.o")]
            res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
        kernels, cur = {}, None
        for line in res.stderr.splitlines():
            m = re.search(r"remark: (.*?): (\S+) \[-Rpass-analysis", line)
            if not m:
                continue
            name, val = m.group(1).strip(), m.group(2)
            if name == "Function Name":
                cur = kernels.setdefault(val, {})
            elif cur is not None and name in keys:
                cur[keys[name]] = int(val)
        return src.name, kernels

    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        return dict(pool.map(one, srcs))


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
    _build_probe(verbose)
    return LIB_PATH


PROBE_SRC = CSRC / "probe"
PROBE_LIB = LIB_DIR / "libgpa_probe.so"


def _build_probe(verbose: bool) -> None:
    """The register-only MFMA probes the benchmark prices its ceilings with
    (csrc/probe/, a library of its own: not part of the product ABI)."""
    sources = sorted(PROBE_SRC.glob("*.hip"))
    if not sources:
        return
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-shared", "-o", str(tmp), *[str(s) for s in sources]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on the probes:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, PROBE_LIB)
    if verbose:
        print(f"built {PROBE_LIB.relative_to(REPO_DIR)}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--report", action="store_true", help="print kernel resource usage")
    args = ap.parse_args(argv)
    build(report=args.report)
    return 0


if __name__ == "__main__":
    sys.exit(main())
