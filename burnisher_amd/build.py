"""Builds libburnisher_hip.so for gfx950 from burnisher_amd/csrc with hipcc.

Every source is compiled to an object in burnisher_amd/_build/ (in parallel), then linked into
burnisher_amd/lib/libburnisher_hip.so. The library is built in-tree so that it travels with the
repository to the GPU box; nothing is installed.

    python -m burnisher_amd.build          # or: python burnisher_amd/build.py
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libburnisher_hip.so"

ARCH = "gfx950"
# Packed fp32 (v_pk_*_f32) generation is switched off for all device code: hipcc forms those
# instructions on its own from ordinary float code and some forms have given wrong results on
# these boxes. The host pass warns that it does not know the feature; that is harmless.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def sources() -> list[Path]:
    return sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp"))


# Per-file code-generation options. flash72.hip keeps its output accumulators in VGPRs (they are
# rescaled by VALU multiplies, and in the default AGPR form every rescale and loop iteration
# copies all 80 of them between the register files), and it is compiled without IEEE NaN rules
# so a maximum over MFMA results is one v_max3 per two inputs, not a quieting v_max per input.
# cross_fused.hip runs the same attention code after its projection, so it takes the same options.
# denoise.hip evaluates the guidance combine and the solver update in fp64 exactly as the
# reference's x86-64 build does, which forms no multiply-add. elementwise.hip holds the kernels
# that reproduce the oracle's arithmetic bit for bit (norms, modulate, add, chunk, activation,
# patch, scale, the timestep embedding), so it forms no contraction either: under the default
# -ffp-contract=fast the compiler also fuses an fp64 -> fp32 -> bf16 conversion chain into one
# rounding, which differs from the reference's two at bf16 ties. probe.hip keeps its MFMA loop's
# accumulators in VGPRs: in the AGPR form the compiler rotates them through ~50 copies per
# eight MFMAs, which would measure the copies rather than the matrix cores.
EXTRA_FLAGS = {"flash72.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
               "cross_fused.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
               "denoise.hip": ["-ffp-contract=off"],
               "elementwise.hip": ["-ffp-contract=off"],
               "probe.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: Path) -> Path:
    obj = OBJ / (src.name + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs), "-lpthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(PKG.parent)} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
