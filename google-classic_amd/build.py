"""Build the HIP op library and the host-side input generator, in-tree.

    python google-classic_amd/build.py          # both libraries
    python google-classic_amd/build.py --hip    # libholo_mi355x.so only

Outputs (git-ignored, shipped with the tree):
    google-classic_amd/libholo_mi355x.so   gfx950 kernels + C ABI (include/*.h)
    google-classic_amd/libholo_synth.so    seeded GGUF-block / activation generator
"""
from __future__ import annotations

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
OBJ = PKG / "_build"
HIP_LIB = PKG / "libholo_mi355x.so"
SYNTH_LIB = PKG / "libholo_synth.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in any kernel (the host pass
# warns that it does not know the feature; harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}",
]
# Per-file extra flags.
EXTRA = {
    "dequant.hip": ["-ffp-contract=off"],
}


def hip_sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[-1]}")


def build_hip(jobs: int = 8) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = hip_sources()
    objs = [OBJ / (s.stem + ".o") for s in srcs]

    def one(src: Path, obj: Path) -> None:
        _run([HIPCC, *HIP_FLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)])

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(one, srcs, objs))
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_synth() -> Path:
    cc = shutil.which("gcc") or "cc"
    tmp = SYNTH_LIB.with_suffix(".so.tmp")
    _run([cc, "-std=c11", "-O2", "-fopenmp", "-fPIC", "-shared", "-Wall",
          str(CSRC / "synth.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


HARNESS_SRC = ROOT / "tests" / "abi_harness.c"
HARNESS = ROOT / "tests" / "abi_harness"


def build_harness() -> Path:
    """The C caller of the drop-in boundary (tests/abi_harness.c), linked
    against the HIP library with an rpath to it; the GPU tests run it."""
    cc = shutil.which("gcc") or "cc"
    tmp = HARNESS.with_suffix(".tmp")
    _run([cc, "-std=c11", "-O2", "-Wall", "-Werror", f"-I{ROOT / 'include'}", str(HARNESS_SRC),
          f"-L{PKG}", "-lholo_mi355x", "-Wl,-rpath,$ORIGIN/../google-classic_amd", "-o", str(tmp)])
    os.replace(tmp, HARNESS)
    return HARNESS


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--hip", action="store_true", help="only the HIP library")
    ap.add_argument("--synth", action="store_true", help="only the generator")
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args()
    if not a.synth:
        print("built", build_hip(a.j))
        print("built", build_harness())
    if not a.hip:
        print("built", build_synth())


if __name__ == "__main__":
    main()
