"""Build recipe for libdspark_hip.so (gfx950) and the oracle's C library.

    python mlx-dspark_amd/build.py            # both libraries
    python mlx-dspark_amd/build.py --hip      # engine library only

Every HIP source is compiled in parallel with hipcc into _build/, then linked into
mlx_dspark/libdspark_hip.so next to the Python package that loads it. The oracle
(oracle/accept_oracle.c) is built with gcc and -ffp-contract=off into oracle/liboracle.so.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent          # mlx-dspark_amd/
REPO = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
BUILD = PKG_ROOT / "_build"
LIB = PKG_ROOT / "mlx_dspark" / "libdspark_hip.so"
ORACLE_SRC = REPO / "oracle" / "accept_oracle.c"
ORACLE_LIB = REPO / "oracle" / "liboracle.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l)  # the host pass does not know the feature
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_hip(jobs: int | None = None) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        lang = ["-x", "hip"] if src.suffix == ".hip" else []
        _run([HIPCC, *HIP_FLAGS, *lang, "-c", str(src), "-o", str(obj)])
        return obj

    jobs = jobs or min(len(sources), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-fPIC", "-shared",
          str(ORACLE_SRC), "-o", str(tmp), "-lm"])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--hip", action="store_true", help="engine library only")
    ap.add_argument("--oracle", action="store_true", help="oracle library only")
    ap.add_argument("--clean", action="store_true")
    args = ap.parse_args(argv)
    if args.clean and BUILD.exists():
        shutil.rmtree(BUILD)
    if not args.oracle:
        print("built", build_hip())
    if not args.hip:
        print("built", build_oracle())
    return 0


if __name__ == "__main__":
    sys.exit(main())
