"""Build recipe for the in-tree native artefacts (no cmake/ninja needed).

Outputs (all git-ignored, all shipped to the GPU box with the tree):
  opworks_amd/lib/libopworks_amd.so      HIP kernels + the extern "C" ABI
  opworks_amd/lib/adapters/*.so          one `solve` adapter per reference challenge
  opworks_amd/lib/tests/*                hipcc-built C++ unit-test executables and test-only
                                         libraries (libprobe_*.so)
  oracle/liboracle.so                    the CPU checker (gcc), via oracle/Makefile
  oracle/_ref/*                          reference host code, when /root/reference exists

Every HIP translation unit is compiled for gfx950 only, with packed-fp32
instruction selection disabled.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG / 'include'}",
    f"-I{ROOT / 'include'}",
]

LIB_SOURCES = sorted(CSRC.glob("*.hip"))
ADAPTER_SOURCES = sorted((CSRC / "adapters").glob("*.hip"))
# One executable per top-level .hip file or per subdirectory (all its .hip files);
# a top-level probe_<name>.hip is a test-only shared library lib<probe_name>.so.
TEST_SOURCES = sorted(p for p in (CSRC / "tests").glob("*.hip") if not p.name.startswith("probe_")) + sorted(
    d for d in (CSRC / "tests").glob("*") if d.is_dir() and any(d.glob("*.hip"))
)
PROBE_SOURCES = sorted((CSRC / "tests").glob("probe_*.hip"))


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    return obj


def build_library(jobs: int) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, LIB_SOURCES))
    so = LIB / "libopworks_amd.so"
    tmp = LIB / "libopworks_amd.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, so)
    return so


def build_adapters(jobs: int) -> list[Path]:
    out_dir = LIB / "adapters"
    out_dir.mkdir(parents=True, exist_ok=True)

    def one(src: Path) -> Path:
        so = out_dir / f"libopw_solve_{src.stem}.so"
        _run([HIPCC, *HIP_FLAGS, "-shared", "-o", str(so), str(src)])
        return so

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        return list(ex.map(one, ADAPTER_SOURCES))


def build_tests(jobs: int) -> list[Path]:
    out_dir = LIB / "tests"
    out_dir.mkdir(parents=True, exist_ok=True)

    def one(src: Path) -> Path:
        exe = out_dir / src.stem
        files = sorted(src.glob("*.hip")) if src.is_dir() else [src]
        _run([HIPCC, *HIP_FLAGS, "-o", str(exe), *map(str, files)])
        return exe

    def probe(src: Path) -> Path:
        so = out_dir / f"lib{src.stem}.so"
        _run([HIPCC, *HIP_FLAGS, "-shared", "-o", str(so), str(src)])
        return so

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        return list(ex.map(one, TEST_SOURCES)) + list(ex.map(probe, PROBE_SOURCES))


def build_oracle() -> None:
    _run(["make", "-B", "-C", str(ROOT / "oracle")])


def build_reference_host() -> None:
    """Compiles the reference's host-only headers (oracle/_ref), if present."""
    recipe = ROOT / "oracle" / "ref_host.mk"
    if Path("/root/reference").is_dir() and recipe.exists():
        _run(["make", "-B", "-f", str(recipe), "-C", str(ROOT / "oracle")])


def build_all(jobs: int | None = None, parts: tuple[str, ...] = ("lib", "adapters", "tests", "oracle", "ref")) -> None:
    jobs = jobs or min(8, os.cpu_count() or 4)
    t0 = time.time()
    if "oracle" in parts:
        build_oracle()
    if "ref" in parts:
        build_reference_host()
    if "lib" in parts:
        build_library(jobs)
    if "adapters" in parts and ADAPTER_SOURCES:
        build_adapters(jobs)
    if "tests" in parts and TEST_SOURCES:
        build_tests(jobs)
    print(f"[opworks_amd.build] {','.join(parts)} built in {time.time() - t0:.1f}s")


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("parts", nargs="*", default=["lib", "adapters", "tests", "oracle", "ref"])
    ap.add_argument("-j", "--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    build_all(args.jobs, tuple(args.parts))
    return 0


if __name__ == "__main__":
    sys.exit(main())
