"""Builds libnerf.so, the HIP backend.

libnerf.so: every nerf_amd/csrc/*.hip file is compiled for gfx950 with hipcc
and linked into one shared library exporting the C ABI of include/nerf.h and
include/nerf_ext.h.  Flags that matter for correctness:
  -ffp-contract=off     no implicit FMA: bit-exact indices, bits and counts
  -packed-fp32-ops off  no v_pk_*_f32 generation
The host harness (nerf_amd/harness, plain C++20 built with g++) gives
libnerf_host.so (PNG, JSON, dataset loading and PSNR behind a C API, no GPU
needed) and nerf_bench, the reference host program's counterpart linked
against libnerf.so.
Run:  python -m nerf_amd.build   (or via __graft_entry__.build()).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libnerf.so"
HARNESS = PKG / "harness"
HOST_LIB = PKG / "libnerf_host.so"
BENCH_EXE = PKG / "nerf_bench"
GXX_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-ffp-contract=off", "-Wall", "-Wextra", "-fvisibility=hidden"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-fvisibility=hidden",
    "-DNERF_BUILD_SHARED",
    "-DNERF_BUILD_EXPORTS",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: no accumulator-register copies before the VALU uses them.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libnerf.so)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build_library(jobs: int = 8) -> Path:
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))

    def compile_one(src: Path) -> Path:
        obj = BUILD / (src.stem + ".o")
        _run([hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)])
        return obj

    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_harness(jobs: int = 8) -> tuple[Path, Path]:
    """libnerf_host.so and nerf_bench (needs libnerf.so for the latter)."""
    gxx = shutil.which("g++") or "g++"
    BUILD.mkdir(exist_ok=True)
    parts = ["png", "json", "dataset"]

    def compile_one(stem: str) -> Path:
        obj = BUILD / f"harness_{stem}.o"
        _run([gxx, *GXX_FLAGS, "-c", str(HARNESS / f"{stem}.cpp"), "-o", str(obj)])
        return obj

    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, parts + ["host_capi", "nerf_bench"]))
    common, capi, main_obj = objs[:3], objs[3], objs[4]
    tmp = HOST_LIB.with_suffix(".so.tmp")
    _run([gxx, "-shared", "-o", str(tmp), *map(str, common), str(capi)])
    os.replace(tmp, HOST_LIB)
    tmp = BENCH_EXE.with_suffix(".tmp")
    _run([gxx, "-o", str(tmp), str(main_obj), *map(str, common), f"-L{PKG}", "-lnerf", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, BENCH_EXE)
    return HOST_LIB, BENCH_EXE


SAN_FLAGS = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]


def build_harness_sanitized(out_dir: Path) -> Path:
    """libnerf_host.so of the host harness (plain C++, g++) with
    AddressSanitizer and UndefinedBehaviorSanitizer, into out_dir."""
    gxx = shutil.which("g++") or "g++"
    out_dir.mkdir(parents=True, exist_ok=True)
    flags = [f for f in GXX_FLAGS if f != "-O2"] + SAN_FLAGS
    objs = []
    for stem in ("png", "json", "dataset", "host_capi"):
        obj = out_dir / f"{stem}.o"
        _run([gxx, *flags, "-c", str(HARNESS / f"{stem}.cpp"), "-o", str(obj)])
        objs.append(obj)
    lib = out_dir / "libnerf_host.so"
    _run([gxx, "-shared", *SAN_FLAGS, "-o", str(lib), *map(str, objs)])
    return lib


def main() -> None:
    lib = build_library()
    print(f"built {lib}")
    for p in build_harness():
        print(f"built {p}")


if __name__ == "__main__":
    main()
