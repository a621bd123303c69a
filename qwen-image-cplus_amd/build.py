"""Build the gfx950 HIP library (and, for tests, the CPU oracle) in-tree.

    python qwen-image-cplus_amd/build.py            # library + oracle
    python qwen-image-cplus_amd/build.py --lib-only

The library is ``qwen_image_hip/libqwen_image_hip.so`` next to its Python
host module.  Every .hip source is compiled for gfx950 only, with packed
fp32 VALU instructions disabled, and linked with hipcc.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "qwen_image_hip"
LIB = OUT_DIR / "libqwen_image_hip.so"
CLI = OUT_DIR / "qi-quantize"  # the pack writer / verifier command (cli/qi_quantize.cpp)
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra"]

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Wall",
    # Packed fp32 VALU forms stay off for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results land in ordinary VGPRs, so the fp32 epilogues read them
    # without an accumulator-register copy per element.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # The host pass does not know the gfx feature name; drop that one notice.
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_library(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objects = []
    todo = []
    for src in sources:
        obj = BUILD / (src.stem + ".o")
        objects.append(obj)
        todo.append((src, obj))

    # Host-only C++ (the QIPACK container) is compiled by the host compiler.
    for src in sorted(CSRC.glob("*.cpp")):
        obj = BUILD / (src.stem + ".cpp.o")
        objects.append(obj)
        todo.append((src, obj))

    def compile_one(pair):
        src, obj = pair
        if src.suffix == ".cpp":
            _run([CXX, *CXX_FLAGS, "-c", str(src), "-o", str(obj)])
        else:
            _run([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        list(pool.map(compile_one, todo))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)])
    os.replace(tmp, LIB)
    return LIB


def build_cli() -> Path:
    """The qi-quantize command, linked against the library next to it."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    tmp = CLI.with_suffix(".tmp")
    _run([CXX, *[f for f in CXX_FLAGS if f != "-fvisibility=hidden"], "-D__HIP_PLATFORM_AMD__",
          f"-I{rocm}/include", str(PKG / "cli" / "qi_quantize.cpp"), "-o", str(tmp), f"-L{OUT_DIR}",
          "-lqwen_image_hip", f"-L{rocm}/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{rocm}/lib"])
    os.replace(tmp, CLI)
    return CLI


PROBE = PKG / "probe"


def build_probe() -> list[Path]:
    """The matrix-core / vector-unit co-execution micro-benchmark
    (probe/mfma_valu_probe.hip, run by ``bench.py --probe-overlap``), built
    with MFMA results in ordinary VGPRs (the product library's flag) and in
    accumulator registers (the compiler's default).  Not part of the
    product library."""
    out = []
    agpr = [f for f in HIP_FLAGS if f not in ("-mllvm", "-amdgpu-mfma-vgpr-form=1")]
    for form, flags in (("vgpr", HIP_FLAGS), ("agpr", agpr)):
        lib = PROBE / f"libqi_probe_{form}.so"
        _run([HIPCC, *flags, "-shared", "-o", str(lib), str(PROBE / "mfma_valu_probe.hip")])
        out.append(lib)
    # The W4A4 GEMM with parts of its work removed (csrc/w4a4_fp6.hip,
    # QI_ABLATE_*), for bench.py --ablate-w4a4: timing only, wrong outputs.
    def ablate(item):
        name, macros = item
        lib = PROBE / f"libqi_fp6_ablate_{name}.so"
        _run([HIPCC, *HIP_FLAGS, *[f"-DQI_ABLATE_{m}" for m in macros], "-shared", "-o", str(lib),
              str(CSRC / "w4a4_fp6.hip")])
        return lib
    with ThreadPoolExecutor(max_workers=8) as pool:
        out += list(pool.map(ablate, ABLATIONS.items()))
    return out


# name -> QI_ABLATE_* macros of the W4A4 measurement builds.
ABLATIONS = {"none": (), "dma": ("DMA",), "lds": ("LDS",), "barrier": ("BARRIER",), "vmwait": ("VMWAIT",), "fma": ("FMA",),
             "mfma": ("MFMA",), "memory": ("DMA", "LDS"), "arith_only": ("DMA", "LDS", "BARRIER")}


def build_oracle() -> Path:
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
    return ROOT / "oracle" / "_build" / "libqi_oracle.so"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    args = ap.parse_args(argv)
    print("built", build_library(args.j))
    print("built", build_cli())
    if not args.lib_only:
        print("built", *build_probe())
        print("built", build_oracle())
    return 0


if __name__ == "__main__":
    sys.exit(main())
