"""Build recipe for libsa_amd.so (gfx950 kernels + C ABI + C++ API mirror).

Every translation unit goes through hipcc; kernels are compiled for gfx950
only.  Objects go to _build/ and the shared library to lib/, both inside this
package directory, so the library travels with the source tree.

    python streaming-attention_amd/build.py            # build the library
    python streaming-attention_amd/build.py --tests    # also the C++ test driver
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
BUILD = PKG / "_build"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libsa_amd.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
# Packed fp32 instructions are disabled for all device code (they have given
# wrong results on this hardware pool); hipcc's host pass ignores the feature.
DEVICE = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


# Per-file device flags.  The prefill kernels keep MFMA accumulators in arch
# VGPRs (their softmax rescales them with VALU ops); the register-staged bf16
# kernel parks Q in AGPRs.
EXTRA = {
    "prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def sources() -> list[Path]:
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    srcs += sorted((CSRC / "compat").glob("*.cpp"))
    return srcs


def compile_one(src: Path) -> Path:
    rel = src.relative_to(CSRC)
    obj = BUILD / (str(rel).replace("/", "__") + ".o")
    obj.parent.mkdir(parents=True, exist_ok=True)
    if src.suffix == ".hip":
        cmd = [HIPCC, "-x", "hip", *COMMON, *DEVICE, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, *COMMON, "-D__HIP_PLATFORM_AMD__", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build_library(jobs: int = 8, verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp),
           *[str(o) for o in objs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


def build_cpp_tests(verbose: bool = True) -> list[Path]:
    """C++ drivers under tests/cpp that exercise the reference-shaped API:
    lib*.cpp become shared libraries (bin/lib*.so, loaded by pytest), the
    others executables."""
    tdir = ROOT / "tests" / "cpp"
    out_dir = tdir / "bin"
    out_dir.mkdir(parents=True, exist_ok=True)
    oracle_lib = ROOT / "oracle" / "liboracle.so"
    outs = []
    for src in sorted(tdir.glob("*.cpp")):
        shared = src.stem.startswith("lib")
        exe = out_dir / (src.stem + (".so" if shared else ""))
        cmd = [HIPCC, "-O2", "-std=c++17", f"-I{ROOT / 'include'}", f"-I{ROOT / 'oracle'}",
               *(["-shared", "-fPIC"] if shared else []),
               str(src), "-o", str(exe), f"-L{LIB_DIR}", "-lsa_amd",
               f"-Wl,-rpath,{LIB_DIR}", f"-Wl,-rpath,$ORIGIN/../../../streaming-attention_amd/lib"]
        if oracle_lib.exists() and not shared:
            cmd += [f"-L{oracle_lib.parent}", "-loracle",
                    "-Wl,-rpath,$ORIGIN/../../../oracle", "-fopenmp"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"test build failed: {src}\n{res.stdout}\n{res.stderr}")
        outs.append(exe)
    if verbose and outs:
        print("built C++ tests:", ", ".join(p.name for p in outs))
    return outs


CLI_DIR = PKG / "cli"
BIN_DIR = PKG / "bin"


def build_cli(verbose: bool = True) -> list[Path]:
    """Host programs over the C ABI (cli/*.cpp -> bin/), linked to lib/libsa_amd.so."""
    BIN_DIR.mkdir(exist_ok=True)
    outs = []
    for src in sorted(CLI_DIR.glob("*.cpp")):
        exe = BIN_DIR / src.stem
        cmd = [HIPCC, "-O2", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", str(src),
               "-o", str(exe), f"-L{LIB_DIR}", "-lsa_amd", "-Wl,-rpath,$ORIGIN/../lib"]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"CLI build failed: {src}\n{res.stdout}\n{res.stderr}")
        outs.append(exe)
    if verbose and outs:
        print("built CLI:", ", ".join(p.name for p in outs))
    return outs


def clean() -> None:
    shutil.rmtree(BUILD, ignore_errors=True)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--tests", action="store_true")
    ap.add_argument("--clean", action="store_true")
    ap.add_argument("-j", type=int, default=8)
    args = ap.parse_args()
    if args.clean:
        clean()
    try:
        build_library(args.j)
        build_cli()
        if args.tests:
            build_cpp_tests()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
