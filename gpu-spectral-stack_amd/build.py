"""Builds the two shared libraries of the MI355X FFT stack, in-tree, for gfx950.

    python gpu-spectral-stack_amd/build.py [--jobs N] [--only capi|torch|tools] [--force]
    python gpu-spectral-stack_amd/build.py --define NAME=VALUE [...] --lib-dir DIR

1. libspectral_hip.so: every HIP kernel plus the C ABI of include/spectral_hip.h. Built with
   hipcc for --offload-arch=gfx950 only; depends on the HIP runtime and nothing from PyTorch.
2. spectral/_C.so: the PyTorch operators (TORCH_LIBRARY "spectral") over that C ABI. Plain
   C++ against the PyTorch-ROCm headers, linked to libspectral_hip.so through $ORIGIN.
3. bin/spectral_peaks: the measured copy-bandwidth and FP32 ceilings (csrc/tools/peaks.hip),
   bin/spectral_bench: every implementation of every operation next to rocFFT, as CSV
   (csrc/tools/spectral_bench.cpp, over the C ABI of libspectral_hip.so), and
   bin/spectral_mfma_dft: C4's pruned column pass as FFTs and as an fp32 matrix-core DFT
   (csrc/tools/mfma_dft.hip).

Both land in python/spectral/, next to the Python package that loads them. Object files go to
_build/ (git-ignored). Every call recompiles what is older than its sources.
"""

from __future__ import annotations

import argparse
import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

ROOT = Path(__file__).resolve().parent
REPO = ROOT.parent
CSRC = ROOT / "csrc"
INCLUDE = REPO / "include"
PKG = ROOT / "python" / "spectral"
BUILD = ROOT / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

# Device-code flags. Packed FP32 instructions are switched off: some of their forms have given
# wrong results on these machines, and the FFT's float arithmetic does not need them.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unknown-pragmas",
    "-ffp-contract=fast",
    "-munsafe-fp-atomics",
    f"-I{CSRC}",
    f"-I{INCLUDE}",
]

CAPI_SOURCES = [
    "stockham_r2.hip",
    "stockham_r4.hip",
    "stockham_r8.hip",
    "stockham_r8_table.hip",
    "real.hip",
    "naive.hip",
    "scale.hip",
    "remap.hip",
    "noalloc.hip",
    "fft2d.hip",
    "pruned.hip",
    "ns.hip",
    "registry.cpp",
    "capi.cpp",
]
# Every header under csrc/ is a dependency of every object: a header edit recompiles them all.
CAPI_HEADERS = sorted(p.name for p in CSRC.glob("*.hpp"))

LIB = PKG / "libspectral_hip.so"
EXT = PKG / "_C.so"
BIN = ROOT / "bin"
# name -> (source, extra compile/link arguments)
TOOLS = {
    "spectral_peaks": (CSRC / "tools" / "peaks.hip", []),
    "spectral_bench": (CSRC / "tools" / "spectral_bench.cpp",
                       ["-x", "hip", f"-L{PKG}", "-lspectral_hip", "-lhipfft",
                        "-Wl,-rpath,$ORIGIN/../python/spectral"]),
    "spectral_mfma_dft": (CSRC / "tools" / "mfma_dft.hip",
                          [f"-L{PKG}", "-lspectral_hip", "-Wl,-rpath,$ORIGIN/../python/spectral"]),
}


def _stale(target: Path, deps: list[Path]) -> bool:
    if not target.exists():
        return True
    t = target.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise SystemExit(f"build failed: {' '.join(cmd[:3])} ... (exit {proc.returncode})")
    # The host pass does not know the packed-fp32 target feature; that warning is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    rest = [line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line]
    if rest:
        sys.stderr.write("\n".join(rest) + "\n")


def _compile(src: Path, force: bool) -> Path:
    obj = BUILD / (src.name + ".o")
    deps = [src] + [CSRC / h for h in CAPI_HEADERS] + [INCLUDE / "spectral_hip.h"]
    if force or _stale(obj, deps):
        print(f"  hipcc {src.name}", flush=True)
        lang = [] if src.suffix == ".hip" else ["-x", "hip"]
        _run([HIPCC, *HIP_FLAGS, *lang, "-c", str(src), "-o", str(obj)])
    return obj


def build_capi(jobs: int, force: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = [CSRC / s for s in CAPI_SOURCES]
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, force), sources))
    if force or _stale(LIB, objs):
        print(f"  link {LIB.name}", flush=True)
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(LIB), *map(str, objs),
              "-Wl,-soname,libspectral_hip.so"])
    return LIB


def build_variant(jobs: int, defines: list[str], lib_dir: Path) -> Path:
    """libspectral_hip.so built with extra -D definitions into lib_dir (its objects under
    lib_dir/obj), for measuring a compile-time alternative next to the product library: the tools
    pick it up through LD_LIBRARY_PATH (their RUNPATH gives way to it)."""
    obj_dir = lib_dir / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    flags = [*HIP_FLAGS, *[f"-D{d}" for d in defines]]

    def compile_one(name: str) -> str:
        src = CSRC / name
        obj = obj_dir / (name + ".o")
        lang = [] if src.suffix == ".hip" else ["-x", "hip"]
        _run([HIPCC, *flags, *lang, "-c", str(src), "-o", str(obj)])
        return str(obj)

    print(f"  variant {' '.join(defines)} -> {lib_dir}", flush=True)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, CAPI_SOURCES))
    lib = lib_dir / LIB.name
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(lib), *objs,
          "-Wl,-soname,libspectral_hip.so"])
    return lib


def _torch_paths() -> tuple[list[str], list[str]]:
    import torch
    from torch.utils import cpp_extension

    return cpp_extension.include_paths(), cpp_extension.library_paths()


def build_torch(force: bool = False) -> Path:
    src = CSRC / "torch_ops.cpp"
    deps = [src, INCLUDE / "spectral_hip.h", LIB]
    if not (force or _stale(EXT, deps)):
        return EXT
    includes, libdirs = _torch_paths()
    py_include = sysconfig.get_paths()["include"]
    import torch

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    print("  g++ torch_ops.cpp", flush=True)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-I{INCLUDE}", f"-I{py_include}", f"-I{ROCM / 'include'}",
        *[f"-I{p}" for p in includes],
        str(src), "-o", str(EXT),
        f"-L{PKG}", "-lspectral_hip",
        *[f"-L{p}" for p in libdirs],
        "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
        "-Wl,-rpath,$ORIGIN",
        *[f"-Wl,-rpath,{p}" for p in libdirs],
        "-Wno-deprecated-declarations",
    ]
    _run(cmd)
    return EXT


def build_tools(force: bool = False) -> list[Path]:
    BIN.mkdir(exist_ok=True)
    built = []
    for name, (src, extra) in TOOLS.items():
        exe = BIN / name
        if force or _stale(exe, [src, INCLUDE / "spectral_hip.h", LIB]):
            print(f"  hipcc {src.name} -> bin/{name}", flush=True)
            lang = extra[:2] if extra[:1] == ["-x"] else []
            link = extra[len(lang):]
            _run([HIPCC, *[f for f in HIP_FLAGS if f != "-fPIC"], *lang, str(src), "-o", str(exe),
                  *link])
        built.append(exe)
    return built


def main(argv: list[str] | None = None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--only", choices=["capi", "torch", "tools"])
    ap.add_argument("--force", action="store_true", help="recompile everything")
    ap.add_argument("--define", action="append", default=[], metavar="NAME=VALUE",
                    help="build only a variant library with this definition (repeatable)")
    ap.add_argument("--lib-dir", type=Path, help="where the --define variant library goes")
    args = ap.parse_args(argv)
    if args.define:
        if args.lib_dir is None:
            ap.error("--define needs --lib-dir")
        build_variant(args.jobs, args.define, args.lib_dir.resolve())
        return
    if args.only in (None, "capi"):
        build_capi(args.jobs, args.force)
    if args.only in (None, "torch"):
        build_torch(args.force)
    if args.only in (None, "tools"):
        build_tools(args.force)


if __name__ == "__main__":
    main()
