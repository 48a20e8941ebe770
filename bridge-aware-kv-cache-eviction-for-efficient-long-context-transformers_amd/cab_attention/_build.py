"""Build libcab_hip.so for gfx950 from ../csrc with hipcc (in-tree).

Each ``csrc/*.hip`` file is compiled to an object in ``_build/`` (in
parallel), then linked into ``cab_attention/libcab_hip.so``, which the ctypes
loader in ``_native.py`` opens. Run as ``python -m cab_attention._build`` from
the package root or through ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
BUILD = ROOT / "_build"
LIB = PKG_DIR / "libcab_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-variable",
    "-Wno-unused-function",
    # Keep packed-fp32 instructions out of the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: no accvgpr moves when the softmax
    # rescales or the epilogue reads them.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP toolchain is required to build libcab_hip.so")


# Per-source extra flags. The attention kernel's device code never produces
# or tests a NaN (masked scores are -inf, the running maximum starts at a
# finite sentinel), so its float maxima need no sNaN canonicalisation.
EXTRA_FLAGS = {
    "sparse_attn.hip": ["-Xarch_device", "-fno-honor-nans"],
}


def _compile(hipcc: str, src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n" + "\n".join(errs))
    if errs:
        sys.stderr.write("\n".join(errs) + "\n")
    return obj


def build(verbose: bool = True) -> pathlib.Path:
    """Compile every csrc/*.hip and link libcab_hip.so. Always rebuilds."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(hipcc, s), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link of libcab_hip.so failed:\n" + res.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


# Host code under AddressSanitizer and UndefinedBehaviorSanitizer (argument
# validation, size arithmetic, error strings), for CPU tests of the C ABI.
# Only host code is instrumented: every -fsanitize= goes through -Xarch_host,
# and the link passes -fno-gpu-sanitize. The device code is the product's.
SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=all",
    "-fno-omit-frame-pointer", "-g", "-Xarch_device", "-g0",
]


def asan_runtime() -> pathlib.Path:
    """The clang AddressSanitizer runtime the sanitized library needs preloaded."""
    llvm = pathlib.Path(_hipcc()).resolve().parent.parent / "llvm" / "lib" / "clang"
    for cand in sorted(llvm.glob("*/lib/linux/libclang_rt.asan-x86_64.so")):
        return cand
    raise RuntimeError(f"no libclang_rt.asan-x86_64.so under {llvm}")


def build_host_sanitized(out_dir: pathlib.Path, verbose: bool = False) -> pathlib.Path:
    """Compile every csrc/*.hip with sanitized host code into out_dir/libcab_hip_asan.so.
    Load it with asan_runtime() in LD_PRELOAD (see tests/test_host_sanitizers.py)."""
    hipcc = _hipcc()
    out_dir = pathlib.Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))

    def compile_one(src: pathlib.Path) -> pathlib.Path:
        obj = out_dir / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-O1", "-Xarch_device", "-O3", *SANITIZE_FLAGS,
               *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"sanitized build of {src.name} failed:\n{res.stderr[-4000:]}")
        return obj

    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, sources))
    lib = out_dir / "libcab_hip_asan.so"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-fsanitize=address,undefined",
           "-fno-gpu-sanitize", "-shared-libsan", "-o", str(lib), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("link of libcab_hip_asan.so failed:\n" + res.stderr)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build()
