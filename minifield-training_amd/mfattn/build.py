"""Build ``libmfattn.so`` (the HIP kernels + C ABI) in-tree for gfx950.

``python minifield-training_amd/mfattn/build.py`` (a plain script: importing the
package needs the library it builds) or
``mfattn.build.build()``.  Every ``.hip`` file under ``csrc/`` is compiled
with ``hipcc --offload-arch=gfx950`` into an object in ``csrc/_build`` and
linked into ``mfattn/libmfattn.so``.  Packed-FP32 instructions are disabled
(``-packed-fp32-ops``); the host pass warns that it does not know that
feature, which is harmless.
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = ROOT / "csrc"
OUT = PKG / "libmfattn.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # min/max need no NaN quieting: masked scores are -inf, never NaN.  IEEE
    # mode stays on (no -mno-amdgpu-ieee): the device libraries are built with
    # it, and the inliner does not inline across a mode mismatch, which turned
    # every threadIdx/blockIdx/blockDim read, rsqrtf and sincosf into a call
    # (a stack frame, and a wait for every load in flight at each call)
    "-fno-honor-nans",
    # the conv backward's ring loop (2K steps, slot indices compile-time only
    # when it is fully unrolled) exceeds the default size limit for pragma
    # unrolls at K >= 7 in bf16; a partial unroll left its ring arrays in
    # scratch memory.  No other loop here reaches the limit.
    "-mllvm", "-pragma-unroll-threshold=65536",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the mfattn kernels need ROCm's hipcc")
    return path


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [_hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = True) -> pathlib.Path:
    sources = sorted(CSRC.glob("*.hip"))
    objdir = CSRC / "_build"
    objdir.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in sources]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        list(pool.map(_compile, sources, objs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


# Host code under AddressSanitizer and UBSan: the C ABI (argument checks,
# plan layout, workspace sizes) compiled with the sanitizers on its host pass
# only, linked with the regular kernel objects.  It loads into a process that
# preloads the sanitizer runtime (``sanitizer_runtime()``); the GPU code is
# the regular build's.
SAN_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O1", "-g", "-fno-omit-frame-pointer",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
]
SAN_OUT = CSRC / "_build" / "libmfattn_san.so"


def sanitizer_runtime() -> pathlib.Path | None:
    """The clang AddressSanitizer runtime of the ROCm toolchain (it carries UBSan's handlers)."""
    hits = sorted(pathlib.Path("/opt/rocm/llvm/lib/clang").glob(
        "*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def build_sanitized() -> pathlib.Path:
    objdir = CSRC / "_build"
    if not OUT.exists() or not all((objdir / (s.stem + ".o")).exists()
                                   for s in CSRC.glob("*.hip")):
        build(verbose=False)
    abi = objdir / "mf_abi_san.o"
    proc = subprocess.run([_hipcc(), *SAN_FLAGS, "-c", str(CSRC / "mf_abi.hip"), "-o", str(abi)],
                          capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for the sanitizer build:\n{proc.stderr}")
    objs = [str(o) for o in sorted(objdir.glob("*.o"))
            if o.name not in ("mf_abi.o", "mf_abi_san.o")]
    proc = subprocess.run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o",
                           str(SAN_OUT), str(abi), *objs], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed for the sanitizer build:\n{proc.stderr}")
    return SAN_OUT


if __name__ == "__main__":
    build()
