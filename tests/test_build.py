"""The shipped device code: every gfx950 kernel of libmfattn.so is one function.

The library's ``.hip_fatbin`` section holds one offload bundle per source
file; each gfx950 code object is disassembled with ROCm's LLVM tools and
searched for calls.  A call (``s_swappc_b64``) means a device-library
function was not inlined: it costs a stack frame whose spills reach memory
and opens with a wait for every load in flight.  This happened while the
kernels were built with IEEE mode off (``-mno-amdgpu-ieee``), which the
inliner does not mix with the device libraries' IEEE mode.
"""

import pathlib
import re
import shutil
import subprocess

import pytest

from mfattn import _lib

LLVM = pathlib.Path("/opt/rocm/llvm/bin")
TOOLS = ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _tool(name):
    path = LLVM / name
    return str(path) if path.exists() else shutil.which(name)


def _code_objects(lib: pathlib.Path, tmp: pathlib.Path):
    fat = tmp / "fatbin"
    subprocess.run([_tool("llvm-objcopy"), "-O", "binary", "--only-section=.hip_fatbin", str(lib),
                    str(fat)], check=True)
    data = fat.read_bytes()
    starts, pos = [], data.find(MAGIC)
    while pos >= 0:
        starts.append(pos)
        pos = data.find(MAGIC, pos + len(MAGIC))
    assert starts, "no offload bundle in .hip_fatbin"
    for k, lo in enumerate(starts):
        hi = starts[k + 1] if k + 1 < len(starts) else len(data)
        bundle, co = tmp / f"b{k}", tmp / f"b{k}.co"
        bundle.write_bytes(data[lo:hi])
        subprocess.run([_tool("clang-offload-bundler"), "--unbundle", "--type=o",
                        f"--input={bundle}", f"--targets={TARGET}", f"--output={co}"], check=True)
        yield co


def _disassembly(tmp_path):
    """Instruction lines of every gfx950 function in the library, by symbol."""
    if not _lib.LIB_PATH.exists():
        pytest.skip("libmfattn.so is not built")
    missing = [t for t in TOOLS if _tool(t) is None]
    if missing:
        pytest.skip(f"ROCm LLVM tools missing: {missing}")
    funcs = {}
    for co in _code_objects(_lib.LIB_PATH, tmp_path):
        dis = subprocess.run([_tool("llvm-objdump"), "-d", "--mcpu=gfx950", str(co)],
                             capture_output=True, text=True, check=True).stdout
        current = None
        for line in dis.splitlines():
            m = re.match(r"^[0-9a-f]+ <(\S+)>:", line)
            if m:
                current = m.group(1)
                funcs.setdefault(current, [])
            elif current is not None and line.strip():
                funcs[current].append(line)
    assert any(k.startswith("_ZN2mf20attn_fwd_bf16_kernel") for k in funcs), sorted(funcs)[:5]
    return funcs


def test_device_code_makes_no_calls(tmp_path):
    funcs = _disassembly(tmp_path)
    calls = sorted(k for k, lines in funcs.items() if any("s_swappc_b64" in l for l in lines))
    assert not calls, calls
    # nothing but kernels: no out-of-line device-library function was emitted
    assert not [k for k in funcs if k.startswith("__o")], sorted(k for k in funcs if k.startswith("__o"))


def test_no_kernel_touches_scratch(tmp_path):
    """Register spills go to scratch memory in HBM (a reload costs a memory round trip, and
    4 bytes per lane of write traffic).  No kernel of the library spills: every value that
    the work loops do not need is recomputed after them instead."""
    funcs = _disassembly(tmp_path)
    use = {k: [l for l in lines if "scratch_" in l] for k, lines in funcs.items()}
    use = {k: v[:2] for k, v in use.items() if v}
    assert not use, use
