"""Builds libpagedattn.so (the C-ABI of include/pagedattn.h) for gfx950.

Every csrc/*.hip translation unit is compiled in parallel with hipcc, then
linked into gb10-attn_amd/libpagedattn.so in-tree (so it travels with the
repository snapshot to the GPU host).  Usage: python gb10-attn_amd/build.py
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libpagedattn.so"
TORCH_LIB = PKG / "libpagedattn_torch.so"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", f"{ROCM}/bin/hipcc")
ARCH = "gfx950"

# Packed fp32 VALU forms are disabled (-packed-fp32-ops): the kernels are
# written for scalar fp32 arithmetic.
FLAGS = [
    "-O3", f"--offload-arch={ARCH}", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_torch_ops(verbose: bool = False) -> Path:
    """libpagedattn_torch.so: the torch.ops.gb10_attn operators (csrc/torch_ext.cpp),
    host C++ against torch's ROCm headers, linked to libpagedattn.so by $ORIGIN."""
    import torch
    import torch.utils.cpp_extension as cx
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{d}" for d in cx.include_paths()] + [f"-I{ROCM}/include"]
    libdirs = cx.library_paths()
    tmp = TORCH_LIB.with_suffix(".so.tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", *inc, str(CSRC / "torch_ext.cpp"), "-o", str(tmp),
           *[f"-L{d}" for d in libdirs], *[f"-Wl,-rpath,{d}" for d in libdirs],
           f"-L{PKG}", "-lpagedattn", "-Wl,-rpath,$ORIGIN",
           "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, TORCH_LIB)
    if verbose:
        print(f"built {TORCH_LIB}")
    return TORCH_LIB


_REMARK_KEYS = {"TotalSGPRs": "SGPRs", "VGPRs": "VGPRs", "AGPRs": "AGPRs",
                "ScratchSize [bytes/lane]": "scratch B/lane", "Occupancy [waves/SIMD]": "waves/SIMD",
                "SGPRs Spill": "SGPR spills", "VGPRs Spill": "VGPR spills", "LDS Size [bytes/block]": "LDS B"}


def resources() -> str:
    """Per-kernel register, LDS, scratch and occupancy figures of every
    csrc/*.hip kernel, from the compiler's kernel-resource-usage remarks
    (same flags as build()), as a markdown table.  Occupancy is the
    compiler's waves per SIMD from registers and LDS alone."""
    import re

    def remarks(src):
        cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-c", str(src), "-o", os.devnull,
               "-Rpass-analysis=kernel-resource-usage"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-6000:]}")
        return src, r

    srcs = sorted(CSRC.glob("*.hip"))
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(remarks, srcs))
    rows = []
    for src, r in results:
        cur = None
        for line in r.stderr.splitlines():
            m = re.search(r"remark: Function Name: (\S+)", line)
            if m:
                cur = {"file": src.name, "mangled": m.group(1)}
                rows.append(cur)
                continue
            m = re.search(r"remark:\s+([^:]+(?:\[[^\]]*\])?): (\S+) \[-Rpass", line)
            if m and cur is not None and m.group(1).strip() in _REMARK_KEYS:
                cur[_REMARK_KEYS[m.group(1).strip()]] = m.group(2)
    names = subprocess.run(["c++filt"], input="\n".join(r["mangled"] for r in rows), capture_output=True,
                           text=True, check=True).stdout.splitlines()
    cols = list(_REMARK_KEYS.values())
    out = ["| kernel | file | " + " | ".join(cols) + " |", "|---|---|" + "---|" * len(cols)]
    for r, n in zip(rows, names):
        n = n.replace("(pa::DecodeParams)", "").replace("(pa::PrefillParams)", "").replace(
            "(pa::ReduceParams)", "").replace("(pa::WriteParams)", "")
        out.append(f"| `{n}` | {r['file']} | " + " | ".join(r.get(c, "") for c in cols) + " |")
    return "\n".join(out) + "\n"


if __name__ == "__main__":
    if sys.argv[1:] == ["--resources"]:
        print(resources(), end="")
        sys.exit(0)
    build(verbose=True)
    build_torch_ops(verbose=True)
    sys.exit(0)
