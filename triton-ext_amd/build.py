"""Build libtxamd.so: gfx950 code objects + the C-ABI host library.

Steps:
  1. every ``csrc/kernels/*.hip`` -> ``_build/<name>.hsaco`` with
     ``hipcc --genco --offload-arch=gfx950`` (device code only);
  2. a generated assembly file embeds each code object with ``.incbin``;
  3. the host sources (``csrc/host/*.cpp``) are compiled with g++ against the
     HIP runtime headers and linked with the embedded code objects into
     ``tx/libtxamd.so``.

Run ``python triton-ext_amd/build.py`` (or call ``build()``).  hipcc
cross-compiles for gfx950 without a GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "tx", "libtxamd.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# Code objects in the order of tx::CodeObject (csrc/host/tx_runtime.h).
KERNEL_SOURCES = ["fp8_codec", "scatter", "gemm_bf16", "gemm_fp8", "gemv", "gemm_mx"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "--genco",
    # hardware fp32 atomic add (global_atomic_add_f32 / ds_add_f32)
    "-munsafe-fp-atomics",
    # never emit packed-fp32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]

HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-fno-exceptions",
    "-fno-rtti", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def _hipcc():
    p = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found")
    return p


def build_kernel(name: str) -> str:
    src = os.path.join(CSRC, "kernels", f"{name}.hip")
    out = os.path.join(BUILD, f"{name}.hsaco")
    _run([_hipcc(), *HIPCC_FLAGS, src, "-o", out])
    return out


def write_embed(paths) -> str:
    asm = os.path.join(BUILD, "tx_embedded.S")
    lines = ['\t.section .rodata.tx_code_objects,"a",@progbits']
    for name, path in zip(KERNEL_SOURCES, paths):
        sym = f"tx_co_{name}"
        lines += [
            "\t.balign 4096",
            f"\t.globl {sym}_begin",
            f"\t.hidden {sym}_begin",
            f"{sym}_begin:",
            f'\t.incbin "{path}"',
            f"\t.globl {sym}_end",
            f"\t.hidden {sym}_end",
            f"{sym}_end:",
            "\t.byte 0",
        ]
    lines.append('\t.section .note.GNU-stack,"",@progbits')
    with open(asm, "w") as f:
        f.write("\n".join(lines) + "\n")
    return asm


# Host sources that also define device data (the no-allocation entry point's
# workspace array): compiled by hipcc for the host and gfx950, registered
# with the HIP runtime when the library loads.
HIP_HOST_FLAGS = [
    f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-fno-exceptions",
    "-fno-rtti", "-Wall", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build_host(asm: str) -> str:
    srcs = sorted(glob.glob(os.path.join(CSRC, "host", "*.cpp")) + glob.glob(os.path.join(CSRC, "host", "*.hip")))
    objs = []
    inc = ["-I", os.path.join(REPO, "include"), "-I", CSRC, "-I", os.path.join(CSRC, "host"),
           "-I", os.path.join(ROCM, "include")]
    cxx = os.environ.get("CXX", "g++")

    def compile_one(src):
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        if src.endswith(".hip"):
            _run([_hipcc(), *HIP_HOST_FLAGS, *inc, "-c", src, "-o", obj])
        else:
            _run([cxx, *HOST_FLAGS, *inc, "-c", src, "-o", obj])
        return obj

    with cf.ThreadPoolExecutor(max_workers=4) as ex:
        objs = list(ex.map(compile_one, srcs))
    emb = os.path.join(BUILD, "tx_embedded.o")
    _run([cxx, "-c", asm, "-o", emb])
    tmp = OUT + ".tmp"
    _run([cxx, "-shared", "-o", tmp, *objs, emb, f"-L{ROCM}/lib", "-lamdhip64",
          f"-Wl,-rpath,{ROCM}/lib", "-Wl,--no-undefined"])
    os.replace(tmp, OUT)
    return OUT


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(KERNEL_SOURCES), 8)) as ex:
        paths = list(ex.map(build_kernel, KERNEL_SOURCES))
    asm = write_embed(paths)
    out = build_host(asm)
    if verbose:
        print(f"built {out}")
    return out


if __name__ == "__main__":
    try:
        build()
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
