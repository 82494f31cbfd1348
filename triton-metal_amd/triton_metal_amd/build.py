"""Build libtm_hip.so in-tree.

Steps (all on the host; hipcc cross-compiles gfx950 without a GPU):
  1. hipcc --genco --offload-arch=gfx950 each csrc/kernels/*.hip -> code object
  2. write an assembler file that .incbin's every code object, plus the
     module list header the runtime includes
  3. g++ the C-ABI sources (csrc/capi/*.cpp) and link libtm_hip.so; the
     library does not link libamdhip64, it resolves HIP at run time

The result lands next to this file (triton_metal_amd/libtm_hip.so), which is
where the ctypes layer loads it from.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
PROJ_DIR = PKG_DIR.parent                    # triton-metal_amd/
REPO_DIR = PROJ_DIR.parent                   # repository root
CSRC = PROJ_DIR / "csrc"
BUILD_DIR = PROJ_DIR / "_build"
INCLUDE_DIR = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libtm_hip.so"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "--genco",
    # packed-fp32 VALU forms are disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-file additions.  kda.hip: MFMA results in VGPRs rather than AGPRs (the
# compiler's choice for kda_state, whose state update scales and packs every
# result on the VALU, would move each one out of AGPRs and back every chunk;
# the file's other kernels compile identically either way).
EXTRA_FLAGS = {
    "kda": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _run(cmd, verbose):
    if verbose:
        print("+", " ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(
            f"build step failed ({r.returncode}): {' '.join(str(c) for c in cmd)}\n"
            f"{r.stdout}\n{r.stderr}")
    return r


def kernel_sources():
    return sorted((CSRC / "kernels").glob("*.hip"))


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every kernel for gfx950 and link libtm_hip.so; returns its path."""
    hipcc = ROCM / "bin" / "hipcc"
    if not hipcc.exists():
        raise RuntimeError(f"hipcc not found at {hipcc}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = kernel_sources()
    jobs = jobs or min(8, max(1, len(srcs)))

    def compile_one(src: Path) -> Path:
        out = BUILD_DIR / (src.stem + ".hsaco")
        _run([hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.stem, []), f"-I{CSRC / 'kernels'}", src,
              "-o", out], verbose)
        return out

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))

    # embedded code objects
    names = [o.stem for o in objs]
    asm = ['  .section .rodata.tm_code_objects,"a",@progbits']
    for name, o in zip(names, objs):
        asm += [
            "  .balign 4096",
            f"  .globl tm_co_{name}_start",
            f"  .hidden tm_co_{name}_start",
            f"tm_co_{name}_start:",
            f'  .incbin "{o}"',
            f"  .globl tm_co_{name}_end",
            f"  .hidden tm_co_{name}_end",
            f"tm_co_{name}_end:",
            "  .byte 0",
        ]
    asm.append('  .section .note.GNU-stack,"",@progbits')
    (BUILD_DIR / "embed.S").write_text("\n".join(asm) + "\n")
    (BUILD_DIR / "modules.inc").write_text(
        "#define TM_MODULE_LIST(X) " + " ".join(f"X({n})" for n in names) + "\n")

    cxx = shutil.which("g++") or "g++"
    cflags = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__",
              f"-I{INCLUDE_DIR}", f"-I{ROCM / 'include'}", f"-I{BUILD_DIR}",
              f"-I{CSRC / 'capi'}", "-fvisibility=hidden"]
    cpp_srcs = sorted((CSRC / "capi").glob("*.cpp"))

    def compile_cpp(src: Path) -> Path:
        out = BUILD_DIR / (src.stem + ".o")
        _run([cxx, *cflags, "-c", src, "-o", out], verbose)
        return out

    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        cobjs = list(ex.map(compile_cpp, cpp_srcs))
    embed_o = BUILD_DIR / "embed.o"
    _run([cxx, "-c", BUILD_DIR / "embed.S", "-o", embed_o], verbose)

    tmp = LIB_PATH.with_name(LIB_PATH.name + ".tmp")
    _run([cxx, "-shared", "-o", tmp, *cobjs, embed_o, "-ldl", "-lpthread",
          "-Wl,--no-undefined", "-Wl,-z,noexecstack"], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
