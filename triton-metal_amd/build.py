"""Build libtritonmetal.so and its gfx950 kernel images, in-tree.

    python triton-metal_amd/build.py [--jobs N]

Steps:
  1. every csrc/kernels/*.hip -> lib/<name>.hsaco  (hipcc --genco, gfx950);
  2. lib/blobs.S: a table linking those images into the library;
  3. csrc/scratch.hip -> lib/scratch.o  (the static device scratch of
     tm_launch_noalloc; hipcc, host and gfx950 device code);
  4. csrc/runtime.cpp + lib/blobs.S + lib/scratch.o -> lib/libtritonmetal.so
     (the tm_* C ABI).

Outputs stay in lib/ (git-ignored, shipped with the tree).  Compiler flags:
-O3, gfx950 only, packed-fp32 instruction selection disabled (the kernels are
written for scalar fp32 VALU).
"""

import argparse
import concurrent.futures
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "lib"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
LIBRARY = LIB / "libtritonmetal.so"


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")
    return proc.stdout


def kernel_sources():
    return sorted((CSRC / "kernels").glob("*.hip"))


def build_kernel(src: Path) -> Path:
    out = LIB / (src.stem + ".hsaco")
    _run([HIPCC, *HIP_FLAGS, "--genco", str(src), "-o", str(out)])
    return out


def write_blobs(images):
    lines = ['.section .note.GNU-stack,"",@progbits', ".section .rodata"]
    for i, img in enumerate(images):
        lines += [
            ".balign 4096",
            f"tm_blob_{i}_start:",
            f'.incbin "{img}"',
            f"tm_blob_{i}_end:",
            ".byte 0",
        ]
    lines += [".section .data.rel.ro", ".balign 8", ".global tm_builtin_blob_table",
              "tm_builtin_blob_table:"]
    for i in range(len(images)):
        lines.append(f".quad tm_blob_{i}_start, tm_blob_{i}_end")
    lines += [".global tm_builtin_blob_count", ".balign 4", "tm_builtin_blob_count:",
              f".long {len(images)}", ""]
    path = LIB / "blobs.S"
    path.write_text("\n".join(lines))
    return path


def build_scratch() -> Path:
    out = LIB / "scratch.o"
    _run([HIPCC, *HIP_FLAGS, "-fPIC", "-c", str(CSRC / "scratch.hip"), "-o", str(out)])
    return out


def build_sanitized() -> Path:
    """The host library alone (runtime + code-object reader, kernels as built)
    under AddressSanitizer and UndefinedBehaviorSanitizer, for CPU test runs:
        LD_PRELOAD="$(gcc -print-file-name=libasan.so) $(gcc -print-file-name=libubsan.so)" \\
        ASAN_OPTIONS=detect_leaks=0 TRITON_METAL_CORE_LIB=<this file> pytest tests -m "not gpu"
    Host code only: the kernels are the normal gfx950 builds."""
    blobs, scratch = LIB / "blobs.S", LIB / "scratch.o"
    if not blobs.exists() or not scratch.exists():
        build()
    out = LIB / "libtritonmetal_asan.so"
    _run([
        "g++", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
        "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
        str(CSRC / "runtime.cpp"), str(CSRC / "codeobject.cpp"), str(blobs), str(scratch),
        "-o", str(out),
        f"-L{ROCM / 'lib'}", "-lamdhip64", "-lhiprtc", f"-Wl,-rpath,{ROCM / 'lib'}",
    ])
    return out


def build(jobs: int = 8) -> Path:
    LIB.mkdir(exist_ok=True)
    srcs = kernel_sources()
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        scratch_job = pool.submit(build_scratch)
        images = list(pool.map(build_kernel, srcs))
        scratch = scratch_job.result()
    blobs = write_blobs(images)
    _run([
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
        str(CSRC / "runtime.cpp"), str(CSRC / "codeobject.cpp"), str(blobs), str(scratch),
        "-o", str(LIBRARY),
        f"-L{ROCM / 'lib'}", "-lamdhip64", "-lhiprtc", f"-Wl,-rpath,{ROCM / 'lib'}",
    ])
    return LIBRARY


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--sanitize", action="store_true",
                    help="also build lib/libtritonmetal_asan.so (host code under ASan + UBSan)")
    args = ap.parse_args()
    print(build(args.jobs))
    if args.sanitize:
        print(build_sanitized())
    sys.exit(0)
