"""The code-object argument reader (triton-metal_amd/csrc/codeobject.cpp), on the
CPU: hipcc cross-compiles a few gfx950 kernels, a small host program built
from the reader prints what it finds, and the layouts are checked against the
AMDGPU kernel ABI (pointers 8 bytes, naturally aligned scalars, a by-value
struct as one parameter).  User launches through tm_launch are checked against
these layouts before they reach the GPU.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "triton-metal_amd" / "csrc"
HIPCC = "/opt/rocm/bin/hipcc"

KERNELS = r'''
#include <hip/hip_runtime.h>
struct Block { const void *a, *b; void *c; int m, n, k, s0, s1, s2, s3, s4, s5; const void *bias; };
extern "C" __global__ void takes_buffer_and_int(float *out, int n) { if (n) out[0] = 1.f; }
extern "C" __global__ void takes_nothing() {}
extern "C" __global__ void takes_mixed(float a, long long b, int *c, float d) {
  if (a > 0.f) c[0] = (int)b + (int)d;
}
extern "C" __global__ void takes_block(Block p) { if (p.m) ((float *)p.c)[0] = 2.f; }
'''

HARNESS = r'''
#include <cstdio>
#include <fstream>
#include <iterator>
#include <vector>
#include "codeobject.h"
int main(int argc, char **argv) {
  std::ifstream f(argv[1], std::ios::binary);
  std::vector<char> data((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  size_t n = data.size();
  if (argc > 2) n = std::min(n, (size_t)std::stoul(argv[2]));
  for (const auto &k : tm_codeobject::read_kernel_arguments(n ? data.data() : nullptr, n)) {
    std::printf("%s", k.first.c_str());
    for (const auto &a : k.second) std::printf(" %ld:%ld:%s", a.offset, a.size, a.kind.c_str());
    std::printf("\n");
  }
  return 0;
}
'''

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists() or shutil.which("g++") is None,
                                reason="needs hipcc (gfx950 cross-compiler) and g++")


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    d = tmp_path_factory.mktemp("codeobject")
    (d / "k.hip").write_text(KERNELS)
    (d / "h.cpp").write_text(HARNESS)
    common = [HIPCC, "--offload-arch=gfx950", "-O2", str(d / "k.hip")]
    subprocess.run(common + ["--genco", "-o", str(d / "bundle.hsaco")], check=True)
    subprocess.run(common + ["--cuda-device-only", "--no-gpu-bundle-output", "-c", "-o",
                             str(d / "raw.o")], check=True)
    subprocess.run(["g++", "-O1", "-std=c++17", f"-I{CSRC}", str(d / "h.cpp"),
                    str(CSRC / "codeobject.cpp"), "-o", str(d / "h")], check=True)
    return d


def read(built, image, limit=None):
    cmd = [str(built / "h"), str(image)] + ([str(limit)] if limit is not None else [])
    out = subprocess.run(cmd, check=True, capture_output=True, text=True).stdout
    result = {}
    for line in out.splitlines():
        name, *slots = line.split()
        result[name] = [tuple(int(x) if x.isdigit() else x for x in s.split(":")) for s in slots]
    return result


@pytest.mark.parametrize("image", ["bundle.hsaco", "raw.o"])
def test_argument_layouts_follow_the_kernel_abi(built, image):
    sig = read(built, built / image)
    assert sig["takes_buffer_and_int"] == [(0, 8, "global_buffer"), (8, 4, "by_value")]
    assert sig["takes_nothing"] == []
    # float at 0, int64 aligned to 8, pointer at 16, float at 24
    assert sig["takes_mixed"] == [(0, 4, "by_value"), (8, 8, "by_value"),
                                  (16, 8, "global_buffer"), (24, 4, "by_value")]
    # one by-value struct of 72 bytes: what a 12-argument launch must not be bound to
    assert sig["takes_block"] == [(0, 72, "by_value")]


def test_truncated_and_foreign_images_yield_nothing(built):
    image = built / "bundle.hsaco"
    size = image.stat().st_size
    for limit in (0, 1, 23, 24, 40, 100, size // 3, size // 2, size - 1):
        got = read(built, image, limit)
        assert got == {} or set(got) <= {"takes_buffer_and_int", "takes_nothing", "takes_mixed",
                                         "takes_block"}
    (built / "junk.bin").write_bytes(bytes(range(256)) * 64)
    assert read(built, built / "junk.bin") == {}


FUZZ = r"""
#include <cstdio>
#include <fstream>
#include <iterator>
#include <random>
#include <vector>
#include "codeobject.h"
int main(int argc, char **argv) {
  long total = 0;
  for (int f = 1; f < argc; ++f) {
    std::ifstream in(argv[f], std::ios::binary);
    std::vector<char> img((std::istreambuf_iterator<char>(in)), std::istreambuf_iterator<char>());
    for (size_t n = 0; n <= img.size(); n += 3) {
      std::vector<char> cut(img.begin(), img.begin() + n);
      total += tm_codeobject::read_kernel_arguments(cut.data(), cut.size()).size();
    }
    std::mt19937 rng(f);
    for (int it = 0; it < 2000; ++it) {
      std::vector<char> mut = img;
      for (int k = 0, flips = 1 + rng() % 8; k < flips; ++k) mut[rng() % mut.size()] = (char)rng();
      total += tm_codeobject::read_kernel_arguments(mut.data(), mut.size()).size();
    }
  }
  std::printf("parsed %ld\n", total);
  return 0;
}
"""


def test_reader_survives_truncated_and_corrupted_images_under_sanitizers(built):
    """Every truncation of a bundle and of a raw ELF, and 2000 random byte
    corruptions of each, through the reader built with AddressSanitizer and
    UndefinedBehaviorSanitizer (host code only): no out-of-bounds read, no
    undefined behaviour, whatever the bytes."""
    (built / "fuzz.cpp").write_text(FUZZ)
    exe = built / "fuzz"
    build = subprocess.run(["g++", "-O1", "-g", "-fsanitize=address,undefined",
                            "-fno-sanitize-recover=all", "-std=c++17", f"-I{CSRC}",
                            str(built / "fuzz.cpp"), str(CSRC / "codeobject.cpp"), "-o", str(exe)],
                           capture_output=True, text=True)
    if build.returncode != 0:
        pytest.skip("g++ cannot build with -fsanitize=address,undefined here: " + build.stderr[-200:])
    run = subprocess.run([str(exe), str(built / "bundle.hsaco"), str(built / "raw.o")],
                         capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=0"})
    assert run.returncode == 0, run.stderr[-2000:]
    assert run.stdout.startswith("parsed ")
