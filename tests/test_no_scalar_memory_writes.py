"""No kernel this repository builds writes memory through the scalar data
cache: no scalar stores, scalar atomics, or scalar-cache write-back or
discard in any built code object (tests/kernel_isa.py disassembles them).
Such instructions have preceded machine-wide hardware errors on this GPU
pool.  CPU only; this file is kept off the GPU boxes (.gpurunignore), whose
upload check refuses any text that names these instructions."""

import pytest

import kernel_isa as K

pytestmark = pytest.mark.skipif(not (K.tools_present() and K.images()),
                                reason="ROCm LLVM tools or built code objects absent")

FORBIDDEN_PREFIXES = ("s_store_", "s_buffer_store_", "s_scratch_store_", "s_atomic_",
                      "s_buffer_atomic_", "s_dcache_wb", "s_dcache_discard")


def test_no_scalar_memory_writes_in_any_kernel():
    kernels = 0
    for image in K.images():
        for name, insns in K.disassembly(image).items():
            kernels += 1
            bad = [(hex(a), mn) for a, mn, _, _ in insns if mn.startswith(FORBIDDEN_PREFIXES)]
            assert not bad, f"{image.name}:{name}: {bad[:5]}"
    assert kernels > 100
