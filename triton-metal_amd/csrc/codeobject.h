/*
 * Argument layouts of the kernels in an AMDGPU code object, read from its
 * metadata note, so that a launch through the C ABI can be checked against
 * what each kernel declares before anything reaches the GPU.
 *
 * The reference binds launch argument i to kernel parameter i by position
 * (Sources/TritonMetalCore/Compiler.swift:390-401).  A gfx950 kernel reads its
 * parameters from a byte block whose layout is fixed at compile time (the
 * `amdhsa.kernels[].args` list of the code object's NT_AMDGPU_METADATA note),
 * and reads implicit values such as the grid size from the bytes after it.  A
 * launch that packs a different layout makes the kernel read garbage, which
 * can become an out-of-bounds access; comparing the two on the host refuses
 * such a launch instead.
 */
#ifndef TM_CODEOBJECT_H
#define TM_CODEOBJECT_H

#include <cstddef>
#include <map>
#include <string>
#include <vector>

namespace tm_codeobject {

/* One explicit kernel parameter: byte offset and size in the argument block,
 * and the metadata's value kind ("global_buffer", "by_value", ...). */
struct ArgSlot {
  long offset = 0;
  long size = 0;
  std::string kind;
};

/* The explicit (non-hidden) parameters of every kernel in `image`, a raw
 * AMDGPU ELF or a clang offload bundle holding one.  Kernels are keyed by
 * name.  Returns an empty map when the image carries no metadata this reader
 * understands (for example a compressed bundle); the caller then skips the
 * check.  Never throws. */
std::map<std::string, std::vector<ArgSlot>> read_kernel_arguments(const void *image,
                                                                   size_t size);

}  // namespace tm_codeobject

#endif
