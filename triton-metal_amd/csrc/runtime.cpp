/*
 * libtritonmetal.so — the tm_* C ABI over HIP, for AMD gfx950 (MI355X).
 *
 * The reference's Swift core (Sources/TritonMetalCore/Runtime.swift and the
 * @_cdecl exports in Compiler.swift:172-479) turns these entry points into
 * Metal calls.  Here they become HIP module calls:
 *
 *   library  = hipModule_t  (hipModuleLoadData of a gfx950 code object, of a
 *              hiprtc build of HIP source, or of the built-in kernel images
 *              linked into this library)
 *   kernel   = hipFunction_t, or a built-in kernel whose launch is planned here
 *   buffer   = hipMalloc'd HBM
 *   launch   = hipModuleLaunchKernel on one library-owned stream
 *
 * Built-in kernels carry the reference's names and argument lists
 * (matmul_kernel, attn_fwd, attn_bwd_preprocess, attn_bwd_dq, attn_bwd_dkdv, and
 * the fused SAE encoder sae_encode_kernel).
 * Their planner checks every argument on the host (kinds, signs, buffer
 * extents), picks the device function for the shape and fills a by-value
 * argument block (tm_args.h), so no malformed request reaches the GPU.
 */
#include "../../include/tritonmetal.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "codeobject.h"
#include "scratch.h"
#include "tm_args.h"

/* Query rows and threads per workgroup of the specialised forward kernels
 * (tm_attn_fwd_fast_*: 32 query rows per wave). */
#ifndef TM_FWD_FAST_ROWS
#define TM_FWD_FAST_ROWS 128
#endif
#ifndef TM_FWD_FAST_THREADS
#define TM_FWD_FAST_THREADS 256
#endif

namespace {

/* ---- errors ----------------------------------------------------------------
 * One process-wide slot under a lock; taking it clears it
 * (reference Compiler.swift:461-479). */

struct TmError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

std::mutex g_error_lock;
std::string g_error;
bool g_has_error = false;

void store_error(const std::string &message) {
  std::lock_guard<std::mutex> guard(g_error_lock);
  g_error = message;
  g_has_error = true;
}

std::string format(const char *fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return buf;
}

char *dup_string(const std::string &s) { return strdup(s.c_str()); }

void hip_check(hipError_t status, const char *what) {
  if (status != hipSuccess)
    throw TmError(format("%s failed: %s (%s)", what, hipGetErrorName(status),
                         hipGetErrorString(status)));
}

/* ---- device ----------------------------------------------------------------*/

struct Device {
  bool present = false;
  std::string absent_reason;
  std::string name;
  std::string arch;
  hipStream_t stream = nullptr;
  int compute_units = 0;
};

Device &device() {
  static Device dev;
  static std::once_flag once;
  std::call_once(once, [] {
    int count = 0;
    hipError_t status = hipGetDeviceCount(&count);
    if (status != hipSuccess || count <= 0) {
      dev.absent_reason = format("no HIP device on this machine (hipGetDeviceCount: %s)",
                                 hipGetErrorName(status));
      (void)hipGetLastError();
      return;
    }
    hipDeviceProp_t prop;
    if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&prop, 0) != hipSuccess) {
      dev.absent_reason = "could not query HIP device 0";
      (void)hipGetLastError();
      return;
    }
    dev.name = prop.name;
    dev.arch = prop.gcnArchName;
    dev.compute_units = prop.multiProcessorCount;
    /* Default priority on purpose: every stream of this library runs at the
     * same priority as torch's and HIP's null stream. */
    if (hipStreamCreateWithFlags(&dev.stream, hipStreamNonBlocking) != hipSuccess) {
      dev.absent_reason = "could not create a HIP stream on device 0";
      (void)hipGetLastError();
      return;
    }
    dev.present = true;
  });
  return dev;
}

Device &require_device() {
  Device &dev = device();
  if (!dev.present) throw TmError("no HIP device available: " + dev.absent_reason);
  return dev;
}

/* ---- built-in code objects --------------------------------------------------
 * The kernel images are linked into this library by blobs.S (generated at build
 * time) as a table of [start, end) pairs. */

extern "C" {
struct TmBlob {
  const char *start;
  const char *end;
};
extern const TmBlob tm_builtin_blob_table[];
extern const int32_t tm_builtin_blob_count;
}

struct BuiltinModules {
  std::vector<hipModule_t> modules;
  std::map<std::string, hipFunction_t> functions;
  std::mutex lock;
};

BuiltinModules &builtin_modules() {
  static BuiltinModules mods;
  return mods;
}

/* Load the built-in kernel images once (caller holds mods.lock). */
void load_builtin_modules(BuiltinModules &mods) {
  if (!mods.modules.empty()) return;
  for (int i = 0; i < tm_builtin_blob_count; ++i) {
    hipModule_t mod;
    hip_check(hipModuleLoadData(&mod, tm_builtin_blob_table[i].start),
              "hipModuleLoadData (built-in kernels)");
    mods.modules.push_back(mod);
  }
}

hipFunction_t builtin_function(const std::string &symbol) {
  require_device();
  BuiltinModules &mods = builtin_modules();
  std::lock_guard<std::mutex> guard(mods.lock);
  load_builtin_modules(mods);
  auto it = mods.functions.find(symbol);
  if (it != mods.functions.end()) return it->second;
  for (hipModule_t mod : mods.modules) {
    hipFunction_t fn;
    if (hipModuleGetFunction(&fn, mod, symbol.c_str()) == hipSuccess) {
      mods.functions[symbol] = fn;
      return fn;
    }
    (void)hipGetLastError();
  }
  throw TmError("built-in device function '" + symbol + "' is missing from the kernel images");
}

/* ---- objects and the handle table (reference Runtime.swift:250-290) -------- */

enum class Kind { Library, Kernel, Buffer };

struct Object {
  virtual ~Object() = default;
  virtual Kind kind() const = 0;
};

enum class Element { F32, F16, BF16 };

const char *element_name(Element e) {
  switch (e) {
    case Element::F32: return "f32";
    case Element::F16: return "f16";
    case Element::BF16: return "bf16";
  }
  return "?";
}
int element_size(Element e) { return e == Element::F32 ? 4 : 2; }

struct BuiltinSpec {
  Element element = Element::F32;
  int head_dim = 64;
  bool causal = false;
  /* bwd=atomic: the library also offers attn_bwd_fused, a backward in one
   * call (one dK/dV/dQ kernel, dQ summed with floating-point atomics, not
   * deterministic).  The reference's split (attn_bwd_dq + attn_bwd_dkdv)
   * stays available in every library. */
  enum class Bwd { Split, Atomic } bwd = Bwd::Split;

  std::string text() const {
    return format("builtin element=%s head_dim=%d causal=%d%s", element_name(element), head_dim,
                  causal ? 1 : 0,
                  bwd == Bwd::Atomic ? " bwd=atomic" : "");
  }
};

struct Library : Object {
  Kind kind() const override { return Kind::Library; }
  bool builtin = false;
  BuiltinSpec spec;
  hipModule_t module = nullptr; /* user code object (not built-in) */
  /* explicit parameters of each kernel, from the code object's metadata
   * (empty when the image carries none this library can read) */
  std::map<std::string, std::vector<tm_codeobject::ArgSlot>> signatures;
  /* work memory of planned dispatch sequences (GEMM K-range partials, the
   * generic attention kernels' range partials, the fp32 dQ accumulator of
   * attn_bwd_fused): see plan_workspace */
  mutable std::mutex workspace_lock;
  mutable void *workspace = nullptr;
  mutable size_t workspace_bytes = 0;
  /* held by a launch from planning (which may hand out, grow or shrink the
   * workspace) until its whole dispatch sequence is queued: two threads
   * launching on one library then neither free a workspace the other's
   * planned dispatches still bind nor interleave their sequences */
  std::mutex launch_lock;
  ~Library() override {
    if (!module && !workspace) return;
    /* a dispatch of one of its kernels may still be queued (tm_launch_async):
     * drain the library stream before the code object or workspace goes away */
    Device &dev = device();
    if (dev.present) (void)hipStreamSynchronize(dev.stream);
    if (workspace) (void)hipFree(workspace);
    if (module) (void)hipModuleUnload(module);
  }
};

enum class Builtin { None, Matmul, AttnFwd, AttnPre, AttnDq, AttnDkdv, AttnFused, SaeEncode, Probe };

struct Kernel : Object {
  Kind kind() const override { return Kind::Kernel; }
  std::shared_ptr<Library> library; /* keeps a user module alive */
  std::string name;
  Builtin builtin = Builtin::None;
  hipFunction_t function = nullptr; /* user kernels */
  bool has_signature = false;                     /* user kernels: declared parameters known */
  std::vector<tm_codeobject::ArgSlot> signature;
  std::mutex lock;
  std::string last_variant;
};

/* A buffer lives in HBM.  tm_buffer_contents gives it a host mirror (pinned
 * host memory, filled from HBM on that first call): the host address a
 * reference caller reads and writes through, as it does the unified memory
 * of the reference's buffers (Compiler.swift:306-311).  While a mirror exists
 * it is the buffer's contents outside launches: tm_buffer_write updates both
 * copies, tm_buffer_read reads the mirror, and a launch that binds the buffer
 * copies the mirror to HBM before the dispatch and back after it completes
 * (the launch then waits, even tm_launch_async).  Buffers without a mirror
 * (the hot path) are never copied. */
struct Buffer : Object {
  Kind kind() const override { return Kind::Buffer; }
  void *ptr = nullptr;
  int64_t length = 0;
  void *host = nullptr; /* the mirror, once tm_buffer_contents was called */
  std::mutex host_lock;
  ~Buffer() override {
    if (host) (void)hipHostFree(host);
    if (ptr) (void)hipFree(ptr);
  }
};

class HandleTable {
 public:
  int64_t insert(std::shared_ptr<Object> obj) {
    std::lock_guard<std::mutex> guard(lock_);
    const int64_t handle = next_++;
    storage_[handle] = std::move(obj);
    return handle;
  }

  template <typename T>
  std::shared_ptr<T> lookup(int64_t handle, Kind kind, const char *what) {
    std::lock_guard<std::mutex> guard(lock_);
    auto it = storage_.find(handle);
    if (it == storage_.end())
      throw TmError(format("%s handle %lld is not live", what, (long long)handle));
    if (it->second->kind() != kind)
      throw TmError(format("handle %lld is not a %s", (long long)handle, what));
    return std::static_pointer_cast<T>(it->second);
  }

  bool remove(int64_t handle, Kind kind) {
    std::shared_ptr<Object> doomed;
    {
      std::lock_guard<std::mutex> guard(lock_);
      auto it = storage_.find(handle);
      if (it == storage_.end() || it->second->kind() != kind) return false;
      doomed = std::move(it->second);
      storage_.erase(it);
    }
    return true; /* the object is destroyed outside the lock */
  }

  int64_t count() {
    std::lock_guard<std::mutex> guard(lock_);
    return (int64_t)storage_.size();
  }

 private:
  std::mutex lock_;
  std::unordered_map<int64_t, std::shared_ptr<Object>> storage_;
  int64_t next_ = 1;
};

HandleTable &handles() {
  static HandleTable table;
  return table;
}

/* ---- built-in library specs -------------------------------------------------
 * "builtin [element=f32|f16|bf16] [head_dim=N] [causal=0|1]": the
 * specialisation the reference bakes into each ttir module (the element type
 * of every pointer argument and the HEAD_DIM constexpr) plus the causal mask,
 * which the reference does not have. */

bool is_builtin_spec(const char *text) {
  while (*text == ' ' || *text == '\n' || *text == '\t') ++text;
  return strncmp(text, "builtin", 7) == 0 &&
         (text[7] == 0 || text[7] == ' ' || text[7] == '\n' || text[7] == '\t');
}

BuiltinSpec parse_spec(const char *text) {
  std::istringstream in(text);
  std::string word;
  in >> word; /* "builtin" */
  BuiltinSpec spec;
  while (in >> word) {
    const size_t eq = word.find('=');
    if (eq == std::string::npos)
      throw TmError("built-in library spec: expected key=value, got '" + word + "'");
    const std::string key = word.substr(0, eq), value = word.substr(eq + 1);
    if (key == "element") {
      if (value == "f32" || value == "float32") spec.element = Element::F32;
      else if (value == "f16" || value == "float16") spec.element = Element::F16;
      else if (value == "bf16" || value == "bfloat16") spec.element = Element::BF16;
      else throw TmError("built-in library spec: unsupported element '" + value + "'");
    } else if (key == "head_dim") {
      char *end = nullptr;
      const long d = strtol(value.c_str(), &end, 10);
      if (!end || *end || d < 1 || d > 128)
        throw TmError("built-in library spec: head_dim must be an integer in 1..128, got '" +
                      value + "'");
      spec.head_dim = (int)d;
    } else if (key == "causal") {
      if (value == "0" || value == "false") spec.causal = false;
      else if (value == "1" || value == "true") spec.causal = true;
      else throw TmError("built-in library spec: causal must be 0 or 1, got '" + value + "'");
    } else if (key == "bwd") {
      if (value == "split") spec.bwd = BuiltinSpec::Bwd::Split;
      else if (value == "atomic") spec.bwd = BuiltinSpec::Bwd::Atomic;
      else throw TmError("built-in library spec: bwd must be split or atomic, got '" + value + "'");
    } else {
      throw TmError("built-in library spec: unknown key '" + key + "'");
    }
  }
  return spec;
}

struct BuiltinInfo {
  Builtin id;
  const char *name;
  std::vector<int> kinds;  /* the reference's argument kinds, in order */
  std::vector<const char *> dtypes;
  int optional_tail;       /* trailing arguments that may be omitted */
};

const std::vector<BuiltinInfo> &builtin_table() {
  static const std::vector<BuiltinInfo> table = {
      {Builtin::Matmul, "matmul_kernel", {0, 0, 0, 1, 1, 1, 1, 1, 1, 1, 1, 1},
       {"E", "E", "E", "i32", "i32", "i32", "i32", "i32", "i32", "i32", "i32", "i32"}, 0},
      {Builtin::AttnFwd, "attn_fwd", {0, 0, 0, 0, 2, 1, 1, 1, 0, 1},
       {"E", "E", "E", "E", "f32", "i32", "i32", "i32", "f32", "i32"}, 2},
      {Builtin::AttnPre, "attn_bwd_preprocess", {0, 0, 0, 1, 1, 1, 1},
       {"E", "E", "f32", "i32", "i32", "i32", "i32"}, 0},
      {Builtin::AttnDq, "attn_bwd_dq", {0, 0, 0, 0, 0, 0, 0, 2, 1, 1, 1, 1},
       {"E", "E", "E", "E", "E", "f32", "f32", "f32", "i32", "i32", "i32", "i32"}, 0},
      {Builtin::AttnDkdv, "attn_bwd_dkdv", {0, 0, 0, 0, 0, 0, 0, 0, 2, 1, 1, 1, 1},
       {"E", "E", "E", "E", "E", "E", "f32", "f32", "f32", "i32", "i32", "i32", "i32"}, 0},
      /* bwd=atomic libraries only: (Q, K, V, dO, dQ, dK, dV, L, Delta, sm_scale,
       * stride_head, stride_seq, stride_lse, n_ctx) */
      {Builtin::AttnFused, "attn_bwd_fused", {0, 0, 0, 0, 0, 0, 0, 0, 0, 2, 1, 1, 1, 1},
       {"E", "E", "E", "E", "E", "E", "E", "f32", "f32", "f32", "i32", "i32", "i32", "i32"}, 0},
      {Builtin::SaeEncode, "sae_encode_kernel", {0, 0, 0, 0, 1, 1, 1},
       {"E", "E", "E", "E", "i32", "i32", "i32"}, 0},
      {Builtin::Probe, "tm_probe", {0}, {"f32"}, 0},
  };
  return table;
}

const BuiltinInfo *find_builtin(const std::string &name) {
  for (const BuiltinInfo &info : builtin_table())
    if (name == info.name) return &info;
  return nullptr;
}

std::string builtin_names() {
  std::string out;
  for (const BuiltinInfo &info : builtin_table()) {
    if (!out.empty()) out += ", ";
    out += info.name;
  }
  return out;
}

/* Workgroup shape each built-in runs at (published through tm_kernel_info). */
struct Published {
  int threads;
  std::vector<int> block_shape;
};

Published published_shape(Builtin id) {
  switch (id) {
    case Builtin::Matmul: return {256, {64, 64}}; /* 512 threads, 256 x 256 on the fast path */
    case Builtin::AttnFwd: return {256, {64}};
    case Builtin::AttnPre: return {256, {64}};
    case Builtin::AttnDq: return {256, {64}};
    case Builtin::AttnDkdv: return {256, {64}};
    case Builtin::AttnFused: return {256, {128}};
    case Builtin::SaeEncode: return {256, {64, 64}}; /* SAEEncoder.swift Blocking() */
    case Builtin::Probe: return {64, {256}};
    default: return {256, {1}};
  }
}

/* ---- launch arguments ------------------------------------------------------ */

struct Arg {
  int kind;
  int64_t value;
  std::shared_ptr<Buffer> buffer; /* kind 0 */
};

std::vector<Arg> decode_args(const int32_t *kinds, const int64_t *values, int32_t argc) {
  std::vector<Arg> args;
  if (argc < 0) throw TmError(format("tm_launch received a negative argument count %d", argc));
  if (argc > 0 && (!kinds || !values)) throw TmError("tm_launch received NULL argument arrays");
  for (int i = 0; i < argc; ++i) {
    Arg a{kinds[i], values[i], nullptr};
    switch (kinds[i]) {
      case TM_ARG_BUFFER:
        a.buffer = handles().lookup<Buffer>(values[i], Kind::Buffer, "buffer");
        break;
      case TM_ARG_I32:
      case TM_ARG_F32:
      case TM_ARG_I64:
        break;
      default:
        throw TmError(format("unknown launch argument kind %d at position %d", kinds[i], i));
    }
    args.push_back(a);
  }
  return args;
}

int32_t as_i32(const Arg &a) { return (int32_t)(uint32_t)(a.value & 0xffffffffu); }
float as_f32(const Arg &a) {
  const uint32_t bits = (uint32_t)(a.value & 0xffffffffu);
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* A planned dispatch: device function, geometry and the by-value argument block. */
struct Plan {
  /* several dispatches in order (attn_bwd_fused); the fields below are then
   * those of the main one, for reporting */
  std::vector<Plan> sequence;
  hipFunction_t function = nullptr;
  std::string variant;
  unsigned grid[3] = {1, 1, 1};
  unsigned block = 0; /* must be set by the planner; 0 is refused at enqueue */
  std::vector<unsigned char> kernarg; /* packed bytes */
  bool empty = false;                 /* nothing to compute (a zero-sized problem) */
  bool by_value_struct = true;        /* built-in: one struct argument */
};

template <typename S>
void set_kernarg(Plan &plan, const S &s) {
  plan.kernarg.resize(sizeof(S));
  memcpy(plan.kernarg.data(), &s, sizeof(S));
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

/* Elements a strided 2-D access touches, from element 0: the host-side proof
 * that a kernel stays inside its buffer. */
/* Saturates at INT64_MAX (int32 sizes and strides cannot reach it in a
 * buffer that exists, but a caller's arithmetic must not wrap a check). */
int64_t extent(int64_t rows, int64_t row_stride, int64_t cols, int64_t col_stride) {
  if (rows <= 0 || cols <= 0) return 0;
  const __int128 e = (__int128)(rows - 1) * row_stride + (__int128)(cols - 1) * col_stride + 1;
  return e > (__int128)INT64_MAX ? INT64_MAX : (int64_t)e;
}

/* a + b for non-negative sizes, saturating like extent() */
int64_t sat_add(int64_t a, int64_t b) { return a > INT64_MAX - b ? INT64_MAX : a + b; }

void require_extent(const Arg &a, int64_t elements, int esize, const char *kernel, int index,
                    const char *what) {
  if (elements > a.buffer->length / esize) {
    const __int128 need = (__int128)elements * esize;
    throw TmError(format("%s argument %d (%s) needs %lld bytes but its buffer holds %lld", kernel,
                         index, what, need > (__int128)INT64_MAX ? (long long)INT64_MAX : (long long)need,
                         (long long)a.buffer->length));
  }
}

void require_nonneg(int64_t v, const char *kernel, const char *what) {
  if (v < 0) throw TmError(format("%s: %s must be non-negative, got %lld", kernel, what,
                                  (long long)v));
}

void check_signature(const BuiltinInfo &info, const std::vector<Arg> &args) {
  const int full = (int)info.kinds.size();
  const int argc = (int)args.size();
  if (argc != full && !(info.optional_tail && argc == full - info.optional_tail)) {
    if (info.optional_tail)
      throw TmError(format("%s expects %d or %d arguments, got %d", info.name,
                           full - info.optional_tail, full, argc));
    throw TmError(format("%s expects %d arguments, got %d", info.name, full, argc));
  }
  static const char *kind_names[] = {"a buffer", "an i32", "an f32", "an i64"};
  for (int i = 0; i < argc; ++i)
    if (args[i].kind != info.kinds[i])
      throw TmError(format("%s argument %d must be %s (kind %d), got kind %d", info.name, i,
                           kind_names[info.kinds[i]], info.kinds[i], args[i].kind));
}

/* TRITON_METAL_GENERIC=1 keeps every dispatch on the generic kernels (for A/B
 * comparisons of the specialised ones). */
bool fast_paths_enabled() {
  static const bool enabled = [] {
    const char *v = getenv("TRITON_METAL_GENERIC");
    return !(v && *v && strcmp(v, "0") != 0);
  }();
  return enabled;
}

/* The specialised attention kernels need a 16-bit element type, head_dim 64
 * or 128, 16-byte aligned rows and a positive finite scale. */
/* The fast kernels copy K/V/Q/dO tiles through a buffer resource based at a
 * head's first row: a head's rows must span fewer than 2^31 bytes. */
bool attn_fast_ok(const BuiltinSpec &spec, int32_t stride_head, int32_t stride_seq,
                  int32_t n_ctx, float sm_scale) {
  const int64_t head_bytes =
      ((int64_t)(n_ctx > 0 ? n_ctx - 1 : 0) * stride_seq + spec.head_dim) * 2;
  return fast_paths_enabled() && spec.element != Element::F32 &&
         (spec.head_dim == 64 || spec.head_dim == 128) && stride_seq % 8 == 0 &&
         stride_head % 8 == 0 && std::isfinite(sm_scale) && sm_scale > 0.f &&
         head_bytes <= INT32_MAX;
}

int padded_head_dim(int d) { return d <= 32 ? 32 : d <= 64 ? 64 : d <= 96 ? 96 : 128; }

std::string attn_symbol(const char *op, const BuiltinSpec &spec) {
  return format("tm_attn_%s_generic_%s_d%d%s", op, element_name(spec.element),
                padded_head_dim(spec.head_dim), spec.causal ? "_causal" : "");
}

void validate_attn_common(const char *name, int64_t heads, int32_t stride_head,
                          int32_t stride_seq, int32_t n_ctx, int head_dim) {
  require_nonneg(stride_head, name, "stride_head");
  require_nonneg(n_ctx, name, "n_ctx");
  if (stride_seq < head_dim && n_ctx > 1)
    throw TmError(format("%s: stride_seq %d is smaller than head_dim %d (rows would overlap)",
                         name, stride_seq, head_dim));
  if (heads > 65535) throw TmError(format("%s: %lld heads exceeds 65535", name, (long long)heads));
}

/* TRITON_METAL_GEMM_W4=0 keeps whole 256 x 256-tile row-major GEMMs on the
 * 8-wave kernel instead of the 4-wave one (A/B comparisons). */
bool gemm_w4_enabled() {
  static const bool enabled = [] {
    const char *v = getenv("TRITON_METAL_GEMM_W4");
    return !(v && strcmp(v, "0") == 0);
  }();
  return enabled;
}


/* 0 turns the bf16/f16 GEMM's K split across workgroups off (measurement builds) */
#ifndef TM_GEMM_SPLITK
#define TM_GEMM_SPLITK 1
#endif

/* 0 turns the bf16/f16 GEMM's intra-workgroup K split off (measurement builds) */
#ifndef TM_GEMM_KSPLIT
#define TM_GEMM_KSPLIT 1
#endif

/* Kernel choice shared by matmul_kernel and sae_encode_kernel.  The
 * specialised kernels take 16-bit elements and row-major operands with unit
 * inner stride, 16-byte aligned rows of A and B, 8-byte aligned rows of C,
 * and rows no shorter than the matrix (lda >= K, ldb >= N): whole tiles (and
 * K a multiple of 64) run the aligned kernel, any other M, N, K the ragged
 * one, whose copies clip at the matrix's last row and whose last k-step and
 * stores are masked.  Either operand (not both) may instead be stored
 * transposed: B with unit stride along K (the x @ W^T layout), read like A,
 * or A with unit stride along M (dY^T X), read like B.  fp32 with the same
 * layouts, 16-byte aligned rows and whole 128 x 128 (or, for problems with
 * few of those, 64 x 64) x 32 tiles runs the fp32 MFMA kernel.  Anything else
 * runs the generic 64 x 64 kernel. */
void choose_gemm(Plan &plan, const TmGemmArgs &p, const BuiltinSpec &spec, const char *family) {
  const char *el = element_name(spec.element);
  /* fp32: whole 128 x 128 x 32 tiles on the fp32 MFMA kernel when there are
   * at least half as many of them as compute units, else whole 64 x 64 tiles
   * (1024^3 ran 29 TFLOP/s on 64 tiles of 128 x 128; 2048^3 runs 116) */
  const bool gemm = strcmp(family, "gemm") == 0;
  const bool f32_big = p.m % 128 == 0 && p.n % 128 == 0 &&
                       2 * (int64_t)(p.m / 128) * (p.n / 128) >= std::max(device().compute_units, 1);
  if (fast_paths_enabled() && spec.element == Element::F32 && p.scn == 1 && p.m % 64 == 0 &&
      p.n % 64 == 0 && p.k % 32 == 0 && p.k > 0 && p.scm % 4 == 0) {
    /* either operand (matmul only, not both) may be stored transposed */
    const bool a_n = p.sak == 1 && p.sam % 4 == 0 && p.sam >= p.k;
    const bool a_t = gemm && !a_n && p.sam == 1 && p.sak % 4 == 0 && p.sak >= p.m;
    const bool b_n = p.sbn == 1 && p.sbk % 4 == 0 && p.sbk >= p.n;
    const bool b_t = gemm && !b_n && p.sbk == 1 && p.sbn % 4 == 0 && p.sbn >= p.k;
    if ((a_n || a_t) && (b_n || b_t) && !(a_t && b_t)) {
      const int tile = f32_big ? 128 : 64;
      const int64_t tiles = (int64_t)(p.m / tile) * (p.n / tile);
      /* About one workgroup per CU or fewer (one wave per SIMD): split the K
       * loop over 2 (128 x 128 tiles) or up to 4 (64 x 64) groups of waves
       * inside the workgroup (plain row-major matmul only) */
      int64_t kg = 1;
      if (gemm && a_n && b_n) {
        const int64_t cus = std::max(device().compute_units, 1);
        kg = std::min<int64_t>({2 * cus / std::max<int64_t>(tiles, 1), f32_big ? 2 : 4, p.k / 32});
        kg = kg >= 4 ? 4 : kg >= 2 ? 2 : 1;
      }
      plan.variant = format("tm_%s_fast%s%s%s_f32", family, b_t ? "_nt" : a_t ? "_tn" : "",
                            f32_big ? "" : "_t64", kg > 1 ? (kg == 4 ? "_k4" : "_k2") : "");
      plan.grid[0] = (unsigned)tiles;
      plan.block = (unsigned)(256 * kg);
      return;
    }
  }
  const bool half = fast_paths_enabled() && spec.element != Element::F32 && p.scn == 1 &&
                    p.k > 0 && p.scm % 4 == 0;
  /* A row-major [M, K], or (matmul only) stored transposed: element (m, k) at
   * k * stride_ak + m, the dY^T X layout */
  const bool a_n = half && p.sak == 1 && p.sam % 8 == 0 && p.sam >= p.k && p.sam <= (1 << 26);
  const bool a_t = half && !a_n && gemm && p.sam == 1 && p.sak % 8 == 0 && p.sak >= p.m &&
                   p.sak <= (1 << 26);
  /* B row-major [K, N], or (matmul only) stored transposed: element (k, n) at
   * n * stride_bn + k, the x @ W^T layout */
  const bool b_n = p.sbn == 1 && p.sbk % 8 == 0 && p.sbk >= p.n && p.sbk <= (1 << 26);
  const bool b_t = !b_n && gemm && p.sbk == 1 && p.sbn % 8 == 0 && p.sbn >= p.k && p.sbn <= (1 << 26);
  const bool nn = a_n && b_n, nt = a_n && b_t, tn = a_t && b_n;
  if (nn || nt || tn) {
    /* 256 x 256 tiles (512 threads, one resident per compute unit) or 128 x
     * 128 tiles (256 threads, two resident), whichever needs less time by
     * rounds of resident tiles: a round of 256 x 256 tiles takes about 31/21
     * of a round of 128 x 128 pairs (4x the work at 1.3/0.95 the rate; on one
     * MI355X 2560^3 runs 747 vs 504 TFLOP/s on 128 x 128 tiles, 3072^3 745 vs
     * 650 on 256 x 256) */
    const int64_t cus = std::max(device().compute_units, 1);
    const bool big = cdiv(cdiv(p.m, 256) * cdiv(p.n, 256), cus) * 31 <=
                     cdiv(cdiv(p.m, 128) * cdiv(p.n, 128), 2 * cus) * 21;
    /* with fewer 128 x 128 tiles than compute units, 64 x 64 tiles (128
     * threads): 1024^3 bf16 had 64 tiles of 128 x 128 */
    const bool small = !big && cdiv(p.m, 128) * cdiv(p.n, 128) < cus;
    const int tile = big ? 256 : small ? 64 : 128;
    const bool whole = p.m % tile == 0 && p.n % tile == 0 && p.k % 64 == 0;
    const int64_t tiles = cdiv(p.m, tile) * cdiv(p.n, tile);
    /* whole row-major tiles with fewer 128 x 128 workgroups than two per CU
     * (one wave per SIMD), or 64 x 64 ones (two waves each): the K loop split
     * over wave groups inside the workgroup -- 128 x 128 tiles over 2 (512
     * threads); 64 x 64 tiles over 4 (512 threads, one workgroup per CU) up to
     * one tile per CU, else over 2 (256 threads, two per CU) up to two */
    const bool ksplit = TM_GEMM_KSPLIT && gemm && nn && whole && !big && p.k >= 128 &&
                        (small ? tiles <= 2 * cus : tiles < 2 * cus);
    const int kg = !ksplit ? 1 : small && tiles > cus ? 2 : small ? 4 : 2;
    plan.variant = format("tm_%s_%s%s%s%s_%s", family, whole ? "fast" : "ragged",
                          nt ? "_nt" : tn ? "_tn" : "", big ? "" : small ? "_t64" : "_t128",
                          kg == 4 ? "_k4" : kg == 2 ? "_k2" : "", el);
    plan.grid[0] = (unsigned)tiles;
    plan.block = (unsigned)(2 * tile * kg);
    /* whole 256 x 256 tiles: the 4-wave kernel (gemm_w4.hip), whose copies
     * address a step's tile of each operand through one 32-bit buffer range:
     * 256 stored rows of a K-contiguous operand (A row-major, B transposed),
     * 64 of the other kind */
    const int64_t a_rows = a_n ? (int64_t)p.sam * 512 : (int64_t)p.sak * 128;
    const int64_t b_rows = b_t ? (int64_t)p.sbn * 512 : (int64_t)p.sbk * 128;
    if (gemm_w4_enabled() && whole && big && a_rows <= INT32_MAX && b_rows <= INT32_MAX) {
      plan.variant = format("tm_%s_w4%s_%s", family, nt ? "_nt" : tn ? "_tn" : "", el);
      plan.block = 256;
    }
  } else {
    plan.variant = format("tm_%s_generic_%s", family, el);
    plan.grid[0] = (unsigned)cdiv(p.m, 64);
    plan.grid[1] = (unsigned)cdiv(p.n, 64);
    plan.block = 256;
  }
}

void finish(hipStream_t stream);

/* attn_bwd_fused as three dispatches: clear the fp32 accumulator (a kernel,
 * not hipMemsetAsync, so a captured graph replays it correctly), the fused
 * dK/dV/dQ pass, then dQ = sm_scale * accumulator in the element type.
 * `acc` holds `count` = heads * n_ctx * head_dim floats. */
void plan_fused_backward(Plan &plan, const BuiltinSpec &spec, const TmAttnDkdvArgs &kv, void *dq,
                         float *acc, int64_t count) {
  const char *el = element_name(spec.element);
  TmAttnDqAccArgs a{};
  a.acc = acc;
  a.dq = dq;
  a.count = count;
  a.sm_scale = kv.sm_scale;
  a.stride_head = kv.stride_head;
  a.stride_seq = kv.stride_seq;
  a.n_ctx = kv.n_ctx;
  a.heads = kv.heads;
  Plan zero, main, convert;
  zero.variant = "tm_attn_dq_acc_zero";
  zero.grid[0] = (unsigned)cdiv(count, 1024);
  zero.block = 256;
  set_kernarg(zero, a);
  TmAttnFusedArgs f{};
  f.kv = kv;
  f.dq_acc = acc;
  main.variant = format("tm_attn_fused_fast_%s_d%d%s", el, spec.head_dim,
                        spec.causal ? "_causal" : "");
  main.grid[0] = (unsigned)(cdiv(kv.n_ctx, 128) * kv.heads);
  main.block = 256;
  set_kernarg(main, f);
  convert.variant = format("tm_attn_dq_convert_%s_d%d", el, spec.head_dim);
  convert.grid[0] = (unsigned)cdiv((int64_t)kv.heads * kv.n_ctx, 256 / (spec.head_dim / 8));
  convert.block = 256;
  set_kernarg(convert, a);
  for (Plan *part : {&zero, &main, &convert}) part->function = builtin_function(part->variant);
  plan.variant = main.variant;
  plan.function = main.function;
  plan.block = main.block;
  plan.sequence = {zero, main, convert};
}

/* Device memory a planned dispatch may use instead of allocating its own work
 * buffer: tm_launch_noalloc passes the static scratch (scratch.hip). */
struct Scratch {
  void *ptr = nullptr;
  size_t bytes = 0;
};

/* A workspace above this size is given back when a later sequence needs less
 * than a quarter of it, so one large request does not pin its memory for the
 * library's lifetime. */
constexpr size_t kWorkspaceKeepBytes = (size_t)256 << 20;

/* `need` bytes of device work memory for one planned dispatch sequence: the
 * static scratch under tm_launch_noalloc (nullptr when it is too small), else
 * the library's workspace, grown on demand and shrunk after a large request.
 * Dispatches of one library run in order on its stream, so consecutive
 * sequences may share the workspace; the caller holds the library's
 * launch_lock until its sequence is queued, so no other launch replaces the
 * workspace in between. */
void *plan_workspace(const Library &lib, size_t need, const Scratch *scratch) {
  if (scratch) return need <= scratch->bytes ? scratch->ptr : nullptr;
  std::lock_guard<std::mutex> guard(lib.workspace_lock);
  const bool shrink = lib.workspace_bytes > kWorkspaceKeepBytes && need < lib.workspace_bytes / 4;
  if (lib.workspace_bytes < need || shrink) {
    /* the old workspace may still be bound to a queued dispatch */
    if (lib.workspace) {
      finish(require_device().stream);
      hip_check(hipFree(lib.workspace), "hipFree");
      lib.workspace = nullptr;
      lib.workspace_bytes = 0;
    }
    hip_check(hipMalloc(&lib.workspace, need), "hipMalloc (workspace)");
    lib.workspace_bytes = need;
  }
  return lib.workspace;
}

/* bf16/f16 GEMMs on 64 x 64 tiles with too few tiles to fill the chip (a
 * few rows against a large N K, or a small M N with a long K): the K loop
 * split across workgroups into `splits` ranges (grid y), each writing an fp32
 * partial product, then a reduce dispatch that sums them in range order into
 * C.  Target: about four 2-wave workgroups per CU (one 8-wave K-group
 * workgroup), at least two k-steps per wave group and range.  Returns false
 * (plan untouched) when the split does not apply or no work memory is
 * available. */
bool plan_gemm_split(Plan &plan, TmGemmArgs &p, const BuiltinSpec &spec, const Library &lib,
                     const Scratch *scratch) {
  /* the split is compiled into "_ks" instantiations of the 64 x 64-tile
   * GEMM kernels only */
  if (!TM_GEMM_SPLITK || spec.element == Element::F32 || plan.variant.find("_t64") == std::string::npos ||
      plan.variant.rfind("tm_gemm_", 0) != 0)
    return false;
  const int64_t cus = std::max(device().compute_units, 1);
  const int64_t tiles = plan.grid[0];
  const int64_t kg = plan.block / 128; /* wave groups of the K split inside the workgroup */
  const int64_t ksteps = cdiv(p.k, 64);
  const int64_t target = (kg == 1 ? 4 : 1) * cus;
  const int64_t splits = std::min<int64_t>({target / std::max<int64_t>(tiles, 1), ksteps / (2 * kg), 16});
  if (splits < 2) return false;
  const int64_t np = (p.n + 3) & ~int64_t(3);
  void *work = plan_workspace(lib, (size_t)splits * (size_t)p.m * (size_t)np * 4, scratch);
  if (!work) return false;
  p.part = (float *)work;
  p.splits = (int32_t)splits;
  Plan main = plan, reduce;
  /* the "_ks" instantiation of the planned kernel */
  const std::string suffix = std::string("_") + element_name(spec.element);
  main.variant = plan.variant.substr(0, plan.variant.size() - suffix.size()) + "_ks" + suffix;
  main.grid[1] = (unsigned)splits;
  set_kernarg(main, p);
  reduce.variant = format("tm_gemm_split_reduce_%s", element_name(spec.element));
  reduce.grid[0] = (unsigned)cdiv((int64_t)p.m * (np / 4), 256);
  reduce.block = 256;
  set_kernarg(reduce, p);
  for (Plan *part : {&main, &reduce}) part->function = builtin_function(part->variant);
  plan.function = main.function;
  plan.variant = format("%s + %s (%d K ranges)", main.variant.c_str(), reduce.variant.c_str(),
                        (int)splits);
  plan.sequence = {main, reduce};
  return true;
}


/* Ranges to split a generic attention kernel's walk into when its grid of
 * `wgs` 64-row workgroups cannot fill the chip twice: enough to (at most 16,
 * each at least two 32-row blocks of the `n_ctx` walked); 1 for no split. */
int64_t split_ranges(int64_t wgs, int64_t n_ctx) {
  const int64_t cus = std::max(device().compute_units, 1);
  if (wgs >= 2 * cus) return 1;
  return std::max<int64_t>(1, std::min<int64_t>({cdiv(2 * cus, wgs), cdiv(n_ctx, 32) / 2, 16}));
}

/* The split form of a generic dq or dkdv plan: the main dispatch over
 * `splits` ranges (grid z) writing fp32 partials to `part`, then the reduce
 * dispatch that sums them into the outputs (dQ * sm_scale, or dK * sm_scale
 * and dV) in the element type. */
template <typename A>
void plan_split_backward(Plan &plan, const BuiltinSpec &spec, A p, float *part, int64_t splits,
                         void *out0, void *out1) {
  p.part = part;
  p.splits = (int32_t)splits;
  Plan main = plan, reduce;
  main.grid[2] = (unsigned)splits;
  set_kernarg(main, p);
  TmAttnSplitReduceArgs r{};
  r.part = part;
  r.out0 = out0;
  r.out1 = out1;
  r.scale0 = p.sm_scale;
  r.scale1 = 1.f;
  r.stride_head = p.stride_head;
  r.stride_seq = p.stride_seq;
  r.n_ctx = p.n_ctx;
  r.head_dim = p.head_dim;
  r.heads = p.heads;
  r.splits = (int32_t)splits;
  r.outputs = out1 ? 2 : 1;
  reduce.variant = format("tm_attn_split_reduce_%s", element_name(spec.element));
  reduce.grid[0] = (unsigned)cdiv((int64_t)p.heads * p.n_ctx, 4);
  reduce.block = 256;
  set_kernarg(reduce, r);
  for (Plan *part_plan : {&main, &reduce}) part_plan->function = builtin_function(part_plan->variant);
  plan.function = main.function;
  plan.variant = format("%s + %s (%d ranges)", main.variant.c_str(), reduce.variant.c_str(),
                        (int)splits);
  plan.sequence = {main, reduce};
}

Plan plan_builtin(Kernel &k, const Library &lib, const std::vector<Arg> &args, int64_t gx,
                  int64_t gy, int64_t gz, const Scratch *scratch = nullptr) {
  const BuiltinInfo &info = *find_builtin(k.name);
  check_signature(info, args);
  const BuiltinSpec &spec = lib.spec;
  const int es = element_size(spec.element);
  const char *el = element_name(spec.element);
  const int64_t heads = gy * gz;
  Plan plan;

  switch (info.id) {
    case Builtin::Matmul: {
      TmGemmArgs p{};
      p.a = args[0].buffer->ptr;
      p.b = args[1].buffer->ptr;
      p.c = args[2].buffer->ptr;
      p.m = as_i32(args[3]);
      p.n = as_i32(args[4]);
      p.k = as_i32(args[5]);
      p.sam = as_i32(args[6]);
      p.sak = as_i32(args[7]);
      p.sbk = as_i32(args[8]);
      p.sbn = as_i32(args[9]);
      p.scm = as_i32(args[10]);
      p.scn = as_i32(args[11]);
      const char *nm = info.name;
      require_nonneg(p.m, nm, "M");
      require_nonneg(p.n, nm, "N");
      require_nonneg(p.k, nm, "K");
      require_nonneg(p.sam, nm, "stride_am");
      require_nonneg(p.sak, nm, "stride_ak");
      require_nonneg(p.sbk, nm, "stride_bk");
      require_nonneg(p.sbn, nm, "stride_bn");
      require_nonneg(p.scm, nm, "stride_cm");
      require_nonneg(p.scn, nm, "stride_cn");
      require_extent(args[0], extent(p.m, p.sam, p.k, p.sak), es, nm, 0, "A");
      require_extent(args[1], extent(p.k, p.sbk, p.n, p.sbn), es, nm, 1, "B");
      require_extent(args[2], extent(p.m, p.scm, p.n, p.scn), es, nm, 2, "C");
      if (p.m == 0 || p.n == 0) {
        plan.empty = true;
        return plan;
      }
      choose_gemm(plan, p, spec, "gemm");
      if (plan_gemm_split(plan, p, spec, lib, scratch)) return plan;
      set_kernarg(plan, p);
      break;
    }
    case Builtin::SaeEncode: {
      /* relu(x @ w + b) with x [M, D], w [D, F], b [F], out [M, F], all
       * row-major contiguous (SAEEncoder.swift:29-40). */
      const char *nm = info.name;
      const int32_t M = as_i32(args[4]), D = as_i32(args[5]), F = as_i32(args[6]);
      require_nonneg(M, nm, "M");
      require_nonneg(D, nm, "D");
      require_nonneg(F, nm, "F");
      TmGemmArgs p{};
      p.a = args[0].buffer->ptr;
      p.b = args[1].buffer->ptr;
      p.bias = args[2].buffer->ptr;
      p.c = args[3].buffer->ptr;
      p.m = M;
      p.n = F;
      p.k = D;
      p.sam = D;
      p.sak = 1;
      p.sbk = F;
      p.sbn = 1;
      p.scm = F;
      p.scn = 1;
      require_extent(args[0], (int64_t)M * D, es, nm, 0, "x");
      require_extent(args[1], (int64_t)D * F, es, nm, 1, "w");
      require_extent(args[2], F, es, nm, 2, "b");
      require_extent(args[3], (int64_t)M * F, es, nm, 3, "out");
      if (M == 0 || F == 0) {
        plan.empty = true;
        return plan;
      }
      choose_gemm(plan, p, spec, "sae");
      set_kernarg(plan, p);
      break;
    }
    case Builtin::AttnFwd: {
      TmAttnFwdArgs p{};
      p.q = args[0].buffer->ptr;
      p.k = args[1].buffer->ptr;
      p.v = args[2].buffer->ptr;
      p.o = args[3].buffer->ptr;
      p.sm_scale = as_f32(args[4]);
      p.stride_head = as_i32(args[5]);
      p.stride_seq = as_i32(args[6]);
      p.n_ctx = as_i32(args[7]);
      p.head_dim = spec.head_dim;
      p.heads = (int32_t)heads;
      const char *nm = info.name;
      validate_attn_common(nm, heads, p.stride_head, p.stride_seq, p.n_ctx, spec.head_dim);
      const int64_t ext = heads > 0 && p.n_ctx > 0
                              ? sat_add((heads - 1) * (int64_t)p.stride_head,
                                    extent(p.n_ctx, p.stride_seq, spec.head_dim, 1))
                              : 0;
      for (int i = 0; i < 4; ++i) require_extent(args[i], ext, es, nm, i, "Q/K/V/O");
      if (args.size() == 10) {
        p.lse = (float *)args[8].buffer->ptr;
        p.stride_lse = as_i32(args[9]);
        require_nonneg(p.stride_lse, nm, "stride_lse");
        require_extent(args[8], heads > 0 && p.n_ctx > 0
                                    ? (heads - 1) * (int64_t)p.stride_lse + p.n_ctx
                                    : 0,
                       4, nm, 8, "L");
      }
      if (p.n_ctx == 0) {
        plan.empty = true;
        return plan;
      }
      if (attn_fast_ok(spec, p.stride_head, p.stride_seq, p.n_ctx, p.sm_scale)) {
        plan.variant = format("tm_attn_fwd_fast_%s_d%d%s", el, spec.head_dim,
                              spec.causal ? "_causal" : "");
        plan.grid[0] = (unsigned)(cdiv(p.n_ctx, TM_FWD_FAST_ROWS) * heads);
        plan.block = TM_FWD_FAST_THREADS;
      } else {
        plan.variant = attn_symbol("fwd", spec);
        plan.grid[0] = (unsigned)cdiv(p.n_ctx, 64);
        plan.grid[1] = (unsigned)heads;
        plan.block = 256;
        /* Too few 64-query workgroups to fill the chip twice, each walking
         * many key blocks: split every workgroup's key blocks into `splits`
         * ranges (at least two 32-key blocks each) and combine the ranges'
         * partials in a second dispatch. */
        const int64_t splits = split_ranges((int64_t)plan.grid[0] * heads, p.n_ctx);
        if (splits > 1) {
          const size_t need =
              (size_t)splits * (size_t)heads * (size_t)p.n_ctx * (size_t)(spec.head_dim + 2) * 4;
          if (void *work = plan_workspace(lib, need, scratch)) {
            p.part = (float *)work;
            p.splits = (int32_t)splits;
            Plan main = plan, combine;
            main.grid[2] = (unsigned)splits;
            set_kernarg(main, p);
            combine.variant = format("tm_attn_fwd_combine_%s", el);
            combine.grid[0] = (unsigned)cdiv(heads * p.n_ctx, 4);
            combine.block = 256;
            set_kernarg(combine, p);
            for (Plan *part : {&main, &combine}) part->function = builtin_function(part->variant);
            plan.function = main.function;
            plan.variant = format("%s + %s (%d key ranges)", main.variant.c_str(),
                                  combine.variant.c_str(), (int)splits);
            plan.sequence = {main, combine};
            return plan;
          }
        }
      }
      set_kernarg(plan, p);
      break;
    }
    case Builtin::AttnPre: {
      TmAttnPreArgs p{};
      p.o = args[0].buffer->ptr;
      p.dout = args[1].buffer->ptr;
      p.delta = (float *)args[2].buffer->ptr;
      p.stride_head = as_i32(args[3]);
      p.stride_seq = as_i32(args[4]);
      p.stride_lse = as_i32(args[5]);
      p.n_ctx = as_i32(args[6]);
      p.head_dim = spec.head_dim;
      p.heads = (int32_t)heads;
      const char *nm = info.name;
      validate_attn_common(nm, heads, p.stride_head, p.stride_seq, p.n_ctx, spec.head_dim);
      require_nonneg(p.stride_lse, nm, "stride_lse");
      const int64_t ext = heads > 0 && p.n_ctx > 0
                              ? sat_add((heads - 1) * (int64_t)p.stride_head,
                                    extent(p.n_ctx, p.stride_seq, spec.head_dim, 1))
                              : 0;
      require_extent(args[0], ext, es, nm, 0, "O");
      require_extent(args[1], ext, es, nm, 1, "dO");
      require_extent(args[2],
                     heads > 0 && p.n_ctx > 0 ? (heads - 1) * (int64_t)p.stride_lse + p.n_ctx : 0,
                     4, nm, 2, "Delta");
      if (p.n_ctx == 0) {
        plan.empty = true;
        return plan;
      }
      if (attn_fast_ok(spec, p.stride_head, p.stride_seq, p.n_ctx, 1.f)) {
        plan.variant = format("tm_attn_pre_fast_%s_d%d", el, spec.head_dim);
        plan.grid[0] = (unsigned)(cdiv(p.n_ctx, 256) * heads);
      } else {
        plan.variant = format("tm_attn_pre_generic_%s", el);
        plan.grid[0] = (unsigned)cdiv(p.n_ctx, 64);
        plan.grid[1] = (unsigned)heads;
      }
      plan.block = 256;
      set_kernarg(plan, p);
      break;
    }
    case Builtin::AttnDq:
    case Builtin::AttnDkdv: {
      const bool dq = info.id == Builtin::AttnDq;
      const int first_stat = dq ? 5 : 6;
      const float sm_scale = as_f32(args[first_stat + 2]);
      const int32_t stride_head = as_i32(args[first_stat + 3]);
      const int32_t stride_seq = as_i32(args[first_stat + 4]);
      const int32_t stride_lse = as_i32(args[first_stat + 5]);
      const int32_t n_ctx = as_i32(args[first_stat + 6]);
      const char *nm = info.name;
      validate_attn_common(nm, heads, stride_head, stride_seq, n_ctx, spec.head_dim);
      require_nonneg(stride_lse, nm, "stride_lse");
      const int64_t ext = heads > 0 && n_ctx > 0
                              ? sat_add((heads - 1) * (int64_t)stride_head,
                                    extent(n_ctx, stride_seq, spec.head_dim, 1))
                              : 0;
      for (int i = 0; i < first_stat; ++i) require_extent(args[i], ext, es, nm, i, "tensor");
      const int64_t sext =
          heads > 0 && n_ctx > 0 ? (heads - 1) * (int64_t)stride_lse + n_ctx : 0;
      require_extent(args[first_stat], sext, 4, nm, first_stat, "L");
      require_extent(args[first_stat + 1], sext, 4, nm, first_stat + 1, "Delta");
      if (n_ctx == 0) {
        plan.empty = true;
        return plan;
      }
      const bool fast = attn_fast_ok(spec, stride_head, stride_seq, n_ctx, sm_scale);
      if (fast) {
        plan.grid[0] = (unsigned)(cdiv(n_ctx, 128) * heads);
      } else {
        plan.grid[0] = (unsigned)cdiv(n_ctx, 64);
        plan.grid[1] = (unsigned)heads;
      }
      const std::string fast_name = format("tm_attn_%s_fast_%s_d%d%s", dq ? "dq" : "dkdv", el,
                                           spec.head_dim, spec.causal ? "_causal" : "");
      plan.block = 256;
      if (dq) {
        TmAttnDqArgs p{};
        p.q = args[0].buffer->ptr;
        p.k = args[1].buffer->ptr;
        p.v = args[2].buffer->ptr;
        p.dout = args[3].buffer->ptr;
        p.dq = args[4].buffer->ptr;
        p.lse = (const float *)args[5].buffer->ptr;
        p.delta = (const float *)args[6].buffer->ptr;
        p.sm_scale = sm_scale;
        p.stride_head = stride_head;
        p.stride_seq = stride_seq;
        p.stride_lse = stride_lse;
        p.n_ctx = n_ctx;
        p.head_dim = spec.head_dim;
        p.heads = (int32_t)heads;
        plan.variant = fast ? fast_name : attn_symbol("dq", spec);
        const int64_t splits = fast ? 1 : split_ranges((int64_t)plan.grid[0] * heads, n_ctx);
        void *work = splits > 1 ? plan_workspace(lib, (size_t)splits * (size_t)heads * (size_t)n_ctx *
                                                          (size_t)spec.head_dim * 4,
                                                 scratch)
                                : nullptr;
        if (work) {
          plan_split_backward(plan, spec, p, (float *)work, splits, p.dq, nullptr);
          return plan;
        }
        set_kernarg(plan, p);
      } else {
        TmAttnDkdvArgs p{};
        p.q = args[0].buffer->ptr;
        p.k = args[1].buffer->ptr;
        p.v = args[2].buffer->ptr;
        p.dout = args[3].buffer->ptr;
        p.dk = args[4].buffer->ptr;
        p.dv = args[5].buffer->ptr;
        p.lse = (const float *)args[6].buffer->ptr;
        p.delta = (const float *)args[7].buffer->ptr;
        p.sm_scale = sm_scale;
        p.stride_head = stride_head;
        p.stride_seq = stride_seq;
        p.stride_lse = stride_lse;
        p.n_ctx = n_ctx;
        p.head_dim = spec.head_dim;
        p.heads = (int32_t)heads;
        plan.variant = fast ? fast_name : attn_symbol("dkdv", spec);
        const int64_t splits = fast ? 1 : split_ranges((int64_t)plan.grid[0] * heads, n_ctx);
        void *work = splits > 1 ? plan_workspace(lib, (size_t)splits * 2 * (size_t)heads *
                                                          (size_t)n_ctx * (size_t)spec.head_dim * 4,
                                                 scratch)
                                : nullptr;
        if (work) {
          plan_split_backward(plan, spec, p, (float *)work, splits, p.dk, p.dv);
          return plan;
        }
        set_kernarg(plan, p);
      }
      break;
    }
    case Builtin::AttnFused: {
      const char *nm = info.name;
      const float sm_scale = as_f32(args[9]);
      TmAttnDkdvArgs kv{};
      kv.stride_head = as_i32(args[10]);
      kv.stride_seq = as_i32(args[11]);
      kv.stride_lse = as_i32(args[12]);
      kv.n_ctx = as_i32(args[13]);
      validate_attn_common(nm, heads, kv.stride_head, kv.stride_seq, kv.n_ctx, spec.head_dim);
      require_nonneg(kv.stride_lse, nm, "stride_lse");
      const int64_t ext = heads > 0 && kv.n_ctx > 0
                              ? sat_add((heads - 1) * (int64_t)kv.stride_head,
                                    extent(kv.n_ctx, kv.stride_seq, spec.head_dim, 1))
                              : 0;
      for (int i = 0; i < 7; ++i) require_extent(args[i], ext, es, nm, i, "tensor");
      const int64_t sext =
          heads > 0 && kv.n_ctx > 0 ? (heads - 1) * (int64_t)kv.stride_lse + kv.n_ctx : 0;
      require_extent(args[7], sext, 4, nm, 7, "L");
      require_extent(args[8], sext, 4, nm, 8, "Delta");
      if (kv.n_ctx == 0 || heads == 0) {
        plan.empty = true;
        return plan;
      }
      if (!attn_fast_ok(spec, kv.stride_head, kv.stride_seq, kv.n_ctx, sm_scale))
        throw TmError(format("%s runs only on the specialised path: 16-bit elements, head_dim 64 "
                             "or 128, strides multiples of 8, a positive finite sm_scale and "
                             "heads under 2 GiB",
                             nm));
      kv.q = args[0].buffer->ptr;
      kv.k = args[1].buffer->ptr;
      kv.v = args[2].buffer->ptr;
      kv.dout = args[3].buffer->ptr;
      kv.dk = args[5].buffer->ptr;
      kv.dv = args[6].buffer->ptr;
      kv.lse = (const float *)args[7].buffer->ptr;
      kv.delta = (const float *)args[8].buffer->ptr;
      kv.sm_scale = sm_scale;
      kv.head_dim = spec.head_dim;
      kv.heads = (int32_t)heads;
      /* the fp32 dQ accumulator */
      const int64_t count = heads * kv.n_ctx * (int64_t)spec.head_dim;
      const size_t need = (size_t)count * sizeof(float);
      void *work = plan_workspace(lib, need, scratch);
      if (!work)
        throw TmError(format("%s through tm_launch_noalloc needs a %zu-byte dQ accumulator "
                             "(heads * n_ctx * head_dim * 4) but the static scratch holds %zu "
                             "bytes; launch it with tm_launch",
                             nm, need, scratch->bytes));
      plan_fused_backward(plan, spec, kv, args[4].buffer->ptr, (float *)work, count);
      return plan;
    }
    case Builtin::Probe: {
      require_extent(args[0], 256, 4, info.name, 0, "out");
      void *out = args[0].buffer->ptr;
      plan.variant = "tm_probe";
      plan.block = 64;
      set_kernarg(plan, out);
      break;
    }
    default:
      throw TmError("unknown built-in kernel");
  }
  (void)gx;
  plan.function = builtin_function(plan.variant);
  /* the workgroup size the planner chose must be one the code object was
   * compiled for (its launch bounds): a larger one would run the kernel
   * outside the assumptions its register and LDS allocation rest on */
  int limit = 0;
  hip_check(hipFuncGetAttribute(&limit, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, plan.function),
            "hipFuncGetAttribute");
  if ((int)plan.block > limit)
    throw TmError(format("internal error: '%s' planned with %u threads per workgroup, but the "
                         "kernel is built for at most %d",
                         plan.variant.c_str(), plan.block, limit));
  return plan;
}

/* User kernels: pack the arguments with natural alignment (pointers and i64 on
 * 8 bytes, i32 and f32 on 4) — the AMDGPU kernarg layout of a kernel whose
 * parameters are declared in the same order. */
/* A user launch must bind the parameter layout the kernel declares: each
 * declared parameter is covered exactly by one bound argument, or (a by-value
 * struct bound field by field, in order) by a run of them, with no argument
 * straddling a parameter boundary.  The kernel reads its implicit values (grid
 * size, workgroup size) from fixed offsets after its parameters, so any other
 * layout would make it read garbage on the GPU. */
void check_signature_layout(const Kernel &k, const std::vector<std::pair<long, long>> &packed) {
  const auto &want = k.signature;
  long want_bytes = 0, have_bytes = 0;
  for (const auto &a : want) want_bytes = std::max(want_bytes, a.offset + a.size);
  for (const auto &a : packed) have_bytes = std::max(have_bytes, a.first + a.second);
  size_t j = 0;
  long bad = -1; /* first declared parameter the launch does not cover */
  for (size_t i = 0; i < want.size() && bad < 0; ++i) {
    const long at = want[i].offset, end = at + want[i].size;
    if (j >= packed.size() || packed[j].first != at) {
      bad = (long)i;
      break;
    }
    const size_t first = j;
    while (j < packed.size() && packed[j].first + packed[j].second <= end) ++j;
    if (j == first) {
      bad = (long)i;
      break;
    }
    const long covered = packed[j - 1].first + packed[j - 1].second;
    /* a by-value struct bound field by field may stop short of its size by its
     * tail padding (less than its 8-byte alignment); the packed block is
     * padded to 8 bytes, so the kernel's implicit values stay in place */
    const bool tail_padding = want[i].kind == "by_value" && want[i].size > 8 && end % 8 == 0 &&
                              end - covered < 8;
    if (covered != end && !tail_padding) bad = (long)i;
  }
  if (bad < 0 && j == packed.size()) return;
  if (want.size() != packed.size() || bad < 0)
    throw TmError(format("kernel '%s' declares %zu argument%s (%ld bytes) but the launch binds "
                         "%zu (%ld bytes)",
                         k.name.c_str(), want.size(), want.size() == 1 ? "" : "s", want_bytes,
                         packed.size(), have_bytes));
  const size_t i = (size_t)bad;
  throw TmError(format("kernel '%s' argument %zu is %ld bytes at offset %ld (%s) but the launch "
                       "binds %ld bytes at offset %ld",
                       k.name.c_str(), i, want[i].size, want[i].offset, want[i].kind.c_str(),
                       packed[i].second, packed[i].first));
}

Plan plan_user(Kernel &k, const std::vector<Arg> &args, int64_t gx, int64_t gy, int64_t gz,
               int64_t threads) {
  Plan plan;
  plan.function = k.function;
  plan.variant = k.name;
  plan.by_value_struct = false;
  plan.grid[0] = (unsigned)gx;
  plan.grid[1] = (unsigned)gy;
  plan.grid[2] = (unsigned)gz;
  plan.block = (unsigned)threads;
  auto &buf = plan.kernarg;
  std::vector<std::pair<long, long>> packed; /* (offset, size) of each bound argument */
  auto put = [&buf, &packed](const void *src, size_t size) {
    while (buf.size() % size) buf.push_back(0);
    const size_t at = buf.size();
    buf.resize(at + size);
    memcpy(buf.data() + at, src, size);
    packed.emplace_back((long)at, (long)size);
  };
  for (const Arg &a : args) {
    switch (a.kind) {
      case TM_ARG_BUFFER: {
        void *p = a.buffer->ptr;
        put(&p, 8);
        break;
      }
      case TM_ARG_I32: {
        int32_t v = as_i32(a);
        put(&v, 4);
        break;
      }
      case TM_ARG_F32: {
        float f = as_f32(a);
        put(&f, 4);
        break;
      }
      case TM_ARG_I64: {
        int64_t v = a.value;
        put(&v, 8);
        break;
      }
    }
  }
  while (buf.size() % 8) buf.push_back(0);
  if (k.has_signature) check_signature_layout(k, packed);
  return plan;
}

int64_t max_threads(Kernel &k) {
  if (k.builtin != Builtin::None) return k.builtin == Builtin::Probe ? 64 : 1024;
  int value = 0;
  hip_check(hipFuncGetAttribute(&value, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, k.function),
            "hipFuncGetAttribute");
  return value;
}

void enqueue(const Plan &plan, hipStream_t stream) {
  if (plan.empty) return;
  if (!plan.sequence.empty()) {
    for (const Plan &part : plan.sequence) enqueue(part, stream);
    return;
  }
  if (!plan.function || plan.block == 0 || plan.block > 1024 || !plan.grid[0] || !plan.grid[1] ||
      !plan.grid[2])
    throw TmError("internal error: dispatch of '" + plan.variant +
                  "' was not fully planned (no function, workgroup size or grid)");
  if (plan.by_value_struct) {
    void *params[] = {(void *)plan.kernarg.data()};
    hip_check(hipModuleLaunchKernel(plan.function, plan.grid[0], plan.grid[1], plan.grid[2],
                                    plan.block, 1, 1, 0, stream, params, nullptr),
              "hipModuleLaunchKernel");
  } else {
    size_t size = plan.kernarg.size();
    void *data = size ? (void *)plan.kernarg.data() : nullptr;
    void *extra[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, data, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                     HIP_LAUNCH_PARAM_END};
    hip_check(hipModuleLaunchKernel(plan.function, plan.grid[0], plan.grid[1], plan.grid[2],
                                    plan.block, 1, 1, 0, stream, nullptr, size ? extra : nullptr),
              "hipModuleLaunchKernel");
  }
}

/* Validation shared by every launch form (reference Runtime.swift:201-211),
 * then the plan.  No HIP call happens before the request is known to be good
 * except the device lookup the built-in planner needs. */
Plan prepare(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
             const int32_t *kinds, const int64_t *values, int32_t argc,
             std::shared_ptr<Kernel> &k_out, std::unique_lock<std::mutex> &launch_guard,
             std::vector<std::shared_ptr<Buffer>> *mirrored = nullptr,
             const Scratch *scratch = nullptr) {
  auto k = handles().lookup<Kernel>(kernel, Kind::Kernel, "kernel");
  k_out = k;
  /* from here until the caller has queued the plan, no other launch on this
   * library plans or queues */
  launch_guard = std::unique_lock<std::mutex>(k->library->launch_lock);
  std::vector<Arg> args = decode_args(kinds, values, argc);
  if (mirrored)
    for (const Arg &a : args)
      if (a.buffer) {
        std::lock_guard<std::mutex> guard(a.buffer->host_lock);
        if (a.buffer->host &&
            std::find(mirrored->begin(), mirrored->end(), a.buffer) == mirrored->end())
          mirrored->push_back(a.buffer);
      }
  if (gx <= 0 || gy <= 0 || gz <= 0)
    throw TmError("threadgroup grid must be positive in every dimension");
  if (gx > 0x7fffffff || gy > 0xffff || gz > 0xffff)
    throw TmError("threadgroup grid exceeds the device's grid limits");
  if (threads <= 0) throw TmError("threadsPerThreadgroup must be positive");
  const int64_t limit = k->builtin != Builtin::None ? max_threads(*k) : -1;
  if (limit > 0 && threads > limit)
    throw TmError(format("threadsPerThreadgroup %lld exceeds the pipeline maximum %lld",
                         (long long)threads, (long long)limit));
  Plan plan;
  if (k->builtin != Builtin::None) {
    plan = plan_builtin(*k, *k->library, args, gx, gy, gz, scratch);
  } else {
    require_device();
    const int64_t user_limit = max_threads(*k);
    if (threads > user_limit)
      throw TmError(format("threadsPerThreadgroup %lld exceeds the pipeline maximum %lld",
                           (long long)threads, (long long)user_limit));
    plan = plan_user(*k, args, gx, gy, gz, threads);
  }
  {
    std::lock_guard<std::mutex> guard(k->lock);
    k->last_variant = plan.empty ? std::string("(empty)") : plan.variant;
  }
  return plan;
}

void finish(hipStream_t stream) {
  hipError_t status = hipStreamSynchronize(stream);
  if (status != hipSuccess)
    throw TmError(format("kernel execution failed: %s (%s)", hipGetErrorName(status),
                         hipGetErrorString(status)));
}

/* ---- the probe (reference Runtime.swift:112-178) --------------------------- */

std::string probe_device() {
  Device &dev = device();
  if (!dev.present) return dev.absent_reason;
  if (dev.arch.rfind("gfx950", 0) != 0)
    return format("%s is %s; this library's kernels are built for gfx950", dev.name.c_str(),
                  dev.arch.c_str());
  try {
    hipFunction_t fn = builtin_function("tm_probe");
    float *out = nullptr;
    hip_check(hipMalloc(&out, 256 * sizeof(float)), "hipMalloc");
    std::unique_ptr<float, void (*)(float *)> guard(out, [](float *p) { (void)hipFree(p); });
    hip_check(hipMemsetAsync(out, 0, 256 * sizeof(float), dev.stream), "hipMemsetAsync");
    void *params[] = {&out};
    hip_check(hipModuleLaunchKernel(fn, 1, 1, 1, 64, 1, 1, 0, dev.stream, params, nullptr),
              "hipModuleLaunchKernel");
    finish(dev.stream);
    float host[256];
    hip_check(hipMemcpy(host, out, sizeof host, hipMemcpyDeviceToHost), "hipMemcpy");
    for (int i = 0; i < 256; ++i)
      if (host[i] != (float)i)
        return format("%s ran the probe kernel but returned %g at %d instead of %d — its MFMA "
                      "support is not usable",
                      dev.name.c_str(), host[i], i, i);
    return "";
  } catch (const std::exception &e) {
    return format("%s cannot run a built-in kernel: %s", dev.name.c_str(), e.what());
  }
}

const std::string &unusable_reason() {
  static std::string reason;
  static std::once_flag once;
  std::call_once(once, [] { reason = probe_device(); });
  return reason;
}

/* ---- hiprtc ------------------------------------------------------------------ */

std::vector<char> compile_hip_source(const char *source) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, source, "tm_user.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    throw TmError("HIP compilation failed: hiprtcCreateProgram");
  const char *options[] = {"--offload-arch=gfx950", "-O3"};
  hiprtcResult status = hiprtcCompileProgram(prog, 2, options);
  if (status != HIPRTC_SUCCESS) {
    size_t log_size = 0;
    hiprtcGetProgramLogSize(prog, &log_size);
    std::string log(log_size, '\0');
    if (log_size) hiprtcGetProgramLog(prog, &log[0]);
    hiprtcDestroyProgram(&prog);
    throw TmError("HIP compilation failed: " + log);
  }
  size_t code_size = 0;
  hiprtcGetCodeSize(prog, &code_size);
  std::vector<char> code(code_size);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  return code;
}

int64_t launch_common(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                      const int32_t *kinds, const int64_t *values, int32_t argc, bool wait,
                      int32_t repeats, float *elapsed_ms, const Scratch *scratch = nullptr) {
  std::shared_ptr<Kernel> k;
  std::vector<std::shared_ptr<Buffer>> mirrored;
  std::unique_lock<std::mutex> launch_guard;
  Plan plan = prepare(kernel, gx, gy, gz, threads, kinds, values, argc, k, launch_guard, &mirrored,
                      scratch);
  Device &dev = require_device();
  /* buffers with a host mirror: mirror -> HBM before, HBM -> mirror after */
  for (const auto &b : mirrored) {
    std::lock_guard<std::mutex> guard(b->host_lock);
    hip_check(hipMemcpyAsync(b->ptr, b->host, (size_t)b->length, hipMemcpyHostToDevice, dev.stream),
              "hipMemcpyAsync (host mirror to HBM)");
  }
  auto refresh_mirrors = [&]() {
    if (mirrored.empty()) return;
    finish(dev.stream);
    for (const auto &b : mirrored) {
      std::lock_guard<std::mutex> guard(b->host_lock);
      hip_check(hipMemcpy(b->host, b->ptr, (size_t)b->length, hipMemcpyDeviceToHost),
                "hipMemcpy (HBM to host mirror)");
    }
  };
  if (repeats <= 0) {
    enqueue(plan, dev.stream);
    launch_guard.unlock();
    if (wait) finish(dev.stream);
    refresh_mirrors();
    return 0;
  }
  hipEvent_t start, stop;
  hip_check(hipEventCreate(&start), "hipEventCreate");
  hip_check(hipEventCreate(&stop), "hipEventCreate");
  std::unique_ptr<void, std::function<void(void *)>> guard((void *)1, [&](void *) {
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
  });
  hip_check(hipEventRecord(start, dev.stream), "hipEventRecord");
  for (int i = 0; i < repeats; ++i) enqueue(plan, dev.stream);
  hip_check(hipEventRecord(stop, dev.stream), "hipEventRecord");
  launch_guard.unlock();
  finish(dev.stream);
  float ms = 0.f;
  hip_check(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
  if (elapsed_ms) *elapsed_ms = ms;
  refresh_mirrors();
  return 0;
}

std::string kernel_info_json(const BuiltinSpec &spec) {
  std::ostringstream out;
  out << "{\n  \"kernels\" : [\n";
  bool first = true;
  for (const BuiltinInfo &info : builtin_table()) {
    if (info.id == Builtin::AttnFused && spec.bwd == BuiltinSpec::Bwd::Split) continue;
    const Published pub = published_shape(info.id);
    if (!first) out << ",\n";
    first = false;
    out << "    {\n      \"args\" : [";
    for (size_t i = 0; i < info.kinds.size(); ++i) {
      const char *dt = strcmp(info.dtypes[i], "E") == 0 ? element_name(spec.element)
                                                         : info.dtypes[i];
      out << (i ? ", " : "") << "{\"dtype\" : \"" << dt << "\", \"index\" : " << i
          << ", \"kind\" : " << info.kinds[i] << "}";
    }
    out << "],\n      \"block_shape\" : [";
    for (size_t i = 0; i < pub.block_shape.size(); ++i)
      out << (i ? ", " : "") << pub.block_shape[i];
    out << "],\n      \"block_size\" : " << pub.block_shape[0] << ",\n      \"causal\" : "
        << (spec.causal ? "true" : "false") << ",\n      \"head_dim\" : " << spec.head_dim
        << ",\n      \"name\" : \"" << info.name << "\",\n      \"threads_per_threadgroup\" : "
        << pub.threads << "\n    }";
  }
  out << "\n  ]\n}";
  return out.str();
}

}  // namespace

/* =============================================================================
 * The C ABI.
 * ===========================================================================*/

#define TM_GUARD_BEGIN try {
#define TM_GUARD_END(sentinel)              \
  }                                         \
  catch (const std::exception &e) {         \
    store_error(e.what());                  \
    return sentinel;                        \
  }

extern "C" {

char *tm_version(void) { return dup_string("0.0.1"); }

void tm_free(void *ptr) { free(ptr); }

char *tm_last_error(void) {
  std::lock_guard<std::mutex> guard(g_error_lock);
  std::string message = g_has_error ? g_error : std::string("no error");
  g_has_error = false;
  g_error.clear();
  return dup_string(message);
}

int32_t tm_is_active(void) { return device().present ? 1 : 0; }

int32_t tm_is_usable(void) { return unusable_reason().empty() ? 1 : 0; }

char *tm_unusable_reason(void) {
  const std::string &reason = unusable_reason();
  return reason.empty() ? nullptr : dup_string(reason);
}

char *tm_device_name(void) {
  Device &dev = device();
  if (!dev.present) return nullptr;
  return dup_string(dev.name.empty() ? "AMD GPU (" + dev.arch + ")"
                                     : dev.name + " (" + dev.arch + ")");
}

char *tm_emit_msl(const char *module, int32_t num_simdgroups) {
  (void)num_simdgroups;
  TM_GUARD_BEGIN
  if (!module) throw TmError("tm_emit_msl received a NULL module");
  if (!is_builtin_spec(module))
    throw TmError("tm_emit_msl: ttir lowering is not part of this library; pass a built-in "
                  "library spec (\"builtin element=... head_dim=... causal=...\")");
  return dup_string(parse_spec(module).text());
  TM_GUARD_END(nullptr)
}

char *tm_kernel_info(const char *module, int32_t num_simdgroups) {
  (void)num_simdgroups;
  TM_GUARD_BEGIN
  if (!module) throw TmError("tm_kernel_info received a NULL module");
  if (!is_builtin_spec(module))
    throw TmError("tm_kernel_info: ttir lowering is not part of this library; pass a built-in "
                  "library spec (\"builtin element=... head_dim=... causal=...\")");
  return dup_string(kernel_info_json(parse_spec(module)));
  TM_GUARD_END(nullptr)
}

int64_t tm_compile_msl(const char *source) {
  TM_GUARD_BEGIN
  if (!source) throw TmError("tm_compile_msl received NULL source");
  auto lib = std::make_shared<Library>();
  if (is_builtin_spec(source)) {
    lib->builtin = true;
    lib->spec = parse_spec(source);
  } else {
    std::vector<char> code = compile_hip_source(source);
    require_device();
    hip_check(hipModuleLoadData(&lib->module, code.data()), "could not load compiled HIP code");
    lib->signatures = tm_codeobject::read_kernel_arguments(code.data(), code.size());
  }
  return handles().insert(lib);
  TM_GUARD_END(0)
}

int64_t tm_load_metallib(const void *image, int64_t length) {
  TM_GUARD_BEGIN
  if (!image || length <= 0) throw TmError("tm_load_metallib received an empty image");
  require_device();
  std::vector<char> copy((const char *)image, (const char *)image + length);
  auto lib = std::make_shared<Library>();
  hipError_t status = hipModuleLoadData(&lib->module, copy.data());
  if (status != hipSuccess) {
    lib->module = nullptr;
    (void)hipGetLastError();
    throw TmError(format("could not load metallib: the image is not a loadable gfx950 code "
                         "object (%s)",
                         hipGetErrorName(status)));
  }
  lib->signatures = tm_codeobject::read_kernel_arguments(copy.data(), copy.size());
  return handles().insert(lib);
  TM_GUARD_END(0)
}

int32_t tm_release_library(int64_t library) {
  TM_GUARD_BEGIN
  if (!handles().remove(library, Kind::Library))
    throw TmError(format("library handle %lld is not live", (long long)library));
  return 0;
  TM_GUARD_END(-1)
}

int64_t tm_load_kernel(int64_t library, const char *name) {
  TM_GUARD_BEGIN
  if (!name) throw TmError("tm_load_kernel received a NULL kernel name");
  auto lib = handles().lookup<Library>(library, Kind::Library, "library");
  auto k = std::make_shared<Kernel>();
  k->library = lib;
  k->name = name;
  if (lib->builtin) {
    const BuiltinInfo *info = find_builtin(name);
    if (!info)
      throw TmError(format("kernel '%s' not found in library (available: %s)", name,
                           builtin_names().c_str()));
    if (info->id == Builtin::AttnFused && lib->spec.bwd == BuiltinSpec::Bwd::Split)
      throw TmError("kernel 'attn_bwd_fused' is offered only by built-in libraries whose spec "
                    "has bwd=atomic (dQ summed with floating-point atomics, not deterministic)");
    k->builtin = info->id;
    /* load the kernel images now, so that launches (tm_launch_noalloc among
     * them) load no code; a failure here resurfaces at the first launch */
    if (device().present) {
      BuiltinModules &mods = builtin_modules();
      std::lock_guard<std::mutex> guard(mods.lock);
      try {
        load_builtin_modules(mods);
      } catch (const TmError &) {
        (void)hipGetLastError();
      }
    }
  } else {
    hipError_t status = hipModuleGetFunction(&k->function, lib->module, name);
    if (status != hipSuccess) {
      (void)hipGetLastError();
      throw TmError(format("kernel '%s' not found in library (%s)", name,
                           hipGetErrorName(status)));
    }
    const auto sig = lib->signatures.find(name);
    if (sig != lib->signatures.end()) {
      k->has_signature = true;
      k->signature = sig->second;
    }
  }
  return handles().insert(k);
  TM_GUARD_END(0)
}

int64_t tm_kernel_max_threads(int64_t kernel) {
  TM_GUARD_BEGIN
  auto k = handles().lookup<Kernel>(kernel, Kind::Kernel, "kernel");
  return max_threads(*k);
  TM_GUARD_END(-1)
}

int32_t tm_release_kernel(int64_t kernel) {
  TM_GUARD_BEGIN
  if (!handles().remove(kernel, Kind::Kernel))
    throw TmError(format("kernel handle %lld is not live", (long long)kernel));
  return 0;
  TM_GUARD_END(-1)
}

int64_t tm_alloc_buffer(int64_t length) {
  TM_GUARD_BEGIN
  if (length <= 0)
    throw TmError(format("buffer length must be positive, got %lld", (long long)length));
  require_device();
  auto buf = std::make_shared<Buffer>();
  /* Padded to 256 bytes: the GEMM's 16-byte tile copies may read up to 14
   * bytes past the end of a matrix whose rows are not a multiple of 8
   * elements (those bytes feed only outputs that are not stored). */
  if (length > INT64_MAX - 255)
    throw TmError(format("could not allocate a %lld-byte device buffer (too large)", (long long)length));
  hipError_t status = hipMalloc(&buf->ptr, (size_t)((length + 255) & ~(int64_t)255));
  if (status != hipSuccess) {
    buf->ptr = nullptr;
    (void)hipGetLastError();
    throw TmError(format("could not allocate a %lld-byte device buffer (%s)", (long long)length,
                         hipGetErrorName(status)));
  }
  buf->length = length;
  return handles().insert(buf);
  TM_GUARD_END(0)
}

void *tm_buffer_contents(int64_t buffer) {
  TM_GUARD_BEGIN
  auto buf = handles().lookup<Buffer>(buffer, Kind::Buffer, "buffer");
  std::lock_guard<std::mutex> guard(buf->host_lock);
  if (!buf->host) {
    Device &dev = require_device();
    finish(dev.stream);
    void *host = nullptr;
    hipError_t status = hipHostMalloc(&host, (size_t)buf->length, hipHostMallocDefault);
    if (status != hipSuccess) {
      (void)hipGetLastError();
      throw TmError(format("could not allocate the %lld-byte host mirror of buffer %lld (%s)",
                           (long long)buf->length, (long long)buffer, hipGetErrorName(status)));
    }
    status = hipMemcpy(host, buf->ptr, (size_t)buf->length, hipMemcpyDeviceToHost);
    if (status != hipSuccess) {
      (void)hipHostFree(host);
      hip_check(status, "hipMemcpy (HBM to host mirror)");
    }
    buf->host = host;
  }
  return buf->host;
  TM_GUARD_END(nullptr)
}

int32_t tm_buffer_unmap(int64_t buffer) {
  TM_GUARD_BEGIN
  auto buf = handles().lookup<Buffer>(buffer, Kind::Buffer, "buffer");
  /* launches that bound the buffer have refreshed the mirror when they
   * returned; host writes since then are copied down before it goes */
  finish(require_device().stream);
  std::lock_guard<std::mutex> guard(buf->host_lock);
  if (buf->host) {
    hip_check(hipMemcpy(buf->ptr, buf->host, (size_t)buf->length, hipMemcpyHostToDevice),
              "hipMemcpy (host mirror to HBM)");
    hip_check(hipHostFree(buf->host), "hipHostFree");
    buf->host = nullptr;
  }
  return 0;
  TM_GUARD_END(-1)
}

int64_t tm_buffer_length(int64_t buffer) {
  TM_GUARD_BEGIN
  return handles().lookup<Buffer>(buffer, Kind::Buffer, "buffer")->length;
  TM_GUARD_END(-1)
}

static int32_t tm_copy(int64_t buffer, int64_t offset, const void *host, int64_t length,
                       bool to_device) {
  TM_GUARD_BEGIN
  if (!host || length < 0 || offset < 0)
    throw TmError("buffer copy received invalid bounds");
  auto buf = handles().lookup<Buffer>(buffer, Kind::Buffer, "buffer");
  /* written so that no sum can wrap */
  if (length > buf->length || offset > buf->length - length)
    throw TmError(format("copy of %lld bytes at offset %lld exceeds the %lld-byte buffer",
                         (long long)length, (long long)offset, (long long)buf->length));
  if (length == 0) return 0;
  Device &dev = require_device();
  /* Work queued on the library stream is ordered before the copy. */
  finish(dev.stream);
  char *dptr = (char *)buf->ptr + offset;
  std::lock_guard<std::mutex> guard(buf->host_lock);
  char *mirror = buf->host ? (char *)buf->host + offset : nullptr;
  if (to_device) {
    hip_check(hipMemcpy(dptr, host, (size_t)length, hipMemcpyHostToDevice), "hipMemcpy");
    if (mirror) memcpy(mirror, host, (size_t)length);
  } else if (mirror) {
    memcpy((void *)host, mirror, (size_t)length);
  } else {
    hip_check(hipMemcpy((void *)host, dptr, (size_t)length, hipMemcpyDeviceToHost), "hipMemcpy");
  }
  return 0;
  TM_GUARD_END(-1)
}

int32_t tm_buffer_write(int64_t buffer, int64_t offset, const void *source, int64_t length) {
  return tm_copy(buffer, offset, source, length, true);
}

int32_t tm_buffer_read(int64_t buffer, int64_t offset, void *destination, int64_t length) {
  return tm_copy(buffer, offset, destination, length, false);
}

int32_t tm_free_buffer(int64_t buffer) {
  TM_GUARD_BEGIN
  if (!handles().remove(buffer, Kind::Buffer))
    throw TmError(format("buffer handle %lld is not live", (long long)buffer));
  return 0;
  TM_GUARD_END(-1)
}

int32_t tm_launch(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                  const int32_t *kinds, const int64_t *values, int32_t argc) {
  TM_GUARD_BEGIN
  return (int32_t)launch_common(kernel, gx, gy, gz, threads, kinds, values, argc, true, 0,
                                nullptr);
  TM_GUARD_END(-1)
}

int32_t tm_launch_async(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                        const int32_t *kinds, const int64_t *values, int32_t argc) {
  TM_GUARD_BEGIN
  return (int32_t)launch_common(kernel, gx, gy, gz, threads, kinds, values, argc, false, 0,
                                nullptr);
  TM_GUARD_END(-1)
}

int32_t tm_synchronize(void) {
  TM_GUARD_BEGIN
  finish(require_device().stream);
  return 0;
  TM_GUARD_END(-1)
}

int32_t tm_launch_timed(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                        const int32_t *kinds, const int64_t *values, int32_t argc,
                        int32_t repeats, float *elapsed_ms) {
  TM_GUARD_BEGIN
  if (repeats <= 0) throw TmError(format("tm_launch_timed: repeats must be positive, got %d",
                                         repeats));
  if (!elapsed_ms) throw TmError("tm_launch_timed received a NULL elapsed_ms");
  return (int32_t)launch_common(kernel, gx, gy, gz, threads, kinds, values, argc, true, repeats,
                                elapsed_ms);
  TM_GUARD_END(-1)
}

/* tm_launch with no allocation: a dispatch that needs a work buffer takes it
 * from the static scratch (scratch.hip) instead of library-owned memory.
 * One lock holds from planning to the wait, so this process's calls never
 * overlap on the scratch; it keeps the last call's contents, and each
 * dispatch clears what it needs zeroed with a kernel. */
int32_t tm_launch_noalloc(int64_t kernel, int64_t gx, int64_t gy, int64_t gz, int64_t threads,
                          const int32_t *kinds, const int64_t *values, int32_t argc) {
  TM_GUARD_BEGIN
  static std::mutex noalloc_lock;
  std::lock_guard<std::mutex> guard(noalloc_lock);
  require_device();
  Scratch scratch;
  hip_check(tm_scratch_address(&scratch.ptr), "hipGetSymbolAddress (static scratch)");
  scratch.bytes = TM_SCRATCH_BYTES;
  return (int32_t)launch_common(kernel, gx, gy, gz, threads, kinds, values, argc, true, 0,
                                nullptr, &scratch);
  TM_GUARD_END(-1)
}

char *tm_kernel_variant(int64_t kernel) {
  TM_GUARD_BEGIN
  auto k = handles().lookup<Kernel>(kernel, Kind::Kernel, "kernel");
  std::lock_guard<std::mutex> guard(k->lock);
  if (k->last_variant.empty())
    throw TmError(format("kernel handle %lld has not been launched", (long long)kernel));
  return dup_string(k->last_variant);
  TM_GUARD_END(nullptr)
}

int64_t tm_live_handle_count(void) { return handles().count(); }

}  // extern "C"
