/*
 * Reader for the kernel argument layouts of an AMDGPU code object (see
 * codeobject.h).  Three layers, each bounds-checked against the image:
 *   - clang offload bundle: "__CLANG_OFFLOAD_BUNDLE__", a u64 entry count, then
 *     per entry u64 offset, u64 size, u64 triple length and the triple; the
 *     first entry whose triple names amdgcn is the device ELF;
 *   - ELF64 little-endian: the section headers locate SHT_NOTE sections; the
 *     note named "AMDGPU" of type 32 (NT_AMDGPU_METADATA) holds MessagePack;
 *   - MessagePack: a small decoder for the types the metadata uses.
 */
#include "codeobject.h"

#include <cstdint>
#include <cstring>

namespace tm_codeobject {
namespace {

/* ---- MessagePack ------------------------------------------------------------ */

struct Value {
  enum Type { Nil, Bool, Int, Float, Str, Bin, Array, Map, Ext } type = Nil;
  int64_t i = 0;
  double f = 0;
  std::string s;
  std::vector<Value> items;                       /* Array */
  std::vector<std::pair<Value, Value>> entries;   /* Map */

  const Value *get(const char *key) const {
    if (type != Map) return nullptr;
    for (const auto &e : entries)
      if (e.first.type == Str && e.first.s == key) return &e.second;
    return nullptr;
  }
};

class Reader {
 public:
  Reader(const uint8_t *p, size_t n) : p_(p), end_(p + n) {}
  bool ok() const { return ok_; }

  Value value(int depth = 0) {
    Value v;
    if (depth > 64 || !need(1)) return fail();
    const uint8_t b = *p_++;
    if (b <= 0x7f) return integer(b);
    if (b >= 0xe0) return integer((int8_t)b);
    if ((b & 0xf0) == 0x80) return map(b & 0x0f, depth);
    if ((b & 0xf0) == 0x90) return array(b & 0x0f, depth);
    if ((b & 0xe0) == 0xa0) return str(b & 0x1f, Value::Str);
    switch (b) {
      case 0xc0: return v;
      case 0xc2: v.type = Value::Bool; v.i = 0; return v;
      case 0xc3: v.type = Value::Bool; v.i = 1; return v;
      case 0xc4: return str(be(1), Value::Bin);
      case 0xc5: return str(be(2), Value::Bin);
      case 0xc6: return str(be(4), Value::Bin);
      case 0xc7: return ext(be(1));
      case 0xc8: return ext(be(2));
      case 0xc9: return ext(be(4));
      case 0xca: {
        uint32_t u = (uint32_t)be(4);
        float f;
        memcpy(&f, &u, 4);
        v.type = Value::Float;
        v.f = f;
        return v;
      }
      case 0xcb: {
        uint64_t u = be(8);
        double d;
        memcpy(&d, &u, 8);
        v.type = Value::Float;
        v.f = d;
        return v;
      }
      case 0xcc: return integer((int64_t)be(1));
      case 0xcd: return integer((int64_t)be(2));
      case 0xce: return integer((int64_t)be(4));
      case 0xcf: return integer((int64_t)be(8));
      case 0xd0: return integer((int8_t)be(1));
      case 0xd1: return integer((int16_t)be(2));
      case 0xd2: return integer((int32_t)be(4));
      case 0xd3: return integer((int64_t)be(8));
      case 0xd4: return ext(1);
      case 0xd5: return ext(2);
      case 0xd6: return ext(4);
      case 0xd7: return ext(8);
      case 0xd8: return ext(16);
      case 0xd9: return str(be(1), Value::Str);
      case 0xda: return str(be(2), Value::Str);
      case 0xdb: return str(be(4), Value::Str);
      case 0xdc: return array(be(2), depth);
      case 0xdd: return array(be(4), depth);
      case 0xde: return map(be(2), depth);
      case 0xdf: return map(be(4), depth);
      default: return fail();
    }
  }

 private:
  bool need(uint64_t n) {
    if (!ok_ || (uint64_t)(end_ - p_) < n) {
      ok_ = false;
      return false;
    }
    return true;
  }
  uint64_t be(int n) {
    if (!need(n)) return 0;
    uint64_t u = 0;
    for (int k = 0; k < n; ++k) u = (u << 8) | *p_++;
    return u;
  }
  Value fail() {
    ok_ = false;
    return Value();
  }
  Value integer(int64_t x) {
    Value v;
    v.type = Value::Int;
    v.i = x;
    return v;
  }
  Value str(uint64_t n, Value::Type t) {
    Value v;
    if (!need(n)) return fail();
    v.type = t;
    v.s.assign((const char *)p_, n);
    p_ += n;
    return v;
  }
  Value ext(uint64_t n) {
    Value v;
    if (!need(n + 1)) return fail();
    p_ += n + 1; /* type byte + data */
    v.type = Value::Ext;
    return v;
  }
  Value array(uint64_t n, int depth) {
    Value v;
    v.type = Value::Array;
    for (uint64_t k = 0; k < n && ok_; ++k) v.items.push_back(value(depth + 1));
    return ok_ ? v : fail();
  }
  Value map(uint64_t n, int depth) {
    Value v;
    v.type = Value::Map;
    for (uint64_t k = 0; k < n && ok_; ++k) {
      Value key = value(depth + 1);
      Value val = value(depth + 1);
      v.entries.emplace_back(std::move(key), std::move(val));
    }
    return ok_ ? v : fail();
  }

  const uint8_t *p_;
  const uint8_t *end_;
  bool ok_ = true;
};

/* ---- ELF -------------------------------------------------------------------- */

template <typename U>
bool load(const uint8_t *base, size_t size, uint64_t at, U *out) {
  if (at > size || size - at < sizeof(U)) return false;
  memcpy(out, base + at, sizeof(U));
  return true;
}

/* The NT_AMDGPU_METADATA descriptor of a little-endian ELF64 image. */
bool find_metadata(const uint8_t *elf, size_t size, const uint8_t **desc, size_t *desc_size) {
  if (size < 64 || memcmp(elf, "\x7f" "ELF", 4) != 0 || elf[4] != 2 || elf[5] != 1) return false;
  uint64_t shoff = 0;
  uint16_t shentsize = 0, shnum = 0;
  if (!load(elf, size, 0x28, &shoff) || !load(elf, size, 0x3a, &shentsize) ||
      !load(elf, size, 0x3c, &shnum) || shentsize < 0x40)
    return false;
  for (uint16_t k = 0; k < shnum; ++k) {
    const uint64_t sh = shoff + (uint64_t)k * shentsize;
    uint32_t type = 0;
    uint64_t off = 0, len = 0;
    if (!load(elf, size, sh + 4, &type) || !load(elf, size, sh + 0x18, &off) ||
        !load(elf, size, sh + 0x20, &len))
      return false;
    if (type != 7 /* SHT_NOTE */ || off > size || len > size - off) continue;
    uint64_t at = off;
    const uint64_t stop = off + len;
    while (at + 12 <= stop) {
      uint32_t namesz = 0, descsz = 0, ntype = 0;
      load(elf, size, at, &namesz);
      load(elf, size, at + 4, &descsz);
      load(elf, size, at + 8, &ntype);
      const uint64_t name_at = at + 12;
      const uint64_t desc_at = name_at + ((namesz + 3ull) & ~3ull);
      const uint64_t next = desc_at + ((descsz + 3ull) & ~3ull);
      if (next > stop) break;
      if (ntype == 32 && namesz >= 6 && memcmp(elf + name_at, "AMDGPU", 6) == 0) {
        *desc = elf + desc_at;
        *desc_size = descsz;
        return true;
      }
      at = next;
    }
  }
  return false;
}

/* The device ELF inside a clang offload bundle, or the image itself. */
bool device_elf(const uint8_t *image, size_t size, const uint8_t **elf, size_t *elf_size) {
  static const char kMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
  const size_t mlen = sizeof(kMagic) - 1;
  if (size >= mlen && memcmp(image, kMagic, mlen) == 0) {
    uint64_t count = 0, at = mlen;
    if (!load(image, size, at, &count)) return false;
    at += 8;
    for (uint64_t k = 0; k < count && k < 1024; ++k) {
      uint64_t off = 0, len = 0, tlen = 0;
      if (!load(image, size, at, &off) || !load(image, size, at + 8, &len) ||
          !load(image, size, at + 16, &tlen))
        return false;
      at += 24;
      if (tlen > size || at > size - tlen) return false;
      const std::string triple((const char *)image + at, tlen);
      at += tlen;
      if (triple.find("amdgcn") != std::string::npos && off <= size && len <= size - off &&
          len > 0) {
        *elf = image + off;
        *elf_size = len;
        return true;
      }
    }
    return false;
  }
  *elf = image;
  *elf_size = size;
  return true;
}

}  // namespace

std::map<std::string, std::vector<ArgSlot>> read_kernel_arguments(const void *image,
                                                                   size_t size) {
  std::map<std::string, std::vector<ArgSlot>> out;
  if (!image || size == 0) return out;
  const uint8_t *elf = nullptr, *desc = nullptr;
  size_t elf_size = 0, desc_size = 0;
  if (!device_elf((const uint8_t *)image, size, &elf, &elf_size) ||
      !find_metadata(elf, elf_size, &desc, &desc_size))
    return out;
  Reader reader(desc, desc_size);
  const Value root = reader.value();
  if (!reader.ok()) return out;
  const Value *kernels = root.get("amdhsa.kernels");
  if (!kernels || kernels->type != Value::Array) return out;
  for (const Value &k : kernels->items) {
    const Value *name = k.get(".name");
    const Value *args = k.get(".args");
    if (!name || name->type != Value::Str) continue;
    std::vector<ArgSlot> slots;
    if (args && args->type == Value::Array) {
      for (const Value &a : args->items) {
        const Value *off = a.get(".offset"), *sz = a.get(".size"), *kind = a.get(".value_kind");
        if (!off || !sz || !kind || off->type != Value::Int || sz->type != Value::Int ||
            kind->type != Value::Str)
          continue;
        if (kind->s.compare(0, 7, "hidden_") == 0) continue;
        ArgSlot slot;
        slot.offset = (long)off->i;
        slot.size = (long)sz->i;
        slot.kind = kind->s;
        slots.push_back(slot);
      }
    }
    out[name->s] = slots;
  }
  return out;
}

}  // namespace tm_codeobject
