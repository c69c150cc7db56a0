// GGUF container reader and AoS -> SoA repack (host code).
//
// Replaces what the reference takes from the PyPI `gguf` package
// (gguf_support.py:101-121: `GGUFReader(path, "c")`, its `.tensors` and
// `get_field`) and the byte shuffle of `pack_gguf_soa` (quantization.py:67-90).
//
// GGUF layout (versions 2 and 3, little-endian):
//   "GGUF", u32 version, u64 tensor count, u64 metadata count,
//   metadata: string key, u32 value type, value,
//   tensor infos: string name, u32 n_dims, u64 dims[n_dims], u32 ggml type,
//                 u64 data offset,
//   padding to `general.alignment` (default 32), tensor data.
// Strings are a u64 byte length and the bytes; an array value is a u32
// element type, a u64 count and the elements. dims[0] varies fastest.
//
// The file is memory-mapped once. Every length, count and offset is checked
// against the mapping before it is used, so a truncated or corrupt file is an
// error, never an out-of-bounds read.
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/svq.h"

namespace svq {
int set_error(int code, const char* msg);  // svq_api.hip
}

namespace {

int gfail(int code, const char* fmt, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return svq::set_error(code, buf);
}

// Value types of GGUF metadata.
enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
  kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12,
};

int scalar_bytes(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
  }
  return 0;
}

// Bytes per block and elements per block of the ggml tensor types whose
// storage size is known here (the ggml block structures).
bool ggml_block(uint32_t type, int* block_bytes, int* block_elems) {
  struct B { uint32_t type; int bytes, elems; };
  static const B table[] = {
      {0, 4, 1},      // F32
      {1, 2, 1},      // F16
      {2, 18, 32},    // Q4_0: fp16 d, 16 nibble bytes
      {3, 20, 32},    // Q4_1: fp16 d, m, 16 nibble bytes
      {6, 22, 32},    // Q5_0: fp16 d, u32 high bits, 16 nibble bytes
      {7, 24, 32},    // Q5_1
      {8, 34, 32},    // Q8_0: fp16 d, 32 int8
      {9, 36, 32},    // Q8_1
      {10, 84, 256},  // Q2_K
      {11, 110, 256}, // Q3_K
      {12, 144, 256}, // Q4_K
      {13, 176, 256}, // Q5_K
      {14, 210, 256}, // Q6_K
      {15, 292, 256}, // Q8_K
      {24, 1, 1},     // I8
      {25, 2, 1},     // I16
      {26, 4, 1},     // I32
      {27, 8, 1},     // I64
      {28, 8, 1},     // F64
      {30, 2, 1},     // BF16
  };
  for (const B& b : table)
    if (b.type == type) {
      *block_bytes = b.bytes;
      *block_elems = b.elems;
      return true;
    }
  return false;
}

struct Cursor {
  const uint8_t* base;
  size_t size, pos;
  bool take(size_t n, const uint8_t** p) {
    if (n > size - pos) return false;
    *p = base + pos;
    pos += n;
    return true;
  }
  template <class T> bool get(T* v) {
    const uint8_t* p;
    if (!take(sizeof(T), &p)) return false;
    memcpy(v, p, sizeof(T));
    return true;
  }
  bool string(const uint8_t** p, uint64_t* len) {
    return get(len) && take(*len, p);
  }
};

}  // namespace

struct svq_gguf {
  int fd = -1;
  uint8_t* map = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t alignment = 32;
  size_t data_start = 0;
  struct KV {
    std::string key;
    uint32_t type;
    const uint8_t* value;  // first byte of the value (of the elements for arrays)
    uint64_t nbytes;       // bytes of the value (of the elements for arrays)
    uint32_t elem_type;    // arrays: element type
    uint64_t count;        // arrays: element count; scalars and strings: 1
  };
  std::vector<KV> kvs;
  struct Tensor {
    std::string name;
    uint32_t type;
    uint32_t n_dims;
    int64_t dims[4];
    uint64_t offset;
    uint64_t nbytes;
  };
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, int64_t> tensor_index, kv_index;

  ~svq_gguf() {
    if (map) munmap(map, size);
    if (fd >= 0) close(fd);
  }
};

namespace {

// Skip one value of type t at the cursor (arrays of arrays included, to a
// bounded depth), leaving the byte range it covers.
bool skip_value(Cursor& c, uint32_t t, int depth) {
  if (depth > 4) return false;
  if (const int b = scalar_bytes(t)) {
    const uint8_t* p;
    return c.take((size_t)b, &p);
  }
  if (t == kString) {
    const uint8_t* p;
    uint64_t len;
    return c.string(&p, &len);
  }
  if (t == kArray) {
    uint32_t et;
    uint64_t n;
    if (!c.get(&et) || !c.get(&n)) return false;
    if (const int b = scalar_bytes(et)) {
      if (n > (c.size - c.pos) / (uint64_t)b) return false;
      c.pos += (size_t)(n * (uint64_t)b);
      return true;
    }
    for (uint64_t i = 0; i < n; ++i)
      if (!skip_value(c, et, depth + 1)) return false;
    return true;
  }
  return false;
}

int parse(svq_gguf* g) {
  Cursor c{g->map, g->size, 0};
  const uint8_t* magic;
  if (!c.take(4, &magic) || memcmp(magic, "GGUF", 4) != 0)
    return gfail(SVQ_E_FORMAT, "not a GGUF file (bad magic)");
  uint64_t n_tensors, n_kv;
  if (!c.get(&g->version) || !c.get(&n_tensors) || !c.get(&n_kv))
    return gfail(SVQ_E_FORMAT, "truncated GGUF header");
  if (g->version != 2 && g->version != 3)
    return gfail(SVQ_E_FORMAT, "unsupported GGUF version %u", g->version);
  // Each metadata entry and tensor info takes at least 12 bytes: a count past
  // the file size is corrupt (and must not size an allocation).
  if (n_kv > g->size / 12 || n_tensors > g->size / 12)
    return gfail(SVQ_E_FORMAT, "corrupt GGUF header counts");
  g->kvs.reserve((size_t)n_kv);
  for (uint64_t i = 0; i < n_kv; ++i) {
    svq_gguf::KV kv{};
    const uint8_t* key;
    uint64_t key_len;
    if (!c.string(&key, &key_len) || !c.get(&kv.type))
      return gfail(SVQ_E_FORMAT, "truncated GGUF metadata entry %llu", (unsigned long long)i);
    kv.key.assign((const char*)key, (size_t)key_len);
    kv.count = 1;
    if (kv.type == kString) {
      uint64_t len;
      if (!c.string(&kv.value, &len))
        return gfail(SVQ_E_FORMAT, "truncated GGUF metadata value %s", kv.key.c_str());
      kv.nbytes = len;
    } else if (kv.type == kArray) {
      if (!c.get(&kv.elem_type) || !c.get(&kv.count))
        return gfail(SVQ_E_FORMAT, "truncated GGUF array %s", kv.key.c_str());
      const size_t start = c.pos;
      Cursor probe = c;
      probe.pos -= 12;  // re-read the array header in skip_value
      if (!skip_value(probe, kArray, 0))
        return gfail(SVQ_E_FORMAT, "corrupt GGUF array %s", kv.key.c_str());
      kv.value = g->map + start;
      kv.nbytes = probe.pos - start;
      c.pos = probe.pos;
    } else if (const int b = scalar_bytes(kv.type)) {
      if (!c.take((size_t)b, &kv.value))
        return gfail(SVQ_E_FORMAT, "truncated GGUF metadata value %s", kv.key.c_str());
      kv.nbytes = (uint64_t)b;
    } else {
      return gfail(SVQ_E_FORMAT, "unknown GGUF value type %u for %s", kv.type, kv.key.c_str());
    }
    if (kv.key == "general.alignment") {
      if (kv.type != kU32) return gfail(SVQ_E_FORMAT, "general.alignment must be a u32");
      uint32_t a;
      memcpy(&a, kv.value, 4);
      if (a == 0 || (a & (a - 1)) != 0)
        return gfail(SVQ_E_FORMAT, "general.alignment %u is not a power of two", a);
      g->alignment = a;
    }
    g->kv_index.emplace(kv.key, (int64_t)g->kvs.size());
    g->kvs.push_back(std::move(kv));
  }
  g->tensors.reserve((size_t)n_tensors);
  for (uint64_t i = 0; i < n_tensors; ++i) {
    svq_gguf::Tensor t{};
    const uint8_t* name;
    uint64_t name_len;
    if (!c.string(&name, &name_len) || !c.get(&t.n_dims))
      return gfail(SVQ_E_FORMAT, "truncated GGUF tensor info %llu", (unsigned long long)i);
    t.name.assign((const char*)name, (size_t)name_len);
    if (t.n_dims < 1 || t.n_dims > 4)
      return gfail(SVQ_E_FORMAT, "tensor %s has %u dimensions", t.name.c_str(), t.n_dims);
    uint64_t elems = 1;
    for (uint32_t d = 0; d < 4; ++d) t.dims[d] = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      uint64_t v;
      if (!c.get(&v)) return gfail(SVQ_E_FORMAT, "truncated dims of tensor %s", t.name.c_str());
      if (v == 0 || v > ((uint64_t)1 << 40) || elems > ((uint64_t)1 << 48) / v)
        return gfail(SVQ_E_FORMAT, "tensor %s has an invalid dimension", t.name.c_str());
      t.dims[d] = (int64_t)v;
      elems *= v;
    }
    if (!c.get(&t.type) || !c.get(&t.offset))
      return gfail(SVQ_E_FORMAT, "truncated GGUF tensor info %s", t.name.c_str());
    int bb, be;
    if (!ggml_block(t.type, &bb, &be))
      return gfail(SVQ_E_DTYPE, "tensor %s has unsupported ggml type %u", t.name.c_str(), t.type);
    if (t.dims[0] % be != 0)
      return gfail(SVQ_E_FORMAT, "tensor %s: row of %lld is not whole blocks of %d",
                   t.name.c_str(), (long long)t.dims[0], be);
    t.nbytes = elems / (uint64_t)be * (uint64_t)bb;
    g->tensors.push_back(std::move(t));
  }
  g->data_start = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
  if (g->data_start > g->size && !g->tensors.empty())
    return gfail(SVQ_E_FORMAT, "GGUF file ends before its tensor data");
  const uint64_t data_bytes = g->size >= g->data_start ? g->size - g->data_start : 0;
  for (size_t i = 0; i < g->tensors.size(); ++i) {
    const svq_gguf::Tensor& t = g->tensors[i];
    if (t.offset % g->alignment != 0)
      return gfail(SVQ_E_FORMAT, "tensor %s data is not aligned to %llu", t.name.c_str(),
                   (unsigned long long)g->alignment);
    if (t.offset > data_bytes || t.nbytes > data_bytes - t.offset)
      return gfail(SVQ_E_FORMAT, "tensor %s data lies outside the file", t.name.c_str());
    g->tensor_index.emplace(t.name, (int64_t)i);  // first occurrence of a name
  }
  return 0;
}

}  // namespace

extern "C" {

int svq_gguf_open(const char* path, int writable_copy, svq_gguf** out) {
  if (!path || !out) return gfail(SVQ_E_NULL, "NULL path or out");
  *out = nullptr;
  svq_gguf* g = new svq_gguf();
  g->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (g->fd < 0) {
    delete g;
    return gfail(SVQ_E_IO, "cannot open %s", path);
  }
  struct stat st;
  if (fstat(g->fd, &st) != 0) {
    delete g;
    return gfail(SVQ_E_IO, "cannot stat %s", path);
  }
  if (st.st_size < 24) {
    delete g;
    return gfail(SVQ_E_FORMAT, "%s is too small for a GGUF header", path);
  }
  g->size = (size_t)st.st_size;
  // Copy-on-write mapping: writes through it stay private to this process.
  const int prot = writable_copy ? PROT_READ | PROT_WRITE : PROT_READ;
  void* m = mmap(nullptr, g->size, prot, MAP_PRIVATE, g->fd, 0);
  if (m == MAP_FAILED) {
    delete g;
    return gfail(SVQ_E_IO, "cannot map %s", path);
  }
  g->map = static_cast<uint8_t*>(m);
  const int rc = parse(g);
  if (rc != 0) {
    delete g;
    return rc;
  }
  *out = g;
  return 0;
}

void svq_gguf_close(svq_gguf* g) { delete g; }

int svq_gguf_version(const svq_gguf* g) { return g ? (int)g->version : SVQ_E_NULL; }

int64_t svq_gguf_alignment(const svq_gguf* g) { return g ? (int64_t)g->alignment : SVQ_E_NULL; }

int64_t svq_gguf_kv_count(const svq_gguf* g) {
  return g ? (int64_t)g->kvs.size() : gfail(SVQ_E_NULL, "NULL reader");
}

int64_t svq_gguf_find_kv(const svq_gguf* g, const char* key) {
  if (!g || !key) return gfail(SVQ_E_NULL, "NULL reader or key");
  const auto it = g->kv_index.find(key);
  return it == g->kv_index.end() ? -1 : it->second;
}

int svq_gguf_kv(const svq_gguf* g, int64_t i, const char** key, int* type, const void** value,
                int64_t* nbytes, int* elem_type, int64_t* count) {
  if (!g) return gfail(SVQ_E_NULL, "NULL reader");
  if (i < 0 || i >= (int64_t)g->kvs.size())
    return gfail(SVQ_E_SHAPE, "metadata index %lld out of range", (long long)i);
  const svq_gguf::KV& kv = g->kvs[(size_t)i];
  if (key) *key = kv.key.c_str();
  if (type) *type = (int)kv.type;
  if (value) *value = kv.value;
  if (nbytes) *nbytes = (int64_t)kv.nbytes;
  if (elem_type) *elem_type = kv.type == kArray ? (int)kv.elem_type : -1;
  if (count) *count = (int64_t)kv.count;
  return 0;
}

int64_t svq_gguf_tensor_count(const svq_gguf* g) {
  return g ? (int64_t)g->tensors.size() : gfail(SVQ_E_NULL, "NULL reader");
}

int64_t svq_gguf_find_tensor(const svq_gguf* g, const char* name) {
  if (!g || !name) return gfail(SVQ_E_NULL, "NULL reader or name");
  const auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : it->second;
}

int svq_gguf_tensor(const svq_gguf* g, int64_t i, const char** name, int* ggml_type,
                    int* n_dims, int64_t* dims, int64_t* data_offset, int64_t* nbytes) {
  if (!g) return gfail(SVQ_E_NULL, "NULL reader");
  if (i < 0 || i >= (int64_t)g->tensors.size())
    return gfail(SVQ_E_SHAPE, "tensor index %lld out of range", (long long)i);
  const svq_gguf::Tensor& t = g->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (ggml_type) *ggml_type = (int)t.type;
  if (n_dims) *n_dims = (int)t.n_dims;
  if (dims)
    for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
  if (data_offset) *data_offset = (int64_t)(g->data_start + t.offset);
  if (nbytes) *nbytes = (int64_t)t.nbytes;
  return 0;
}

const void* svq_gguf_tensor_data(const svq_gguf* g, int64_t i) {
  if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return nullptr;
  return g->map + g->data_start + g->tensors[(size_t)i].offset;
}

int svq_pack_soa(const uint8_t* aos, int64_t nblocks, int qtype, uint8_t* q, uint8_t* s,
                 int threads) {
  if (qtype != SVQ_Q4_0 && qtype != SVQ_Q5_0 && qtype != SVQ_Q8_0)
    return gfail(SVQ_E_QTYPE, "unsupported qtype %d", qtype);
  if (nblocks < 0) return gfail(SVQ_E_SHAPE, "negative block count");
  if (nblocks == 0) return 0;
  if (!aos || !q || !s) return gfail(SVQ_E_NULL, "NULL aos, q or s");
  const int64_t bb = qtype == SVQ_Q4_0 ? 18 : qtype == SVQ_Q5_0 ? 22 : 34;
  const int64_t w = bb - 2;
  // A few MiB per thread; at most the hardware threads (and 64).
  const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
  int64_t nt = threads > 0 ? threads : (int64_t)hw;
  nt = std::min<int64_t>({nt, 64, std::max<int64_t>(1, nblocks * bb / (4 << 20))});
  auto work = [=](int64_t b0, int64_t b1) {
    for (int64_t b = b0; b < b1; ++b) {
      const uint8_t* src = aos + b * bb;
      s[2 * b] = src[0];
      s[2 * b + 1] = src[1];
      memcpy(q + b * w, src + 2, (size_t)w);
    }
  };
  if (nt <= 1) {
    work(0, nblocks);
    return 0;
  }
  std::vector<std::thread> pool;
  pool.reserve((size_t)nt);
  for (int64_t t = 0; t < nt; ++t)
    pool.emplace_back(work, nblocks * t / nt, nblocks * (t + 1) / nt);
  for (std::thread& th : pool) th.join();
  return 0;
}

}  // extern "C"
