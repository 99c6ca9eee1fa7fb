// GGUF (v3) weight files for the quantized Linear path.
//
// The reference parses a GGUF file with buffered stream reads
// (src/gguf.cc:398-573), reads each tensor into a host vector
// (readGgufTensorRaw, src/gguf.cc:621-662), builds AoS block vectors
// (src/gguf_loader.cc:118-199) and uploads those (src/cuda_weight_upload.cc).
// Here the file is memory-mapped once; tensor data is handed out as
// pointers into the mapping, and mlq_gguf_upload copies a quantized tensor
// from the mapping straight to device memory and repacks it there into the
// tiled layout, so no host-side block vector exists.
//
// Validation follows the reference reader's rules (same accepted files):
// magic "GGUF", version 3, at most 1e6 tensors / metadata entries, strings
// <= 16 MiB, arrays <= 1e7 elements (nested arrays allowed; this reader
// stops at 64 levels), unique metadata keys and tensor names, 1..8
// non-zero dimensions, quantized element counts a multiple of 32, every
// sized tensor's data inside the file, and general.alignment (default 32)
// a power of two <= 1 MiB. The reference reads the alignment by printing
// the value and parsing the text as an unsigned decimal
// (src/gguf.cc:366-390), so integer values, floats whose default "%g"
// text is a plain integer, and decimal strings are accepted; booleans,
// arrays and anything else are not.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_set>
#include <vector>

#include "kernels/launch.h"
#include "mlq.h"

struct mlq_gguf {
  const uint8_t* map = nullptr;
  size_t size = 0;
  uint64_t data_offset = 0;
  uint64_t alignment = 32;
  std::vector<std::string> names;
  std::vector<mlq_gguf_tensor> tensors;  // name pointers into `names`
};

namespace {

thread_local std::string g_error;

constexpr uint64_t kMaxEntries = 1000000;
constexpr uint64_t kMaxString = 16ull << 20;
constexpr uint64_t kMaxArray = 10000000;
constexpr uint32_t kMaxDims = 8;
constexpr uint64_t kMaxAlignment = 1ull << 20;

// GGUF metadata value types
enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
  kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};

int scalar_size(uint32_t t) {
  switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
  }
}

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
  const uint8_t* p;
  size_t size, pos = 0;
  bool take(void* out, size_t n) {
    if (n > size - pos) return false;
    std::memcpy(out, p + pos, n);
    pos += n;
    return true;
  }
  bool skip(uint64_t n) {
    if (n > size - pos) return false;
    pos += n;
    return true;
  }
  bool u32(uint32_t& v) { return take(&v, 4); }
  bool u64(uint64_t& v) { return take(&v, 8); }
  bool str(std::string& s) {
    uint64_t n;
    if (!u64(n) || n > kMaxString || n > size - pos) return false;
    s.assign((const char*)p + pos, n);
    pos += n;
    return true;
  }
};

bool mul_ok(uint64_t a, uint64_t b, uint64_t& out) {
  if (a != 0 && b > UINT64_MAX / a) return false;
  out = a * b;
  return true;
}

// Byte size of a tensor's data (0 for types without a known size).
bool data_bytes(uint32_t type, const uint64_t* dims, uint32_t nd, uint64_t& out) {
  uint64_t numel = 1;
  for (uint32_t i = 0; i < nd; ++i)
    if (dims[i] == 0 || !mul_ok(numel, dims[i], numel)) return false;
  switch (type) {
    case 0: return mul_ok(numel, 4, out);  // F32
    case 1: return mul_ok(numel, 2, out);  // F16
    case 2: case 3: case 8: {              // Q4_0, Q4_1, Q8_0: 32 per block
      if (numel % 32 != 0) return false;
      return mul_ok(numel / 32, type == 2 ? 18 : type == 3 ? 20 : 34, out);
    }
    default: out = 0; return true;
  }
}

int fail(const std::string& msg) {
  g_error = msg;
  return MLQ_ERR_FORMAT;
}

// Skip one metadata value of type t (arrays recursively).
bool skip_value(Cursor& c, uint32_t t, int depth) {
  if (t == kString) {
    std::string v;
    return c.str(v);
  }
  if (t == kArray) {
    uint32_t et;
    uint64_t n;
    if (depth >= 64 || !c.u32(et) || !c.u64(n) || n > kMaxArray) return false;
    const int es = scalar_size(et);
    if (es != 0) return n * (uint64_t)es <= c.size - c.pos && c.skip(n * (uint64_t)es);
    for (uint64_t j = 0; j < n; ++j)
      if (!skip_value(c, et, depth + 1)) return false;
    return true;
  }
  const int sz = scalar_size(t);
  return sz != 0 && c.skip((uint64_t)sz);
}

// The reference's reading of general.alignment: the value's decimal text
// parsed as std::stoull does (leading blanks, optional sign, all of it).
bool alignment_value(Cursor& c, uint32_t t, uint64_t& out) {
  auto from_text = [&](const std::string& s) {
    size_t i = 0;
    while (i < s.size() && (s[i] == ' ' || (s[i] >= '\t' && s[i] <= '\r'))) ++i;
    bool neg = false;
    if (i < s.size() && (s[i] == '+' || s[i] == '-')) neg = s[i++] == '-';
    if (i == s.size()) return false;
    uint64_t v = 0;
    for (; i < s.size(); ++i) {
      if (s[i] < '0' || s[i] > '9') return false;
      const uint64_t d = (uint64_t)(s[i] - '0');
      if (v > (UINT64_MAX - d) / 10) return false;  // out of range
      v = v * 10 + d;
    }
    out = neg ? (uint64_t)0 - v : v;  // stoull wraps negative values
    return true;
  };
  uint64_t raw = 0;
  switch (t) {
    case kString: {
      std::string s;
      return c.str(s) && from_text(s);
    }
    case kU8: case kU16: case kU32: case kU64:
      if (!c.take(&raw, scalar_size(t))) return false;
      out = raw;
      return true;
    case kI8: case kI16: case kI32: case kI64: {
      if (!c.take(&raw, scalar_size(t))) return false;
      const int sh = 64 - 8 * scalar_size(t);
      out = (uint64_t)(((int64_t)(raw << sh)) >> sh);  // negative -> wraps
      return true;
    }
    case kF32: case kF64: {
      double v;
      if (t == kF32) {
        float f;
        if (!c.take(&f, 4)) return false;
        v = f;
      } else if (!c.take(&v, 8)) {
        return false;
      }
      // the text an ostream prints by default (%g, 6 significant digits)
      char buf[64];
      std::snprintf(buf, sizeof(buf), "%g", v);
      return from_text(buf);
    }
    default:
      return false;
  }
}

int parse(mlq_gguf& g) {
  Cursor c{g.map, g.size};
  char magic[4];
  uint32_t version;
  uint64_t n_tensors, n_kv;
  if (!c.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return fail("invalid GGUF magic");
  if (!c.u32(version)) return fail("failed to read version");
  if (version != 3) return fail("unsupported GGUF version: " + std::to_string(version));
  if (!c.u64(n_tensors) || !c.u64(n_kv)) return fail("failed to read header counts");
  if (n_tensors > kMaxEntries) return fail("too many tensors");
  if (n_kv > kMaxEntries) return fail("too many metadata entries");

  std::unordered_set<std::string> keys;
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key;
    uint32_t type;
    if (!c.str(key)) return fail("failed to read metadata key " + std::to_string(i));
    if (!keys.insert(key).second) return fail("duplicate metadata key: " + key);
    if (!c.u32(type)) return fail("failed to read metadata type for key: " + key);
    if (key == "general.alignment") {
      const size_t at = c.pos;
      uint64_t v = 0;
      if (!alignment_value(c, type, v)) {
        // well-formed but not a usable number, or malformed
        c.pos = at;
        if (!skip_value(c, type, 0)) return fail("failed to read metadata value for key: " + key);
        return fail("invalid general.alignment");
      }
      if (v == 0 || v > kMaxAlignment || (v & (v - 1)) != 0)
        return fail("invalid general.alignment");
      g.alignment = v;
    } else if (!skip_value(c, type, 0)) {
      return fail("failed to read metadata value for key: " + key);
    }
  }

  g.names.resize(n_tensors);
  g.tensors.resize(n_tensors);
  std::unordered_set<std::string> seen;
  for (uint64_t i = 0; i < n_tensors; ++i) {
    mlq_gguf_tensor& t = g.tensors[i];
    std::memset(&t, 0, sizeof(t));
    if (!c.str(g.names[i])) return fail("failed to read tensor name " + std::to_string(i));
    const std::string& name = g.names[i];
    if (!c.u32(t.n_dims)) return fail("failed to read tensor n_dims for: " + name);
    if (t.n_dims == 0 || t.n_dims > kMaxDims) return fail("invalid tensor n_dims for: " + name);
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      if (!c.u64(t.dims[d])) return fail("failed to read tensor shape for: " + name);
      if (t.dims[d] == 0) return fail("invalid zero tensor dimension for: " + name);
    }
    uint64_t rel;
    if (!c.u32(t.ggml_type)) return fail("failed to read tensor type for: " + name);
    if (!c.u64(rel)) return fail("failed to read tensor offset for: " + name);
    if (!seen.insert(name).second) return fail("duplicate tensor name: " + name);
    t.offset = rel;  // relative until the data section is known
  }
  const uint64_t pad = (g.alignment - c.pos % g.alignment) % g.alignment;
  g.data_offset = c.pos + pad;
  if (g.data_offset > g.size) return fail("GGUF file ended before tensor data section");
  for (uint64_t i = 0; i < n_tensors; ++i) {
    mlq_gguf_tensor& t = g.tensors[i];
    t.name = g.names[i].c_str();
    if (!data_bytes(t.ggml_type, t.dims, t.n_dims, t.bytes))
      return fail("invalid tensor data size for: " + g.names[i]);
    const uint64_t rel = t.offset;
    if (rel > UINT64_MAX - g.data_offset) return fail("tensor offset overflow for: " + g.names[i]);
    t.offset = g.data_offset + rel;
    if (t.bytes == 0) continue;
    if (t.bytes > UINT64_MAX - t.offset) return fail("tensor data range overflow for: " + g.names[i]);
    if (t.offset + t.bytes > g.size) return fail("tensor data outside file bounds: " + g.names[i]);
  }
  return MLQ_OK;
}

}  // namespace

extern "C" {

const char* mlq_gguf_last_error(void) { return g_error.c_str(); }

int mlq_gguf_open(const char* path, mlq_gguf** out) {
  if (path == nullptr || out == nullptr) return MLQ_ERR_INVALID_ARG;
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) return fail(std::string("failed to open: ") + path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    ::close(fd);
    return fail(std::string("failed to open: ") + path);
  }
  void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (map == MAP_FAILED) return fail(std::string("failed to map: ") + path);
  mlq_gguf* g = new mlq_gguf;
  g->map = (const uint8_t*)map;
  g->size = (size_t)st.st_size;
  const int rc = parse(*g);
  if (rc != MLQ_OK) {
    munmap((void*)g->map, g->size);
    delete g;
    return rc;
  }
  g_error.clear();
  *out = g;
  return MLQ_OK;
}

void mlq_gguf_close(mlq_gguf* g) {
  if (g == nullptr) return;
  munmap((void*)g->map, g->size);
  delete g;
}

int mlq_gguf_tensor_count(const mlq_gguf* g, int64_t* count) {
  if (g == nullptr || count == nullptr) return MLQ_ERR_INVALID_ARG;
  *count = (int64_t)g->tensors.size();
  return MLQ_OK;
}

int mlq_gguf_data_offset(const mlq_gguf* g, uint64_t* offset, uint64_t* alignment) {
  if (g == nullptr || offset == nullptr || alignment == nullptr) return MLQ_ERR_INVALID_ARG;
  *offset = g->data_offset;
  *alignment = g->alignment;
  return MLQ_OK;
}

int mlq_gguf_tensor_info(const mlq_gguf* g, int64_t index, mlq_gguf_tensor* out) {
  if (g == nullptr || out == nullptr) return MLQ_ERR_INVALID_ARG;
  if (index < 0 || index >= (int64_t)g->tensors.size()) return MLQ_ERR_INVALID_ARG;
  *out = g->tensors[(size_t)index];
  return MLQ_OK;
}

int mlq_gguf_find(const mlq_gguf* g, const char* name, int64_t* index) {
  if (g == nullptr || name == nullptr || index == nullptr) return MLQ_ERR_INVALID_ARG;
  for (size_t i = 0; i < g->names.size(); ++i)
    if (g->names[i] == name) {
      *index = (int64_t)i;
      return MLQ_OK;
    }
  *index = -1;
  return MLQ_ERR_SHAPE;
}

const void* mlq_gguf_data(const mlq_gguf* g, int64_t index) {
  if (g == nullptr || index < 0 || index >= (int64_t)g->tensors.size()) return nullptr;
  const mlq_gguf_tensor& t = g->tensors[(size_t)index];
  return t.bytes ? g->map + t.offset : nullptr;
}

int mlq_gguf_upload(const mlq_gguf* g, int64_t index, void* aos_dev, size_t aos_bytes,
                    mlq_weight* w, mlq_stream_t stream) {
  if (g == nullptr || w == nullptr || aos_dev == nullptr || w->base == nullptr)
    return MLQ_ERR_INVALID_ARG;
  if (index < 0 || index >= (int64_t)g->tensors.size()) return MLQ_ERR_INVALID_ARG;
  const mlq_gguf_tensor& t = g->tensors[(size_t)index];
  int type;
  switch (t.ggml_type) {
    case 8: type = MLQ_Q8_0; break;
    case 2: type = MLQ_Q4_0; break;
    case 3: type = MLQ_Q4_1; break;
    default: return MLQ_ERR_UNSUPPORTED;
  }
  // a Linear weight: GGUF dims [k, n] (k innermost) = the [n][k] matrix
  if (t.n_dims != 2 || t.dims[0] > INT32_MAX || t.dims[1] > INT32_MAX) return MLQ_ERR_SHAPE;
  const int k = (int)t.dims[0], n = (int)t.dims[1];
  if (w->type != type || w->n != n || w->k != k) return MLQ_ERR_SHAPE;
  if (aos_bytes < t.bytes) return MLQ_ERR_BUFFER_TOO_SMALL;
  const hipStream_t s = (hipStream_t)stream;
  // pageable source: the runtime stages the copy; the mapping is read once
  hipError_t e = hipMemcpyAsync(aos_dev, g->map + t.offset, t.bytes, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = mlq::launch_repack(type, aos_dev, n, k, *w, s);
  return mlq::record_hip(e);
}

}  // extern "C"
