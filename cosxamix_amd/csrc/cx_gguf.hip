// cx_gguf.hip — GGUF v2/v3 reading and writing on the host
// (src/gguf.rs:119-436, src/gguf_write.rs). The GGUF container is the
// interface: header, typed metadata, a tensor table, then the data section
// aligned to general.alignment (default 32).
//
// Reading is the reference's Gguf::abrir: metadata and tensor table only; the
// bytes of a tensor are read on request, with the reference's bounds checks
// (Pesos::de, src/gguf.rs:413-436: every offset sum checked for overflow and
// against the file size). Writing lays out a file the reader (and the
// reference's) accepts: tensors in declaration order, each at a 32-byte
// aligned offset of the data section.

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "cx_internal.h"

namespace {

// TipoGgml (src/gguf.rs:39-116): every type the reference recognises, with
// its block geometry (values, bytes)
bool ggml_geometry(uint32_t t, uint64_t* vpb, uint64_t* bpb) {
  switch (t) {
    case 0: *vpb = 1; *bpb = 4; return true;      // F32
    case 1: *vpb = 1; *bpb = 2; return true;      // F16
    case 2: *vpb = 32; *bpb = 18; return true;    // Q4_0
    case 3: *vpb = 32; *bpb = 20; return true;    // Q4_1
    case 6: *vpb = 32; *bpb = 22; return true;    // Q5_0
    case 7: *vpb = 32; *bpb = 24; return true;    // Q5_1
    case 8: *vpb = 32; *bpb = 34; return true;    // Q8_0
    case 9: *vpb = 32; *bpb = 36; return true;    // Q8_1
    case 10: *vpb = 256; *bpb = 84; return true;  // Q2_K
    case 11: *vpb = 256; *bpb = 110; return true; // Q3_K
    case 12: *vpb = 256; *bpb = 144; return true; // Q4_K
    case 13: *vpb = 256; *bpb = 176; return true; // Q5_K
    case 14: *vpb = 256; *bpb = 210; return true; // Q6_K
    case 15: *vpb = 256; *bpb = 292; return true; // Q8_K
    default: return false;
  }
}

// Valor (src/gguf.rs:121-136): metadata value types 0..12
struct Value {
  uint32_t type = 0;
  uint64_t u = 0;   // integers and bool, as stored
  double f = 0.0;   // F32 / F64
  std::string s;    // string
  std::vector<Value> list;
};

// Valor::entero: any integer width, signed ones cast to u64 (src/gguf.rs:143-155)
bool value_int(const Value& v, uint64_t* out) {
  switch (v.type) {
    case 0: case 2: case 4: case 10: *out = v.u; return true;
    case 1: *out = (uint64_t)(int64_t)(int8_t)v.u; return true;
    case 3: *out = (uint64_t)(int64_t)(int16_t)v.u; return true;
    case 5: *out = (uint64_t)(int64_t)(int32_t)v.u; return true;
    case 11: *out = v.u; return true;
    default: return false;
  }
}
// Valor::decimal: floats, else the integer as f64 (src/gguf.rs:157-163)
bool value_float(const Value& v, double* out) {
  if (v.type == 6 || v.type == 12) {
    *out = v.f;
    return true;
  }
  uint64_t i;
  if (!value_int(v, &i)) return false;
  // a signed integer converts through its signed value
  if (v.type == 1 || v.type == 3 || v.type == 5 || v.type == 11)
    *out = (double)(int64_t)i;
  else
    *out = (double)i;
  return true;
}

struct Reader {
  FILE* f;
  std::string err;
  bool bytes(void* p, size_t n) {
    if (n && fread(p, 1, n, f) != n) {
      err = "truncated file: it ends inside the header";
      return false;
    }
    return true;
  }
  bool u32(uint32_t* v) {
    uint8_t b[4];
    if (!bytes(b, 4)) return false;
    *v = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
    return true;
  }
  bool u64(uint64_t* v) {
    uint32_t lo, hi;
    if (!u32(&lo) || !u32(&hi)) return false;
    *v = (uint64_t)lo | ((uint64_t)hi << 32);
    return true;
  }
  // src/gguf.rs:228-240: u64 length, bytes, no terminator; over 64 MiB means
  // the position is lost
  bool text(std::string* s) {
    uint64_t n;
    if (!u64(&n)) return false;
    if (n > 64ull * 1024 * 1024) {
      err = "a string of " + std::to_string(n) + " bytes: the file does not add up";
      return false;
    }
    s->resize(n);
    return bytes(s->empty() ? nullptr : &(*s)[0], n);
  }
  // src/gguf.rs:243-271
  bool value(uint32_t type, Value* v, int depth = 0) {
    v->type = type;
    uint8_t b[8] = {0};
    switch (type) {
      case 0: case 1: case 7:
        if (!bytes(b, 1)) return false;
        v->u = b[0];
        if (type == 7) v->u = b[0] != 0;
        return true;
      case 2: case 3:
        if (!bytes(b, 2)) return false;
        v->u = (uint64_t)b[0] | ((uint64_t)b[1] << 8);
        return true;
      case 4: case 5: {
        uint32_t x;
        if (!u32(&x)) return false;
        v->u = x;
        return true;
      }
      case 6: {
        uint32_t x;
        if (!u32(&x)) return false;
        float f;
        memcpy(&f, &x, 4);
        v->f = (double)f;
        return true;
      }
      case 8: return text(&v->s);
      case 9: {
        uint32_t inner;
        uint64_t n;
        if (!u32(&inner) || !u64(&n)) return false;
        if (depth > 4) {
          err = "metadata lists nested too deep";
          return false;
        }
        for (uint64_t i = 0; i < n; i++) {
          Value e;
          if (!value(inner, &e, depth + 1)) return false;
          v->list.push_back(std::move(e));
        }
        return true;
      }
      case 10: case 11: return u64(&v->u);
      case 12: {
        uint64_t x;
        if (!u64(&x)) return false;
        memcpy(&v->f, &x, 8);
        return true;
      }
      default:
        err = "unknown metadata type " + std::to_string(type);
        return false;
    }
  }
};

}  // namespace

struct cx_gguf {
  std::string path;
  uint32_t version = 0;
  uint64_t alignment = 32, data_start = 0, file_size = 0;
  std::map<std::string, Value> meta;
  std::vector<std::string> meta_order;
  std::vector<cx_gguf_tensor> tensors;
};

// ---------------------------------------------------------------- reading
// Gguf::abrir (src/gguf.rs:274-342)
int cx_gguf_read(const char* path, cx_gguf** out) {
  CX_REQUIRE(path && out, "gguf: null argument");
  *out = nullptr;
  FILE* f = fopen(path, "rb");
  CX_REQUIRE(f, "cannot open %s: %s", path, strerror(errno));
  std::unique_ptr<FILE, int (*)(FILE*)> guard(f, fclose);
  auto g = std::make_unique<cx_gguf>();
  g->path = path;
  Reader r{f, ""};
  char magic[4];
  if (!r.bytes(magic, 4) || memcmp(magic, "GGUF", 4) != 0) {
    cx_set_error("%s does not start with GGUF: not a file of this format", path);
    return CX_EINVAL;
  }
  uint64_t nt = 0, nm = 0;
  if (!r.u32(&g->version) || !r.u64(&nt) || !r.u64(&nm)) {
    cx_set_error("%s", r.err.c_str());
    return CX_EINVAL;
  }
  CX_REQUIRE(g->version == 2 || g->version == 3, "GGUF version %u: only 2 and 3 are read",
             g->version);
  for (uint64_t i = 0; i < nm; i++) {
    std::string key;
    uint32_t type;
    Value v;
    if (!r.text(&key) || !r.u32(&type) || !r.value(type, &v)) {
      cx_set_error("%s", r.err.c_str());
      return CX_EINVAL;
    }
    if (!g->meta.count(key)) g->meta_order.push_back(key);
    g->meta[key] = std::move(v);
  }
  for (uint64_t i = 0; i < nt; i++) {
    cx_gguf_tensor t{};
    std::string name;
    uint32_t nd;
    if (!r.text(&name) || !r.u32(&nd)) {
      cx_set_error("%s", r.err.c_str());
      return CX_EINVAL;
    }
    CX_REQUIRE(nd <= 4, "%s: %u dimensions, the format allows 4", name.c_str(), nd);
    CX_REQUIRE(name.size() < sizeof t.name, "gguf: tensor name of %zu bytes", name.size());
    memcpy(t.name, name.c_str(), name.size() + 1);
    t.n_dims = nd;
    uint64_t elems = 1;
    for (uint32_t d = 0; d < 4; d++) t.dims[d] = 1;
    for (uint32_t d = 0; d < nd; d++) {
      if (!r.u64(&t.dims[d])) {
        cx_set_error("%s", r.err.c_str());
        return CX_EINVAL;
      }
      CX_REQUIRE(t.dims[d] == 0 || elems <= UINT64_MAX / t.dims[d], "%s: too many elements",
                 name.c_str());
      elems *= t.dims[d];
    }
    uint32_t raw;
    if (!r.u32(&raw) || !r.u64(&t.offset)) {
      cx_set_error("%s", r.err.c_str());
      return CX_EINVAL;
    }
    uint64_t vpb, bpb;
    CX_REQUIRE(ggml_geometry(raw, &vpb, &bpb), "%s: unknown tensor type %u", name.c_str(),
               raw);
    t.type = (int)raw;
    t.elements = elems;
    t.bytes = elems / vpb * bpb;  // InfoTensor::bytes (src/gguf.rs:191-193)
    g->tensors.push_back(t);
  }
  // the data section starts aligned to general.alignment (default 32)
  uint64_t al = 32;
  auto it = g->meta.find("general.alignment");
  if (it != g->meta.end()) value_int(it->second, &al);  // left at 32 unless an integer
  g->alignment = al < 1 ? 1 : al;
  const long pos = ftell(f);
  CX_REQUIRE(pos >= 0, "gguf: cannot tell the file position");
  g->data_start = ((uint64_t)pos + g->alignment - 1) / g->alignment * g->alignment;
  CX_REQUIRE(fseek(f, 0, SEEK_END) == 0, "gguf: seek");
  const long end = ftell(f);
  CX_REQUIRE(end >= 0, "gguf: file size");
  g->file_size = (uint64_t)end;
  *out = g.release();
  return CX_OK;
}

void cx_gguf_release(cx_gguf* g) { delete g; }

const cx_gguf_tensor* cx_gguf_tensors(const cx_gguf* g, size_t* n) {
  *n = g->tensors.size();
  return g->tensors.data();
}

// Pesos::de (src/gguf.rs:413-436): [data_start + offset, + bytes) inside the
// file, every sum checked; then the bytes
int cx_gguf_range(const cx_gguf* g, const cx_gguf_tensor& t, uint64_t* from) {
  const uint64_t a = g->data_start + t.offset;
  CX_REQUIRE(a >= g->data_start, "%s: the offset overflows", t.name);
  const uint64_t b = a + t.bytes;
  CX_REQUIRE(b >= a, "%s: the size overflows", t.name);
  CX_REQUIRE(b <= g->file_size, "%s: reaches byte %llu and the file has %llu", t.name,
             (unsigned long long)b, (unsigned long long)g->file_size);
  *from = a;
  return CX_OK;
}

int cx_gguf_read_bytes(const cx_gguf* g, uint64_t from, void* host, size_t n, FILE* f) {
  CX_REQUIRE(fseek(f, (long)from, SEEK_SET) == 0, "gguf: seek to %llu", (unsigned long long)from);
  CX_REQUIRE(fread(host, 1, n, f) == n, "gguf: short read of %zu bytes", n);
  return CX_OK;
}

// ----------------------------------------------------------- the C ABI
extern "C" int cx_gguf_open(const char* path, cx_gguf** out) { return cx_gguf_read(path, out); }
extern "C" void cx_gguf_free(cx_gguf* g) { cx_gguf_release(g); }

extern "C" int cx_gguf_header(const cx_gguf* g, uint32_t* version, uint64_t* n_tensors,
                              uint64_t* n_meta, uint64_t* data_start, uint64_t* alignment) {
  CX_REQUIRE(g, "gguf: null handle");
  if (version) *version = g->version;
  if (n_tensors) *n_tensors = g->tensors.size();
  if (n_meta) *n_meta = g->meta.size();
  if (data_start) *data_start = g->data_start;
  if (alignment) *alignment = g->alignment;
  return CX_OK;
}

static const Value* find_meta(const cx_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->meta.find(key);
  return it == g->meta.end() ? nullptr : &it->second;
}

extern "C" int cx_gguf_meta_int(const cx_gguf* g, const char* key, uint64_t* out) {
  const Value* v = find_meta(g, key);
  CX_REQUIRE(v && out, "missing metadata %s", key ? key : "(null)");
  CX_REQUIRE(value_int(*v, out), "metadata %s: not an integer", key);
  return CX_OK;
}
extern "C" int cx_gguf_meta_float(const cx_gguf* g, const char* key, double* out) {
  const Value* v = find_meta(g, key);
  CX_REQUIRE(v && out, "missing metadata %s", key ? key : "(null)");
  CX_REQUIRE(value_float(*v, out), "metadata %s: not a number", key);
  return CX_OK;
}
// a string value, or element `index` of a list of strings (index < 0: the value itself)
extern "C" int cx_gguf_meta_str(const cx_gguf* g, const char* key, long index, char* buf,
                                size_t cap, size_t* len) {
  const Value* v = find_meta(g, key);
  CX_REQUIRE(v, "missing metadata %s", key ? key : "(null)");
  if (index >= 0) {
    CX_REQUIRE(v->type == 9 && (size_t)index < v->list.size(), "metadata %s: no element %ld",
               key, index);
    v = &v->list[(size_t)index];
  }
  CX_REQUIRE(v->type == 8, "metadata %s: not a string", key);
  if (len) *len = v->s.size();
  if (buf && cap) snprintf(buf, cap, "%s", v->s.c_str());
  return CX_OK;
}
// GGUF value type of a key, and the element count when it is a list
extern "C" int cx_gguf_meta_type(const cx_gguf* g, const char* key, uint32_t* type,
                                 uint64_t* count) {
  const Value* v = find_meta(g, key);
  CX_REQUIRE(v, "missing metadata %s", key ? key : "(null)");
  if (type) *type = v->type;
  if (count) *count = v->type == 9 ? v->list.size() : 1;
  return CX_OK;
}

extern "C" int cx_gguf_find(const cx_gguf* g, const char* name) {
  if (!g || !name) return -1;
  for (size_t i = 0; i < g->tensors.size(); i++)
    if (strcmp(g->tensors[i].name, name) == 0) return (int)i;
  return -1;
}

extern "C" int cx_gguf_tensor_info(const cx_gguf* g, int idx, cx_gguf_tensor* out) {
  CX_REQUIRE(g && out && idx >= 0 && (size_t)idx < g->tensors.size(), "gguf: tensor %d", idx);
  *out = g->tensors[(size_t)idx];
  return CX_OK;
}

// Gguf::datos_de / Pesos::de: the tensor's bytes into a host buffer
extern "C" int cx_gguf_tensor_read(const cx_gguf* g, const cx_gguf_tensor* t, void* host,
                                   size_t cap) {
  CX_REQUIRE(g && t, "gguf: null argument");
  uint64_t from;
  int rc = cx_gguf_range(g, *t, &from);  // the range first: it is what can be wrong in a file
  if (rc) return rc;
  CX_REQUIRE(host && cap >= t->bytes, "gguf: %s needs %llu bytes, the buffer has %zu", t->name,
             (unsigned long long)t->bytes, host ? cap : (size_t)0);
  FILE* f = fopen(g->path.c_str(), "rb");
  CX_REQUIRE(f, "cannot open %s: %s", g->path.c_str(), strerror(errno));
  rc = cx_gguf_read_bytes(g, from, host, (size_t)t->bytes, f);
  fclose(f);
  return rc;
}

// ---------------------------------------------------------------- writing
namespace {
struct Writer {
  FILE* f;
  bool ok = true;
  void bytes(const void* p, size_t n) { ok = ok && (n == 0 || fwrite(p, 1, n, f) == n); }
  void u32(uint32_t v) {
    uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
    bytes(b, 4);
  }
  void u64(uint64_t v) {
    u32((uint32_t)v);
    u32((uint32_t)(v >> 32));
  }
  void text(const std::string& s) {
    u64(s.size());
    bytes(s.data(), s.size());
  }
};
}  // namespace

// Escritor::escribir's layout (src/gguf_write.rs): header, metadata, tensor
// table with 32-byte aligned offsets, zero padding to the data section, data
int cx_gguf_write(const char* path, const std::vector<cx_gguf_meta>& meta,
                  const std::vector<cx_gguf_tensor>& tensors,
                  const std::vector<const void*>& host_data) {
  CX_REQUIRE(path && tensors.size() == host_data.size(), "gguf write: bad arguments");
  FILE* f = fopen(path, "wb");
  CX_REQUIRE(f, "cannot create %s: %s", path, strerror(errno));
  std::unique_ptr<FILE, int (*)(FILE*)> guard(f, fclose);
  Writer w{f};
  w.bytes("GGUF", 4);
  w.u32(3);
  w.u64(tensors.size());
  w.u64(meta.size());
  for (const cx_gguf_meta& m : meta) {
    w.text(m.key);
    w.u32(m.type);
    switch (m.type) {
      case 4: w.u32((uint32_t)m.u); break;
      case 10: w.u64(m.u); break;
      case 6: {
        const float v = (float)m.f;
        uint32_t x;
        memcpy(&x, &v, 4);
        w.u32(x);
        break;
      }
      case 8: w.text(m.s); break;
      default:
        cx_set_error("gguf write: metadata type %u is not written here", m.type);
        return CX_EINVAL;
    }
  }
  uint64_t off = 0;
  std::vector<uint64_t> offs;
  for (const cx_gguf_tensor& t : tensors) {
    w.text(t.name);
    w.u32(t.n_dims);
    for (uint32_t d = 0; d < t.n_dims; d++) w.u64(t.dims[d]);
    w.u32((uint32_t)t.type);
    w.u64(off);
    offs.push_back(off);
    off = (off + t.bytes + 31) / 32 * 32;
  }
  long pos = ftell(f);
  CX_REQUIRE(pos >= 0, "gguf write: position");
  static const uint8_t zero[32] = {0};
  w.bytes(zero, (32 - (size_t)pos % 32) % 32);
  uint64_t at = 0;
  for (size_t i = 0; i < tensors.size(); i++) {
    w.bytes(zero, (size_t)(offs[i] - at));
    w.bytes(host_data[i], (size_t)tensors[i].bytes);
    at = offs[i] + tensors[i].bytes;
  }
  CX_REQUIRE(w.ok, "gguf write: %s: %s", path, strerror(errno));
  return CX_OK;
}
