// libosmos MI355X - GGUF model files as data (include/osmos/model/gguf.h): gguf_create, gguf_header, gguf_destroy,
// gguf_tensor, gguf_kv, gguf_bytes, gguf_int. Host code.
//
// What it accepts and refuses follows the reference's reader (src/model/gguf.c:59-199, gguf_read.c:1-151): GGUF
// version 3, little-endian; metadata values of the 13 GGUF value types; `general.alignment` (a power of two, 32 if
// absent); tensors of 1-4 dims, each a type a file may hold (the table below), rows of whole blocks, aligned offsets,
// inside their file and overlapping no other; split models by llama.cpp's "-NNNNN-of-MMMMM" names, each shard's
// split.count / split.no checked; one name once across the model. The header is read front to back through a
// bounded cursor: a count is checked against the bytes left before anything is allocated for it, so a hostile file
// cannot make it allocate more than the file could hold.
#include <inttypes.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include <memory>

#include "osmos/model/gguf.h"

#define OSM_API __attribute__((visibility("default")))

namespace osm {
namespace gguf {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint32_t kVersion = 3;
constexpr uint64_t kAlign = 32;
constexpr uint32_t kMXFP8 = 43, kF8E4M3 = 0x12B;  // (the reference's own id for ggml's F8_E4M3: 0x100 | 43)

// the ggml types a file may hold: id, values a block, bytes a block (the reference's qtype.h:29-54 rows with
// QTYPE_FILE). F8_E4M3 has no id of a file's own (0x100 | 43): a file's 43 is read as it (see read_file)
struct TypeRow {
  uint32_t id, values, bytes;
};
constexpr TypeRow kTypes[] = {
    {0, 1, 4},       {2, 32, 18},    {7, 32, 24},    {8, 32, 34},    {12, 256, 144}, {13, 256, 176}, {10, 256, 84},
    {11, 256, 110},  {14, 256, 210}, {16, 256, 66},  {17, 256, 74},  {18, 256, 98},  {19, 256, 50},  {20, 32, 18},
    {22, 256, 82},   {23, 256, 136}, {26, 1, 4},     {27, 1, 8},     {29, 256, 56},  {30, 1, 2},     {39, 32, 17},
    {40, 64, 36},    {42, 64, 18},   {kMXFP8, 32, 33}, {kF8E4M3, 1, 1},
};

const TypeRow* type_row(uint32_t id) {
  for (const TypeRow& t : kTypes)
    if (t.id == id) return &t;
  return nullptr;
}

uint64_t bytes_of(uint32_t type, uint64_t values) {
  const TypeRow* t = type_row(type);
  if (!t || values % t->values) return 0;
  const uint64_t blocks = values / t->values;
  return blocks > UINT64_MAX / t->bytes ? 0 : blocks * t->bytes;
}

uint64_t width_of(uint32_t t) {  // a scalar value type's bytes (0: not a scalar)
  switch (t) {
    case GGUF_UINT8: case GGUF_INT8: case GGUF_BOOL: return 1;
    case GGUF_UINT16: case GGUF_INT16: return 2;
    case GGUF_UINT32: case GGUF_INT32: case GGUF_FLOAT32: return 4;
    case GGUF_UINT64: case GGUF_INT64: case GGUF_FLOAT64: return 8;
    default: return 0;
  }
}

bool is_signed(uint32_t t) { return t == GGUF_INT8 || t == GGUF_INT16 || t == GGUF_INT32 || t == GGUF_INT64; }

void kv_free(GgufKv& kv) {
  free(kv.key);
  if (kv.type == GGUF_STRING) {
    free(kv.v.s);
  } else if (kv.type == GGUF_ARRAY) {
    if (kv.item == GGUF_STRING && kv.v.items)
      for (uint64_t i = 0; i < kv.n; i++) free(((char**) kv.v.items)[i]);
    free(kv.v.items);
  }
  memset(&kv, 0, sizeof kv);
}

// a file's header read front to back; every read bounded by the file's size; the first failure's message kept
class Cursor {
 public:
  Cursor(const char* path, char* err) : path_(path), err_(err) {}
  ~Cursor() {
    if (f_) fclose(f_);
  }
  bool open(uint64_t* size) {
    struct stat st;
    if (stat(path_, &st) != 0 || !(f_ = fopen(path_, "rb"))) return fail("cannot open");
    size_ = (uint64_t) st.st_size;
    *size = size_;
    return true;
  }
  bool fail(const char* what) {
    if (err_ && !failed_) snprintf(err_, GGUF_ERR, "%s: offset %" PRIu64 ": %s", path_, pos_, what);
    failed_ = true;
    return false;
  }
  uint64_t left() const { return size_ - pos_; }
  uint64_t pos() const { return pos_; }
  void seek_note(uint64_t p) { pos_ = p; }  // (where a failure found after the header is reported)
  bool bytes(void* dst, uint64_t n) {
    if (n > left()) return fail("past the end of the file");
    if (n && fread(dst, 1, (size_t) n, f_) != n) return fail("read failed");
    pos_ += n;
    return true;
  }
  bool u32(uint32_t* v) { return bytes(v, 4); }
  bool u64(uint64_t* v) { return bytes(v, 8); }
  char* str() {  // a length-prefixed string, NUL terminated, malloc'd; NULL on failure
    uint64_t n = 0;
    if (!u64(&n)) return nullptr;
    if (n > left()) {
      fail("a string past the end of the file");
      return nullptr;
    }
    char* s = (char*) malloc((size_t) n + 1);
    if (!s) {
      fail("out of memory");
      return nullptr;
    }
    if (!bytes(s, n)) {
      free(s);
      return nullptr;
    }
    s[n] = 0;
    return s;
  }
  // a value after its key (what it allocated stays in kv for kv_free, also on failure)
  bool value(GgufKv& kv) {
    uint32_t t = 0;
    if (!u32(&t)) return false;
    if (t > GGUF_FLOAT64) return fail("an unknown value type");  // (checked before it is stored as the enum)
    kv.type = (GgufValueType) t;
    if (t == GGUF_STRING) return (kv.v.s = str()) != nullptr;
    if (t != GGUF_ARRAY) return scalar(t, kv);
    uint32_t item = 0;
    uint64_t n = 0;
    if (!u32(&item) || !u64(&n)) return false;
    if (item > GGUF_FLOAT64) return fail("an array of an unknown value type");
    kv.item = (GgufValueType) item;
    if (item == GGUF_STRING) {
      if (n > left() / 8) return fail("an array longer than the file");  // (each string at least its length)
      char** s = (char**) calloc(n ? (size_t) n : 1, sizeof(char*));
      if (!s) return fail("out of memory");
      kv.v.items = s;
      for (uint64_t i = 0; i < n; i++) {
        if (!(s[i] = str())) return false;
        kv.n = i + 1;
      }
      kv.n = n;
      return true;
    }
    const uint64_t w = width_of(item);
    if (!w) return fail("an array of an unknown value type");
    if (n > left() / w) return fail("an array longer than the file");
    if (!(kv.v.items = malloc(n ? (size_t) (n * w) : 1))) return fail("out of memory");
    kv.n = n;
    return bytes(kv.v.items, n * w);
  }

 private:
  bool scalar(uint32_t t, GgufKv& kv) {
    const uint64_t w = width_of(t);
    if (!w) return fail("an unknown value type");
    uint8_t raw[8] = {0};
    if (!bytes(raw, w)) return false;
    switch (t) {
      case GGUF_INT8: kv.v.i = (int8_t) raw[0]; break;
      case GGUF_INT16: { int16_t x; memcpy(&x, raw, 2); kv.v.i = x; break; }
      case GGUF_INT32: { int32_t x; memcpy(&x, raw, 4); kv.v.i = x; break; }
      case GGUF_INT64: memcpy(&kv.v.i, raw, 8); break;
      case GGUF_FLOAT32: { float x; memcpy(&x, raw, 4); kv.v.f = x; break; }
      case GGUF_FLOAT64: memcpy(&kv.v.f, raw, 8); break;
      default: { uint64_t x = 0; memcpy(&x, raw, w); kv.v.u = x; break; }
    }
    return true;
  }
  const char* path_;
  char* err_;
  FILE* f_ = nullptr;
  uint64_t pos_ = 0, size_ = 0;
  bool failed_ = false;
};

void destroy(Gguf* g) {
  if (!g) return;
  for (size_t i = 0; i < g->n_kv; i++) kv_free(g->kv[i]);
  free(g->kv);
  for (size_t i = 0; i < g->n_tensors; i++) free(g->tensors[i].name);
  free(g->tensors);
  for (int i = 0; g->paths && i < g->n_files; i++) free(g->paths[i]);
  free(g->paths);
  free(g->sizes);
  free(g);
}
struct Destroy {
  void operator()(Gguf* g) const { destroy(g); }
};
using Owned = std::unique_ptr<Gguf, Destroy>;

struct Split {
  uint64_t count = 0, no = 0;
};

// one file's header into g: its metadata (kept for file 0 only) and its tensors (appended)
bool read_file(Gguf* g, int file, Cursor& c, Split* split) {
  uint32_t magic = 0, version = 0;
  uint64_t n_tensors = 0, n_kv = 0;
  if (!c.u32(&magic) || !c.u32(&version) || !c.u64(&n_tensors) || !c.u64(&n_kv)) return false;
  if (magic != kMagic) return c.fail("not a GGUF file");
  if (version != kVersion) return c.fail("not GGUF version 3");
  // (an entry is at least 12 bytes: key length and value type; a tensor at least 24)
  if (n_kv > c.left() / 12 || n_tensors > c.left() / 24) return c.fail("more entries than the file holds");
  uint64_t align = kAlign;
  GgufKv* kv = (GgufKv*) calloc(n_kv ? (size_t) n_kv : 1, sizeof(GgufKv));
  if (!kv) return c.fail("out of memory");
  size_t got = 0;
  bool ok = true;
  while (ok && got < n_kv) {
    GgufKv& k = kv[got++];
    ok = (k.key = c.str()) != nullptr && c.value(k);
    if (!ok) break;
    if (!strcmp(k.key, "general.alignment")) {
      align = k.type == GGUF_UINT32 ? k.v.u : 0;
    } else if (!strcmp(k.key, "split.count") || !strcmp(k.key, "split.no")) {
      if (k.type != GGUF_UINT16 && k.type != GGUF_UINT32 && k.type != GGUF_UINT64)
        ok = c.fail("split.count or split.no not an unsigned integer");
      else
        (!strcmp(k.key, "split.count") ? split->count : split->no) = k.v.u;
    }
  }
  if (ok && (align == 0 || (align & (align - 1)))) ok = c.fail("an alignment that is not a power of two");
  if (ok && file == 0) {
    g->kv = kv, g->n_kv = got;
    kv = nullptr;
  }
  for (size_t i = 0; kv && i < got; i++) kv_free(kv[i]);
  free(kv);
  if (!ok) return false;
  GgufTensor* ts = (GgufTensor*) realloc(g->tensors, (g->n_tensors + (size_t) n_tensors + 1) * sizeof(GgufTensor));
  if (!ts) return c.fail("out of memory");
  g->tensors = ts;
  const size_t first = g->n_tensors;
  for (uint64_t i = 0; i < n_tensors; i++) {
    GgufTensor& t = g->tensors[g->n_tensors];
    memset(&t, 0, sizeof t);
    if (!(t.name = c.str())) return false;
    g->n_tensors++;
    if (!c.u32(&t.n_dims)) return false;
    if (t.n_dims < 1 || t.n_dims > GGUF_MAX_DIMS) return c.fail("a tensor of more than 4 dims or none");
    uint64_t values = 1;
    for (uint32_t d = 0; d < t.n_dims; d++) {
      if (!c.u64(&t.dims[d])) return false;
      if (t.dims[d] == 0 || values > UINT64_MAX / t.dims[d]) return c.fail("a tensor's dims are 0 or overflow");
      values *= t.dims[d];
    }
    if (!c.u32(&t.type) || !c.u64(&t.offset)) return false;
    const TypeRow* row = type_row(t.type);
    if (!row || t.type >= 0x100) return c.fail("a tensor type this build does not know");
    if (t.dims[0] % row->values || !(t.bytes = bytes_of(t.type, values)))
      return c.fail("a tensor's rows are not whole blocks");
    if (t.offset % align) return c.fail("a tensor's offset is not aligned");
    t.file = file;
  }
  const uint64_t size = c.pos() + c.left(), data = (c.pos() + align - 1) / align * align;
  // a 43 read as MXFP8 (33 bytes a 32 values) that runs past its room (the next tensor's offset, else the file's end)
  // but fits it at a byte a value is ggml's F8_E4M3 (the reference reads it so: gguf.c:151-165)
  for (size_t i = first; i < g->n_tensors && data <= size; i++) {
    GgufTensor& t = g->tensors[i];
    if (t.type != kMXFP8) continue;
    uint64_t room = t.offset <= size - data ? size - data - t.offset : 0;
    for (size_t j = first; j < g->n_tensors; j++)
      if (g->tensors[j].offset > t.offset && g->tensors[j].offset - t.offset < room) room = g->tensors[j].offset - t.offset;
    const uint64_t f8 = bytes_of(kF8E4M3, t.bytes / 33 * 32);
    if (t.bytes > room && f8 && f8 <= room) t.type = kF8E4M3, t.bytes = f8;
  }
  for (size_t i = first; i < g->n_tensors; i++) {
    GgufTensor& t = g->tensors[i];
    if (t.offset > size || data > size - t.offset || t.bytes > size - data - t.offset) {
      c.seek_note(data);
      return c.fail("a tensor's bytes leave the file");
    }
    t.offset += data;
  }
  for (size_t i = first; i < g->n_tensors; i++)
    for (size_t j = i + 1; j < g->n_tensors; j++) {
      const GgufTensor &a = g->tensors[i], &b = g->tensors[j];
      if (a.offset < b.offset + b.bytes && b.offset < a.offset + a.bytes) return c.fail("two tensors' bytes overlap");
    }
  return true;
}

bool open_file(Gguf* g, int file, const char* path, char* err, Split* split) {
  Cursor c(path, err);
  return c.open(&g->sizes[file]) && read_file(g, file, c, split);
}

// shard `no` (1-based) of `count` beside `first` (which holds "-00001-of-<count, 5 digits>"); NULL if it does not
char* shard_path(const char* first, int no, int count) {
  char want[32], have[32];
  snprintf(want, sizeof want, "-00001-of-%05d", count);
  snprintf(have, sizeof have, "-%05d-of-%05d", no, count);
  const char* at = strstr(first, want);
  if (!at || strlen(have) != strlen(want)) return nullptr;
  char* p = strdup(first);
  if (p) memcpy(p + (at - first), have, strlen(have));
  return p;
}

void fail_at(const char* path, char* err, const char* what) {
  if (err) snprintf(err, GGUF_ERR, "%s: offset 0: %s", path, what);
}

Gguf* create(const char* path, bool siblings, char* err) {
  if (err) err[0] = 0;
  if (!path) {
    fail_at("(null)", err, "cannot open");
    return nullptr;
  }
  Owned g((Gguf*) calloc(1, sizeof(Gguf)));
  if (!g) return nullptr;
  g->paths = (char**) calloc(1, sizeof(char*));
  g->sizes = (uint64_t*) calloc(1, sizeof(uint64_t));
  if (!g->paths || !g->sizes || !(g->paths[0] = strdup(path))) return nullptr;
  g->n_files = 1;
  Split split;
  if (!open_file(g.get(), 0, path, err, &split)) return nullptr;
  if (split.count > 1 && siblings) {
    if (split.no != 0 || split.count > 999 || !strstr(path, "-00001-of-")) {
      fail_at(path, err, "a split model is opened by its first shard (-00001-of-)");
      return nullptr;
    }
    const int count = (int) split.count;
    char** paths = (char**) realloc(g->paths, (size_t) count * sizeof(char*));
    if (paths) g->paths = paths;
    uint64_t* sizes = paths ? (uint64_t*) realloc(g->sizes, (size_t) count * sizeof(uint64_t)) : nullptr;
    if (sizes) g->sizes = sizes;
    if (!paths || !sizes) return nullptr;
    for (int i = 1; i < count; i++) {
      if (!(g->paths[i] = shard_path(path, i + 1, count))) {
        if (err) snprintf(err, GGUF_ERR, "%s: a split model's first shard is named -00001-of-%05d", path, count);
        return nullptr;
      }
      g->n_files = i + 1;
      Split s;
      if (!open_file(g.get(), i, g->paths[i], err, &s)) return nullptr;
      if (s.count != split.count || s.no != (uint64_t) i) {
        fail_at(g->paths[i], err, "a shard of another split");
        return nullptr;
      }
    }
  }
  for (size_t i = 0; i < g->n_tensors; i++)
    for (size_t j = i + 1; j < g->n_tensors; j++)
      if (!strcmp(g->tensors[i].name, g->tensors[j].name)) {
        fail_at(g->paths[g->tensors[j].file], err, "a tensor name twice");
        return nullptr;
      }
  return g.release();
}

}  // namespace gguf
}  // namespace osm

using namespace osm;

extern "C" OSM_API Gguf* gguf_create(const char* path, char err[GGUF_ERR]) { return gguf::create(path, true, err); }

extern "C" OSM_API Gguf* gguf_header(const char* path, char err[GGUF_ERR]) { return gguf::create(path, false, err); }

extern "C" OSM_API void gguf_destroy(Gguf* g) { gguf::destroy(g); }

extern "C" OSM_API const GgufTensor* gguf_tensor(const Gguf* g, const char* name) {
  for (size_t i = 0; g && name && i < g->n_tensors; i++)
    if (!strcmp(g->tensors[i].name, name)) return &g->tensors[i];
  return nullptr;
}

extern "C" OSM_API const GgufKv* gguf_kv(const Gguf* g, const char* key) {
  for (size_t i = 0; g && key && i < g->n_kv; i++)
    if (!strcmp(g->kv[i].key, key)) return &g->kv[i];
  return nullptr;
}

extern "C" OSM_API uint64_t gguf_bytes(uint32_t type, uint64_t values) { return gguf::bytes_of(type, values); }

extern "C" OSM_API bool gguf_int(const GgufKv* kv, size_t i, int64_t* out) {
  if (!kv || !out) return false;
  if (kv->type != GGUF_ARRAY) {
    if (gguf::is_signed(kv->type)) {
      *out = kv->v.i;
      return true;
    }
    if (!gguf::width_of(kv->type) || kv->type == GGUF_FLOAT32 || kv->type == GGUF_FLOAT64 || kv->v.u > INT64_MAX)
      return false;
    *out = (int64_t) kv->v.u;
    return true;
  }
  if (i >= kv->n) return false;
  const void* p = kv->v.items;
  switch (kv->item) {
    case GGUF_UINT8: *out = ((const uint8_t*) p)[i]; return true;
    case GGUF_INT8: *out = ((const int8_t*) p)[i]; return true;
    case GGUF_UINT16: *out = ((const uint16_t*) p)[i]; return true;
    case GGUF_INT16: *out = ((const int16_t*) p)[i]; return true;
    case GGUF_UINT32: *out = ((const uint32_t*) p)[i]; return true;
    case GGUF_INT32: *out = ((const int32_t*) p)[i]; return true;
    case GGUF_INT64: *out = ((const int64_t*) p)[i]; return true;
    case GGUF_UINT64:
      if (((const uint64_t*) p)[i] > INT64_MAX) return false;
      *out = (int64_t) ((const uint64_t*) p)[i];
      return true;
    default: return false;
  }
}
