/* libosmos MI355X: GGUF model files as data - their metadata and their tensors' places (drop-in for the reference's
   include/osmos/model/gguf.h:1-75, src/model/gguf.c, src/model/gguf_read.c). Host code: nothing here touches the GPU.
   Only the headers are read; a tensor's bytes stay in its file at `offset`, for the caller to read or map in place
   (libosmos_amd/gguf.py puts expert slices on the device for the lane layer). The structs are the reference's layout,
   field for field, so a caller built against its header links against this library unchanged. */
#ifndef GGUF_H
#define GGUF_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGUF_ERR 256     /* the size of an error buffer: "<file>: offset <n>: <what>" */
#define GGUF_MAX_DIMS 4

typedef enum GgufValueType
{
  GGUF_UINT8 = 0,
  GGUF_INT8 = 1,
  GGUF_UINT16 = 2,
  GGUF_INT16 = 3,
  GGUF_UINT32 = 4,
  GGUF_INT32 = 5,
  GGUF_FLOAT32 = 6,
  GGUF_BOOL = 7,
  GGUF_STRING = 8,
  GGUF_ARRAY = 9,
  GGUF_UINT64 = 10,
  GGUF_INT64 = 11,
  GGUF_FLOAT64 = 12,
} GgufValueType;

/* one metadata entry: a scalar widened into v.u (unsigned, bool), v.i (signed) or v.f (float); a string in v.s (NUL
   terminated, owned); an array's element type in `item`, its length in `n`, its elements in v.items - `n` packed
   values of the element's own width, or for strings a char *[n] */
typedef struct GgufKv
{
  char *key;
  GgufValueType type;
  GgufValueType item;
  uint64_t n;
  union
  {
    uint64_t u;
    int64_t i;
    double f;
    char *s;
    void *items;
  } v;
} GgufKv;

/* one tensor: its ggml type id, dims innermost first, the file (shard) it is in, the absolute offset of its first
   byte in that file, and its size in bytes (whole blocks of its type) */
typedef struct GgufTensor
{
  char *name;
  uint32_t type;
  uint32_t n_dims;
  uint64_t dims[GGUF_MAX_DIMS];
  int file;
  uint64_t offset;
  uint64_t bytes;
} GgufTensor;

/* a model: its files (a split model's shards in order, each file's size), the first file's metadata, every file's
   tensors */
typedef struct Gguf
{
  int n_files;
  char **paths;
  uint64_t *sizes;
  GgufKv *kv;
  size_t n_kv;
  GgufTensor *tensors;
  size_t n_tensors;
} Gguf;

/* a model from `path` (a file, or a split model's "-00001-of-NNNNN" first shard, its siblings opened by name). the
   file is untrusted: every count, length and offset is checked against the file's size, and a model with a string
   or array past the end, an unknown value or tensor type, a tensor whose bytes leave its file or overlap another's,
   a misaligned tensor, a name twice, or a missing or foreign shard is refused - NULL, the reason in `err` (may be
   NULL), nothing left allocated. replaces reference gguf.h:68 (src/model/gguf.c:313-316) */
Gguf *gguf_create(const char *path, char err[GGUF_ERR]);
/* one file alone, as gguf_create reads it, a split model's shard without its siblings. replaces reference gguf.h:69
   (gguf.c:318-321) */
Gguf *gguf_header(const char *path, char err[GGUF_ERR]);
/* frees the model and all it owns; NULL is nothing to do. replaces reference gguf.h:70 (gguf.c:323-337) */
void gguf_destroy(Gguf *g);

/* by exact name; NULL when absent. pointers into the model, valid until gguf_destroy. replace reference gguf.h:72-73 */
const GgufTensor *gguf_tensor(const Gguf *g, const char *name);
const GgufKv *gguf_kv(const Gguf *g, const char *key);
/* the bytes `values` values of `type` take: 0 for a type no file may hold or a count that is not whole blocks.
   replaces reference gguf.h:74 (gguf.c:48-57) */
uint64_t gguf_bytes(uint32_t type, uint64_t values);
/* an integer entry at its own width: a scalar's value (i ignored) or an array's item i (i < n); false for another type
   or an unsigned 64-bit value above INT64_MAX. replaces reference gguf.h:75 (gguf.c:20-46) */
bool gguf_int(const GgufKv *kv, size_t i, int64_t *out);

#ifdef __cplusplus
}
#endif

#endif
