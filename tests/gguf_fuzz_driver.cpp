// Test infrastructure: loads every file named on the command line with gguf_header and gguf_create (the reader of
// include/osmos/model/gguf.h) and walks every key, string, array item and tensor a loaded model holds. Built with
// the address and undefined-behaviour sanitizers by tests/test_gguf_fuzz.py, which feeds it mutated files: any
// out-of-bounds access, leak or undefined operation in the reader aborts the run.
#include <cstdio>
#include <cstring>
#include "osmos/model/gguf.h"
static unsigned long sink;
static void walk(const Gguf* g) {
  for (size_t i = 0; i < g->n_kv; i++) {
    const GgufKv& k = g->kv[i];
    sink += strlen(k.key);
    if (k.type == GGUF_STRING) sink += strlen(k.v.s);
    if (k.type == GGUF_ARRAY) {
      for (uint64_t j = 0; j < k.n; j++) {
        if (k.item == GGUF_STRING) sink += strlen(((char**) k.v.items)[j]);
        int64_t v; if (gguf_int(&k, j, &v)) sink += v;
      }
    }
    sink += gguf_kv(g, k.key) == &k;
  }
  for (size_t i = 0; i < g->n_tensors; i++) sink += strlen(g->tensors[i].name) + (gguf_tensor(g, g->tensors[i].name) != 0);
}
int main(int argc, char** argv) {
  int ok = 0;
  for (int i = 1; i < argc; i++) {
    char err[GGUF_ERR];
    Gguf* g = gguf_header(argv[i], err);
    if (g) { walk(g); gguf_destroy(g); ok++; }
    g = gguf_create(argv[i], err);
    if (g) { walk(g); gguf_destroy(g); }
  }
  printf("loaded %d of %d\n", ok, argc - 1);
  return 0;
}
