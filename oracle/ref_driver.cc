// TEST INFRASTRUCTURE ONLY: C entry points over the reference's compiled CPU path (oracle/ref.mk), for the golden
// vectors (tests/golden/make_golden.py) and bench.py's CPU baseline. this file is this repository's; what it calls
// is the reference's src/cpu/q8.c (built as C++, so its functions have C++ linkage here) and src/cpu/expert.c (C).
#include <pthread.h>
#include <cmath>
#include <cstdint>

#include "lane.h"
#include "osmos/cpu/q8.h"
extern "C" {
#include "osmos/cpu/expert.h"
}

extern "C" {

bool ref_q8_ready(void) { return cpu_q8_ready(); }

// the reference's kernels/lane.h, compiled here as the CPU lane compiles it
float ref_lane_exp(float x) { return lane_exp(x); }
float ref_lane_swiglu(float g, float u, float lim, float scale) { return lane_swiglu(g, u, lim, scale); }

bool ref_q8_round(const float *x, uint32_t rows, uint32_t cols, uint32_t xs, int8_t *q, float *d)
{
  return cpu_q8_round(x, rows, cols, xs, q, d);
}

bool ref_q8_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const int8_t *q,
                 const float *d, uint32_t n, float *y, uint32_t ys)
{
  return cpu_q8_rows(type, w, cols, r0, r1, q, d, n, y, ys);
}

bool ref_mv_rows(uint32_t type, const void *w, uint32_t cols, uint32_t r0, uint32_t r1, const float *x, uint32_t xs,
                 uint32_t n, float *y, uint32_t ys)
{
  return cpu_mv_rows(type, w, cols, r0, r1, x, xs, n, y, ys);
}

// rows split evenly over `threads` threads (reference src/cpu/lane.c:53-57's share), each its own range
struct Share {
  uint32_t type, cols, r0, r1, n, ys;
  const void *w;
  const int8_t *q;
  const float *d;
  float *y;
  bool ok;
};

static void *share_run(void *p)
{
  Share *s = (Share *)p;
  s->ok = cpu_q8_rows(s->type, s->w, s->cols, s->r0, s->r1, s->q, s->d, s->n, s->y, s->ys);
  return nullptr;
}

bool ref_q8_rows_mt(uint32_t type, const void *w, uint32_t cols, uint32_t rows, const int8_t *q, const float *d,
                    uint32_t n, float *y, uint32_t ys, int threads)
{
  if (threads < 1 || threads > 256) return false;
  pthread_t th[256];
  Share sh[256];
  for (int i = 0; i < threads; i++) {
    sh[i] = Share{type, cols, (uint32_t)((uint64_t)rows * i / threads), (uint32_t)((uint64_t)rows * (i + 1) / threads),
                  n, ys, w, q, d, y, false};
    if (pthread_create(&th[i], nullptr, share_run, &sh[i])) return false;
  }
  bool ok = true;
  for (int i = 0; i < threads; i++) pthread_join(th[i], nullptr), ok = ok && sh[i].ok;
  return ok;
}

// one bs-n lane layer's experts on `threads` host threads (the CPU baseline): the reference's cpu_q8_rows over each
// phase's rows split evenly (src/cpu/lane.c:53-57's share, 98-118's phases: gate/up + lane_swiglu, the activations
// rounded, down), a barrier between phases. expert e's gate/up/down at g[e], u[e], dn[e], over rows r0[e] .. + cnt[e]
// of q / d (x rounded); y rows of dim. the threads are created once and run `reps` layers back to back.
struct Layer {
  uint32_t type, dim, ff, n_e, n_rows;
  const void *const *g, *const *u, *const *dn;
  const uint32_t *r0, *cnt;
  const int8_t *q;
  const float *d, *scale;
  float *gs, *us, *h, *hd, *y;
  int8_t *hq;
  int threads, reps;
  uint32_t copies;  // rep r reads weight copy r % copies: tables g, u, dn hold copies x n_e matrices
  pthread_barrier_t bar;
  bool ok;
};

struct Worker {
  Layer *L;
  int id;
};

static void span(uint64_t total, int id, int n, uint64_t *a, uint64_t *b)
{
  *a = total * (uint64_t)id / (uint64_t)n, *b = total * (uint64_t)(id + 1) / (uint64_t)n;
}

static void *layer_worker(void *p)
{
  Worker *w = (Worker *)p;
  Layer *L = w->L;
  const uint32_t D = L->dim, F = L->ff;
  for (int rep = 0; rep < L->reps; rep++) {
    const uint64_t cp = (uint64_t)(rep % L->copies) * L->n_e;
    const void *const *G = L->g + cp, *const *U = L->u + cp, *const *DN = L->dn + cp;
    uint64_t a, b;
    span((uint64_t)L->n_e * F, w->id, L->threads, &a, &b);  // gate / up rows of all experts end to end
    for (uint32_t e = 0; e < L->n_e; e++) {
      const uint64_t lo = (uint64_t)e * F, r0 = a > lo ? a - lo : 0, r1 = b < lo + F ? b - lo : F;
      if (r0 >= r1 || lo >= b) continue;
      const uint64_t row = L->r0[e];
      if (!cpu_q8_rows(L->type, G[e], D, (uint32_t)r0, (uint32_t)r1, L->q + row * D, L->d + row * (D / 32),
                       L->cnt[e], L->gs + row * F, F) ||
          !cpu_q8_rows(L->type, U[e], D, (uint32_t)r0, (uint32_t)r1, L->q + row * D, L->d + row * (D / 32),
                       L->cnt[e], L->us + row * F, F))
        L->ok = false;
      for (uint32_t t = 0; t < L->cnt[e]; t++)
        for (uint64_t r = r0; r < r1; r++) {
          const uint64_t i = (row + t) * F + r;
          L->h[i] = lane_swiglu(L->gs[i], L->us[i], INFINITY, L->scale[row + t]);
        }
    }
    pthread_barrier_wait(&L->bar);
    for (uint32_t r = (uint32_t)w->id; r < L->n_rows; r += (uint32_t)L->threads)
      if (!cpu_q8_round(L->h + (uint64_t)r * F, 1, F, F, L->hq + (uint64_t)r * F, L->hd + (uint64_t)r * (F / 32)))
        L->ok = false;
    pthread_barrier_wait(&L->bar);
    span((uint64_t)L->n_e * D, w->id, L->threads, &a, &b);
    for (uint32_t e = 0; e < L->n_e; e++) {
      const uint64_t lo = (uint64_t)e * D, r0 = a > lo ? a - lo : 0, r1 = b < lo + D ? b - lo : D;
      if (r0 >= r1 || lo >= b) continue;
      const uint64_t row = L->r0[e];
      if (!cpu_q8_rows(L->type, DN[e], F, (uint32_t)r0, (uint32_t)r1, L->hq + row * F, L->hd + row * (F / 32),
                       L->cnt[e], L->y + row * D, D))
        L->ok = false;
    }
    pthread_barrier_wait(&L->bar);
  }
  return nullptr;
}

// the layer `reps` times on `threads` threads, repetition r on weight copy r % copies (g, u and dn hold copies x n_e
// matrix addresses, copy after copy): with more copies than the host's last-level cache holds, every repetition reads
// its weights from DRAM, as a decode step does
bool ref_lane_layer_rot(uint32_t type, uint32_t dim, uint32_t ff, const void *const *g, const void *const *u,
                        const void *const *dn, const uint32_t *r0, const uint32_t *cnt, uint32_t n_e, uint32_t n_rows,
                        const int8_t *q, const float *d, const float *scale, float *y, int threads, int reps,
                        uint32_t copies)
{
  if (threads < 1 || threads > 256 || reps < 1 || copies < 1) return false;
  Layer L = {type, dim, ff, n_e, n_rows, g, u, dn, r0, cnt, q, d, scale, nullptr, nullptr, nullptr, nullptr, y,
             nullptr, threads, reps, copies, {}, true};
  L.gs = new float[(size_t)n_rows * ff], L.us = new float[(size_t)n_rows * ff], L.h = new float[(size_t)n_rows * ff];
  L.hd = new float[(size_t)n_rows * (ff / 32)], L.hq = new int8_t[(size_t)n_rows * ff];
  pthread_barrier_init(&L.bar, nullptr, (unsigned)threads);
  pthread_t th[256];
  Worker w[256];
  for (int i = 0; i < threads; i++) w[i] = Worker{&L, i}, pthread_create(&th[i], nullptr, layer_worker, &w[i]);
  for (int i = 0; i < threads; i++) pthread_join(th[i], nullptr);
  pthread_barrier_destroy(&L.bar);
  delete[] L.gs, delete[] L.us, delete[] L.h, delete[] L.hd, delete[] L.hq;
  return L.ok;
}

bool ref_lane_layer_mt(uint32_t type, uint32_t dim, uint32_t ff, const void *const *g, const void *const *u,
                       const void *const *dn, const uint32_t *r0, const uint32_t *cnt, uint32_t n_e, uint32_t n_rows,
                       const int8_t *q, const float *d, const float *scale, float *y, int threads, int reps)
{
  return ref_lane_layer_rot(type, dim, ff, g, u, dn, r0, cnt, n_e, n_rows, q, d, scale, y, threads, reps, 1);
}

}  // extern "C"
