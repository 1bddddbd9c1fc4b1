// TEST INFRASTRUCTURE ONLY: C entry points over the reference's compiled CPU path (oracle/ref.mk), for the golden
// vectors (tests/golden/make_golden.py) and bench.py's CPU baseline. this file is this repository's; what it calls
// is the reference's src/cpu/q8.c (built as C++, so its functions have C++ linkage here) and src/cpu/expert.c (C).
#include <pthread.h>
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

}  // extern "C"
