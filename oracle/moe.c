/* TEST INFRASTRUCTURE ONLY (the CPU oracle; see oracle.h): the lane's layer, the token sums, the MoE plumbing and
   a threaded row split for the CPU baseline.

   reference: src/cpu/lane.c:71-118 (the layer's phases), src/run/hip_lane.c:164-177,220 and kernels/ops.hip:515-530
   (each token's expert rows summed in ascending expert id, then the shared part added), kernels/q4x_moe.hip:38-65
   (softmax top-k, the lowest id among equals, weights over max(sum, 6.103515625e-5)), kernels/q4x_moe.hip:172-180
   (the weighted sum with the sigmoid-gated shared expert). */
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

bool orc_lane_layer(uint32_t type_gu, uint32_t type_down, uint32_t dim, uint32_t ff, float lim, const float *x,
                    const float *scale, uint32_t n_rows, const void *const *gate, const void *const *up,
                    const void *const *down, const uint32_t *row0, const uint32_t *cnt, uint32_t n_e, float *y)
{
  const uint32_t D = dim, F = ff;
  int8_t *q = malloc((size_t)n_rows * D), *qh = malloc((size_t)n_rows * F);
  float *qd = malloc((size_t)n_rows * (D / 32) * 4), *qhd = malloc((size_t)n_rows * (F / 32) * 4);
  float *g = malloc((size_t)n_rows * F * 4), *u = malloc((size_t)n_rows * F * 4), *h = malloc((size_t)n_rows * F * 4);
  bool ok = q && qh && qd && qhd && g && u && h && orc_q8_round(x, n_rows, D, D, q, qd);
  for (uint32_t e = 0; ok && e < n_e; e++)
  {
    const uint64_t r0 = row0[e];
    ok = orc_q8_rows(type_gu, gate[e], D, 0, F, q + r0 * D, qd + r0 * (D / 32), cnt[e], g + r0 * F, F) &&
         orc_q8_rows(type_gu, up[e], D, 0, F, q + r0 * D, qd + r0 * (D / 32), cnt[e], u + r0 * F, F);
    for (uint32_t t = 0; ok && t < cnt[e]; t++)
      for (uint32_t r = 0; r < F; r++)
      {
        const uint64_t i = (r0 + t) * F + r;
        h[i] = orc_lane_swiglu(g[i], u[i], lim, scale[r0 + t]);
      }
  }
  ok = ok && orc_q8_round(h, n_rows, F, F, qh, qhd);
  for (uint32_t e = 0; ok && e < n_e; e++)
  {
    const uint64_t r0 = row0[e];
    ok = orc_q8_rows(type_down, down[e], F, 0, D, qh + r0 * F, qhd + r0 * (F / 32), cnt[e], y + r0 * D, D);
  }
  free(q), free(qh), free(qd), free(qhd), free(g), free(u), free(h);
  return ok;
}

void orc_gather_sum_add(float *y, const float *src, const int32_t *idx, uint32_t m, uint32_t n, uint32_t dim,
                        const float *add)
{
  for (uint32_t t = 0; t < n; t++)
    for (uint32_t d = 0; d < dim; d++)
    {
      float s = 0.0f;
      for (uint32_t j = 0; j < m; j++)
        s += src[(uint64_t)idx[t * m + j] * dim + d];
      y[(uint64_t)t * dim + d] = add ? s + add[(uint64_t)t * dim + d] : s;
    }
}

void orc_route(const float *logits, uint32_t n_tok, uint32_t n_exp, uint32_t k, int32_t *ids, float *w)
{
  float *p = malloc((size_t)n_exp * sizeof *p);
  char *taken = malloc(n_exp);
  for (uint32_t t = 0; t < n_tok; t++)
  {
    const float *l = logits + (uint64_t)t * n_exp;
    float m = -INFINITY, sum = 0.0f;
    for (uint32_t i = 0; i < n_exp; i++)
      m = fmaxf(m, l[i]);
    for (uint32_t i = 0; i < n_exp; i++)
      sum += (p[i] = expf(l[i] - m));
    const float inv = 1.0f / sum;
    for (uint32_t i = 0; i < n_exp; i++)
      p[i] *= inv, taken[i] = 0;
    float pick[64], total = 0.0f;
    for (uint32_t j = 0; j < k; j++)
    {
      int bi = -1;
      for (uint32_t i = 0; i < n_exp; i++) /* ascending ids, a strict > keeps the lowest among equals */
        if (!taken[i] && (bi < 0 || (p[i] == p[i] ? p[i] : -INFINITY) > p[bi]))
          bi = (int)i;
      taken[bi] = 1, pick[j] = p[bi], total += p[bi], ids[t * k + j] = bi;
    }
    const float div = fmaxf(total, 6.103515625e-5f);
    for (uint32_t j = 0; j < k; j++)
      w[t * k + j] = pick[j] / div;
  }
  free(p), free(taken);
}

void orc_moe_sum(const float *y, const int32_t *where, const float *w, uint32_t n_tok, uint32_t k, uint32_t dim,
                 const float *shared, const float *shared_logit, float *out)
{
  for (uint32_t t = 0; t < n_tok; t++)
  {
    const float gsh = 1.0f / (1.0f + expf(-shared_logit[t]));
    for (uint32_t d = 0; d < dim; d++)
    {
      float s = 0.0f;
      for (uint32_t j = 0; j < k; j++)
        s += y[(uint64_t)where[t * k + j] * dim + d] * w[t * k + j];
      out[(uint64_t)t * dim + d] = s + shared[(uint64_t)t * dim + d] * gsh;
    }
  }
}

typedef struct
{
  uint32_t type, cols, r0, r1, n, ys;
  const void *w;
  const int8_t *q;
  const float *d;
  float *y;
  bool ok;
} Share;

static void *share_run(void *p)
{
  Share *s = p;
  s->ok = orc_q8_rows(s->type, s->w, s->cols, s->r0, s->r1, s->q, s->d, s->n, s->y, s->ys);
  return NULL;
}

bool orc_q8_rows_mt(uint32_t type, const void *w, uint32_t cols, uint32_t rows, const int8_t *q, const float *d,
                    uint32_t n, float *y, uint32_t ys, int threads)
{
  if (threads < 1 || threads > 256)
    return false;
  pthread_t th[256];
  Share sh[256];
  for (int i = 0; i < threads; i++)
  {
    sh[i] = (Share){type, cols, (uint32_t)((uint64_t)rows * i / threads), (uint32_t)((uint64_t)rows * (i + 1) / threads),
                    n, ys, w, q, d, y, false};
    if (pthread_create(&th[i], NULL, share_run, &sh[i]))
      return false;
  }
  bool ok = true;
  for (int i = 0; i < threads; i++)
    pthread_join(th[i], NULL), ok = ok && sh[i].ok;
  return ok;
}
