// libosmos MI355X - the lane's CPU half (include/osmos/cpu/lane.h): cpu_lane_create, cpu_lane_destroy, cpu_lane_submit,
// cpu_lane_wait. host code only.
//
// a job is one step's cold experts (reference src/cpu/lane.c:71-118, src/run/hip_lane.c:205-222): each of its rows
// (a (token, expert) pair) is computed exactly as the GPU's lane computes it - x rounded to int8 a 32-value block,
// gate and up as the lane's row sums, lane_swiglu with the row's weight, the activation rounded, down - so a row's
// output has the GPU's bits whichever side computes it, and the GPU takes the rows once the job's flag is posted
// (ops_wait, ops_copy_rows).
//
// the arithmetic (the lane contract, reference kernels/lane.h:43-75, kernels/q8.h:28-212): a weight block of 32 values
// becomes int8 codes from the GGUF layout; each 16-value half's exact integer dot with the int8 activations is scaled
// ((d * s21) / 8) * isum, each product rounded (the K-quants with a minimum subtract their min part); the halves added;
// the row's blocks s go to logical lane s % L (L = 32 from 4096 columns, else 16), fmaf'd onto the lane's sum in
// order; then the lanes' xor tree. compiled with -ffp-contract=off: every product and sum rounded on its own.
//
// the pool: workers asleep between jobs (a condition variable), within a job moving through its four phases together
// (a spinning barrier: a phase is tens of microseconds); each phase's rows split evenly over the workers - any split
// gives the same bits, each row's sums its own.
#include <pthread.h>
#include <sched.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <new>

#include "common.h"

extern "C" {
#include "../../include/osmos/cpu/lane.h"
}

namespace osm {
namespace cpu {

static const Grids kG = make_grids();

inline uint32_t u16at(const uint8_t* p) { return (uint32_t) p[0] | (uint32_t) p[1] << 8; }
inline uint32_t u32at(const uint8_t* p) { return u16at(p) | u16at(p + 2) << 16; }
inline float half_to_float(uint32_t h) {  // exact: normals, subnormals, infinities and NaNs
  const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  if (e == 31) {
    const uint32_t bits = sign | 0x7F800000u | m << 13;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
  }
  const float v = e ? std::ldexp((float) (1024 + m), (int) e - 25) : std::ldexp((float) m, -24);
  return sign ? -v : v;
}
inline uint32_t sign_field(uint32_t i) { return i | ((uint32_t) (__builtin_popcount(i) & 1) << 7); }

// ((d * s21) / 8) * isum, each product rounded
inline float part(float d, int s21, int isum) {
  float t = d * (float) s21;
  t = t * 0.125f;
  return t * (float) isum;
}

// a weight block's 32 codes, their dots with x's 32 int8 codes by 16-value half, x's sums by half
struct Dots {
  int c[32];
  int isum[2], xsum[2];
  void run(const int8_t* x) {
    for (int h = 0; h < 2; h++) {
      int s = 0, sx = 0;
      for (int i = 16 * h; i < 16 * h + 16; i++) s += c[i] * (int) x[i], sx += (int) x[i];
      isum[h] = s, xsum[h] = sx;
    }
  }
};
// 8 grid bytes into codes c[0 .. 8), negated where the sign bit says
inline void signed_bytes(uint64_t grid, uint32_t signs, int* c) {
  for (int i = 0; i < 8; i++) {
    const int v = (int) ((grid >> (8 * i)) & 0xFF);
    c[i] = (signs >> i) & 1 ? -v : v;
  }
}

// block s (32 values) of a row of `type` against x's codes: the contract's `sub`
float block_sub(uint32_t type, const uint8_t* row, uint32_t s, const int8_t* x) {
  Dots b;
  const uint32_t j = s % 8;  // (the 32-value block within a 256-value one)
  switch (type) {
    case kIQ2_XXS: {
      const uint8_t* blk = row + (s / 8) * 66;
      const uint8_t* g8 = blk + 2 + 8 * j;
      const uint32_t aux = u32at(g8 + 4);
      for (int k = 0; k < 4; k++) signed_bytes(kG.iq2xxs[g8[k]], sign_field((aux >> (7 * k)) & 127), b.c + 8 * k);
      b.run(x);
      const int s21 = 2 * (int) (aux >> 28) + 1;
      const float d = half_to_float(u16at(blk));
      return part(d, s21, b.isum[0]) + part(d, s21, b.isum[1]);
    }
    case kIQ2_XS: {
      const uint8_t* blk = row + (s / 8) * 74;
      for (int k = 0; k < 4; k++) {
        const uint32_t e = u16at(blk + 2 + 2 * (4 * j + k));
        signed_bytes(kG.iq2xs[e & 511], sign_field(e >> 9), b.c + 8 * k);
      }
      b.run(x);
      const uint32_t sc = blk[66 + j];
      const float d = half_to_float(u16at(blk));
      return part(d, 2 * (int) (sc & 15) + 1, b.isum[0]) + part(d, 2 * (int) (sc >> 4) + 1, b.isum[1]);
    }
    case kIQ2_S: {
      const uint8_t* blk = row + (s / 8) * 82;
      for (int k = 0; k < 4; k++) {
        const uint32_t idx = blk[2 + 4 * j + k] | ((blk[66 + j] >> (2 * k)) & 3u) << 8;
        signed_bytes(kG.iq2s[idx], blk[34 + 4 * j + k], b.c + 8 * k);
      }
      b.run(x);
      const uint32_t sc = blk[74 + j];
      const float d = half_to_float(u16at(blk));
      return part(d, 2 * (int) (sc & 15) + 1, b.isum[0]) + part(d, 2 * (int) (sc >> 4) + 1, b.isum[1]);
    }
    case kIQ3_XXS: {
      const uint8_t* blk = row + (s / 8) * 98;
      const uint8_t* q = blk + 2 + 8 * j;
      const uint32_t aux = u32at(blk + 66 + 4 * j);
      for (int k = 0; k < 4; k++) {
        const uint64_t g = (uint64_t) kG.iq3xxs[q[2 * k]] | (uint64_t) kG.iq3xxs[q[2 * k + 1]] << 32;
        signed_bytes(g, sign_field((aux >> (7 * k)) & 127), b.c + 8 * k);
      }
      b.run(x);
      const int s21 = 2 * (2 * (int) (aux >> 28) + 1);
      const float d = half_to_float(u16at(blk));
      return part(d, s21, b.isum[0]) + part(d, s21, b.isum[1]);
    }
    case kIQ1_S: {
      const uint8_t* blk = row + (s / 8) * 50;
      const uint32_t h = u16at(blk + 34 + 2 * j);
      const int delta = h & 0x8000u ? -1 : 1;
      for (int k = 0; k < 4; k++) {
        const uint64_t g = kG.iq1s[blk[2 + 4 * j + k] | ((h >> (3 * k)) & 7u) << 8];
        for (int i = 0; i < 8; i++) b.c[8 * k + i] = 8 * (int) (int8_t) (g >> (8 * i)) + delta;
      }
      b.run(x);
      const int s21 = 2 * (int) ((h >> 12) & 7u) + 1;
      const float d = half_to_float(u16at(blk));
      return part(d, s21, b.isum[0]) + part(d, s21, b.isum[1]);
    }
    case kIQ1_M: {
      const uint8_t* blk = row + (s / 8) * 56;
      for (int k = 0; k < 4; k++) {
        const uint32_t kk = 4 * j + k, hn = (blk[32 + kk / 2] >> (4 * (kk % 2))) & 15u;
        const uint64_t g = kG.iq1s[blk[kk] | (hn & 7u) << 8];
        const int delta = hn & 8u ? -1 : 1;
        for (int i = 0; i < 8; i++) b.c[8 * k + i] = 8 * (int) (int8_t) (g >> (8 * i)) + delta;
      }
      b.run(x);
      uint32_t dbits = 0;
      int s21[2];
      for (int i = 0; i < 4; i++) dbits |= (u16at(blk + 48 + 2 * i) >> 12) << (4 * i);
      for (int h = 0; h < 2; h++) {
        const uint32_t kk = 4 * j + 2 * h;  // (a 3-bit scale a 16 values: four to a u16)
        s21[h] = 2 * (int) ((u16at(blk + 48 + 2 * (kk / 8)) >> (3 * ((kk / 2) % 4))) & 7u) + 1;
      }
      const float d = half_to_float(dbits);
      return part(d, s21[0], b.isum[0]) + part(d, s21[1], b.isum[1]);
    }
    case kQ2_K: {
      const uint8_t* blk = row + (s / 8) * 84;
      const uint8_t* qs = blk + 16 + 32 * (j / 4);
      for (int i = 0; i < 32; i++) b.c[i] = (qs[i] >> (2 * (j % 4))) & 3;
      b.run(x);
      const float d = half_to_float(u16at(blk + 80)), dmin = half_to_float(u16at(blk + 82));
      float p[2];
      for (int h = 0; h < 2; h++) {
        const uint32_t sc = blk[2 * j + h];
        p[h] = part(d, 8 * (int) (sc & 15), b.isum[h]) - part(dmin, 8 * (int) (sc >> 4), b.xsum[h]);
      }
      return p[0] + p[1];
    }
    case kQ4_0: {  // (build-defined: codes q - 8 over the whole 32, one part with s21 8)
      const uint8_t* blk = row + s * 18;
      for (int i = 0; i < 16; i++) b.c[i] = (blk[2 + i] & 15) - 8, b.c[16 + i] = (blk[2 + i] >> 4) - 8;
      b.run(x);
      return part(half_to_float(u16at(blk)), 8, b.isum[0] + b.isum[1]);
    }
    case kQ4_K: {  // (build-defined: group j's 6-bit sc and m; (d 8 sc) / 8 isum - (dmin 8 m) / 8 xsum, the whole 32)
      const uint8_t* blk = row + (s / 8) * 144;
      const uint8_t* t = blk + 4;
      uint32_t sc, mn;
      if (j < 4) {
        sc = t[j] & 63u, mn = t[j + 4] & 63u;
      } else {
        sc = (t[j + 4] & 15u) | (t[j - 4] >> 6) << 4, mn = (t[j + 4] >> 4) | (t[j] >> 6) << 4;
      }
      const uint8_t* qs = blk + 16 + 32 * (j / 2);
      for (int i = 0; i < 32; i++) b.c[i] = (qs[i] >> (4 * (j % 2))) & 15;
      b.run(x);
      const float d = half_to_float(u16at(blk)), dmin = half_to_float(u16at(blk + 2));
      return part(d, 8 * (int) sc, b.isum[0] + b.isum[1]) - part(dmin, 8 * (int) mn, b.xsum[0] + b.xsum[1]);
    }
    case kQ3_K: {  // (build-defined: codes q2 + 4 hbit - 4; each half's 6-bit scale - 32, times 8)
      const uint8_t* blk = row + (s / 8) * 110;
      const uint32_t n = j / 4, r = j % 4;
      for (int i = 0; i < 32; i++)
        b.c[i] = (int) ((blk[32 + 32 * n + i] >> (2 * r)) & 3u) + 4 * (int) ((blk[i] >> (4 * n + r)) & 1u) - 4;
      b.run(x);
      const uint8_t* t = blk + 96;
      int s21[2];
      for (int h = 0; h < 2; h++) {
        const uint32_t g = 2 * j + h;  // the 16-value group
        const uint32_t lo = (t[g & 7] >> (4 * (g >> 3))) & 15u, hi = (t[8 + (g & 3)] >> (2 * (g >> 2))) & 3u;
        s21[h] = 8 * ((int) (lo | hi << 4) - 32);
      }
      const float d = half_to_float(u16at(blk + 108));
      return part(d, s21[0], b.isum[0]) + part(d, s21[1], b.isum[1]);
    }
    default: return NAN;
  }
}

bool lane_type(uint32_t t) {
  switch (t) {
    case kIQ2_XXS: case kIQ2_XS: case kIQ2_S: case kIQ3_XXS: case kIQ1_S: case kIQ1_M: case kQ2_K: case kQ4_0:
    case kQ4_K: case kQ3_K:
      return true;
    default:
      return false;
  }
}
uint32_t block_bytes(uint32_t t) {
  switch (t) {
    case kIQ2_XXS: return 66; case kIQ2_XS: return 74; case kIQ2_S: return 82; case kIQ3_XXS: return 98;
    case kIQ1_S: return 50; case kIQ1_M: return 56; case kQ2_K: return 84; case kQ4_0: return 18; case kQ4_K: return 144;
    case kQ3_K: return 110; default: return 0;
  }
}
uint32_t block_values(uint32_t t) { return t == kQ4_0 ? 32 : 256; }

// rows of x to int8 a 32-value block (q8_round's bits): amax; q = rint(x (127 / amax)); d = amax / 127
void round_rows(const float* x, uint32_t rows, uint32_t cols, int8_t* q, float* d) {
  for (uint64_t b = 0; b < (uint64_t) rows * cols / 32; b++) {
    const float* v = x + 32 * b;
    float am = 0.0f;
    for (int i = 0; i < 32; i++) am = std::fmax(am, std::fabs(v[i]));
    const float inv = am > 0.0f ? 127.0f / am : 0.0f;
    for (int i = 0; i < 32; i++) q[32 * b + i] = (int8_t) (int) std::rint(v[i] * inv);
    d[b] = am / 127.0f;
  }
}

// rows r0 .. r1 of a matrix (cols) against cnt rows of codes q / scales d: y[t ys + r]
void lane_rows(uint32_t type, const void* w, uint32_t cols, uint32_t r0, uint32_t r1, const int8_t* q, const float* d,
               uint32_t cnt, float* y, uint32_t ys) {
  const uint32_t nblk = cols / 32, L = cols >= 4096 ? 32 : 16;
  const uint64_t rb = (uint64_t) (cols / block_values(type)) * block_bytes(type);
  for (uint32_t r = r0; r < r1; r++) {
    const uint8_t* row = (const uint8_t*) w + r * rb;
    for (uint32_t t = 0; t < cnt; t++) {
      float acc[32] = {};
      for (uint32_t s = 0; s < nblk; s++)
        acc[s % L] = std::fma(d[(uint64_t) t * nblk + s], block_sub(type, row, s, q + (uint64_t) t * cols + 32 * s),
                              acc[s % L]);
      for (uint32_t o = L / 2; o > 0; o >>= 1) {  // (each level's pairs from the level before)
        float nx[32];
        for (uint32_t l = 0; l < L; l++) nx[l] = acc[l] + acc[l ^ o];
        std::memcpy(acc, nx, sizeof(float) * L);
      }
      y[(uint64_t) t * ys + r] = acc[0];
    }
  }
}

float lane_exp(float x) {
  if (x > 88.72283905f) return INFINITY;
  const float k = std::rint(x * 1.44269504089f);
  float r = std::fma(-k, 0.693145751953125f, x);
  r = std::fma(-k, 1.428606765330187e-06f, r);
  float p = 1.0f / 5040.0f;
  p = std::fma(p, r, 1.0f / 720.0f);
  p = std::fma(p, r, 1.0f / 120.0f);
  p = std::fma(p, r, 1.0f / 24.0f);
  p = std::fma(p, r, 1.0f / 6.0f);
  p = std::fma(p, r, 0.5f);
  p = std::fma(p, r, 1.0f);
  p = std::fma(p, r, 1.0f);
  return std::ldexp(p, (int) k);
}
float lane_swiglu(float g, float u, float lim, float scale) {
  const float gv = std::fmin(g, lim), uv = std::fmin(std::fmax(u, -lim), lim);
  const float den = 1.0f + lane_exp(-gv);
  const float sg = gv / den;
  const float h = sg * uv;
  return h * scale;
}

}  // namespace cpu
}  // namespace osm

using namespace osm;

struct CpuLane {
  int n = 0;
  pthread_t th[CPU_LANE_THREADS_MAX];
  uint32_t max_rows = 0, dim = 0, ff = 0;
  int8_t *q = nullptr, *qh = nullptr;  // x's rows, then the activations, as int8
  float *qd = nullptr, *qhd = nullptr;  // their blocks' scales
  float *g = nullptr, *u = nullptr, *h = nullptr;
  pthread_mutex_t mu;
  pthread_cond_t wake, idle;
  CpuLaneJob job{};
  uint64_t gen = 0;
  bool busy = false, quit = false, all_ok = true;  // (mu's)
  std::atomic<int> left{0}, arrived{0};
  std::atomic<bool> failed{false};
  std::atomic<unsigned> phase{0};
};

namespace {

struct WorkerArg {
  CpuLane* c;
  int id;
  int core;
};

void spin_barrier(CpuLane* c) {
  const unsigned ph = c->phase.load(std::memory_order_acquire);
  if (c->arrived.fetch_add(1, std::memory_order_acq_rel) + 1 == c->n) {
    c->arrived.store(0, std::memory_order_relaxed);
    c->phase.store(ph + 1, std::memory_order_release);
    return;
  }
  while (c->phase.load(std::memory_order_acquire) == ph) {
#if defined(__x86_64__)
    __builtin_ia32_pause();
#endif
  }
}

void share(int id, int n, uint64_t total, uint64_t* a, uint64_t* b) {
  *a = total * (uint64_t) id / (uint64_t) n, *b = total * (uint64_t) (id + 1) / (uint64_t) n;
}

// the experts' rows laid end to end (`rows` each): fn(expert, r0, r1) over rows a .. b of them
template <typename F>
void over_parts(const CpuLaneJob& j, uint32_t rows, uint64_t a, uint64_t b, F fn) {
  for (uint32_t k = (uint32_t) (a / rows); k < j.n_e && (uint64_t) k * rows < b; k++) {
    const uint64_t lo = (uint64_t) k * rows, r0 = a > lo ? a - lo : 0, r1 = b < lo + rows ? b - lo : rows;
    fn(j.e[k], (uint32_t) r0, (uint32_t) r1);
  }
}

void run_job(CpuLane* c, int id) {
  const CpuLaneJob& j = c->job;
  const uint32_t D = j.dim, F = j.ff;
  for (uint32_t r = (uint32_t) id; r < j.n_rows; r += (uint32_t) c->n)  // x's rows rounded
    cpu::round_rows(j.x + (uint64_t) r * D, 1, D, c->q + (uint64_t) r * D, c->qd + (uint64_t) r * (D / 32));
  spin_barrier(c);
  uint64_t a, b;
  share(id, c->n, (uint64_t) j.n_e * F, &a, &b);  // gate and up rows, the activation
  over_parts(j, F, a, b, [&](const CpuLaneExpert& e, uint32_t r0, uint32_t r1) {
    const int8_t* q = c->q + (uint64_t) e.row0 * D;
    const float* qd = c->qd + (uint64_t) e.row0 * (D / 32);
    float *g = c->g + (uint64_t) e.row0 * F, *u = c->u + (uint64_t) e.row0 * F, *h = c->h + (uint64_t) e.row0 * F;
    cpu::lane_rows(j.type_gu, e.gate, D, r0, r1, q, qd, e.cnt, g, F);
    cpu::lane_rows(j.type_gu, e.up, D, r0, r1, q, qd, e.cnt, u, F);
    for (uint32_t t = 0; t < e.cnt; t++)
      for (uint32_t r = r0; r < r1; r++) {
        const uint64_t i = (uint64_t) t * F + r;
        h[i] = cpu::lane_swiglu(g[i], u[i], j.lim, j.scale[e.row0 + t]);
      }
  });
  spin_barrier(c);
  for (uint32_t r = (uint32_t) id; r < j.n_rows; r += (uint32_t) c->n)  // the activations rounded
    cpu::round_rows(c->h + (uint64_t) r * F, 1, F, c->qh + (uint64_t) r * F, c->qhd + (uint64_t) r * (F / 32));
  spin_barrier(c);
  share(id, c->n, (uint64_t) j.n_e * D, &a, &b);  // down rows
  over_parts(j, D, a, b, [&](const CpuLaneExpert& e, uint32_t r0, uint32_t r1) {
    cpu::lane_rows(j.type_down, e.down, F, r0, r1, c->qh + (uint64_t) e.row0 * F, c->qhd + (uint64_t) e.row0 * (F / 32),
                   e.cnt, j.y + (uint64_t) e.row0 * D, D);
  });
}

void* worker(void* p) {
  WorkerArg arg = *(WorkerArg*) p;
  delete (WorkerArg*) p;
  CpuLane* c = arg.c;
  uint64_t seen = 0;
  for (;;) {
    pthread_mutex_lock(&c->mu);
    while (c->gen == seen && !c->quit) pthread_cond_wait(&c->wake, &c->mu);
    if (c->quit) {
      pthread_mutex_unlock(&c->mu);
      return nullptr;
    }
    seen = c->gen;
    pthread_mutex_unlock(&c->mu);
    run_job(c, arg.id);
    if (c->left.fetch_sub(1, std::memory_order_acq_rel) == 1) {  // the last one done: post, then the pool idle
      const bool failed = c->failed.load(std::memory_order_relaxed);
      __atomic_store_n(c->job.seq, c->job.value | (failed ? CPU_LANE_FAILED : 0u), __ATOMIC_RELEASE);
      pthread_mutex_lock(&c->mu);
      c->all_ok = c->all_ok && !failed, c->busy = false;
      pthread_cond_broadcast(&c->idle);
      pthread_mutex_unlock(&c->mu);
    }
  }
}

bool job_ok(const CpuLane* c, const CpuLaneJob* j) {
  if (!cpu::lane_type(j->type_gu) || !cpu::lane_type(j->type_down) || j->dim != c->dim || j->ff != c->ff || !j->x ||
      !j->scale || !j->e || !j->n_e || !j->y || !j->seq || !j->n_rows || j->n_rows > c->max_rows)
    return false;
  for (uint32_t k = 0; k < j->n_e; k++)
    if (!j->e[k].gate || !j->e[k].up || !j->e[k].down || !j->e[k].cnt || j->e[k].row0 + j->e[k].cnt > j->n_rows)
      return false;
  return true;
}

}  // namespace

extern "C" OSM_API CpuLane* cpu_lane_create(int threads, const int* cores, uint32_t max_rows, uint32_t dim, uint32_t ff) {
  if (threads < 1 || threads > CPU_LANE_THREADS_MAX || !max_rows || !dim || dim % 256 || !ff || ff % 256) return nullptr;
  CpuLane* c = new (std::nothrow) CpuLane;
  if (!c) return nullptr;
  c->max_rows = max_rows, c->dim = dim, c->ff = ff;
  const uint64_t rd = (uint64_t) max_rows * dim, rf = (uint64_t) max_rows * ff;
  c->q = (int8_t*) std::malloc(rd), c->qh = (int8_t*) std::malloc(rf);
  c->qd = (float*) std::malloc(rd / 32 * 4), c->qhd = (float*) std::malloc(rf / 32 * 4);
  c->g = (float*) std::malloc(rf * 4), c->u = (float*) std::malloc(rf * 4), c->h = (float*) std::malloc(rf * 4);
  pthread_mutex_init(&c->mu, nullptr), pthread_cond_init(&c->wake, nullptr), pthread_cond_init(&c->idle, nullptr);
  if (!c->q || !c->qh || !c->qd || !c->qhd || !c->g || !c->u || !c->h) {
    cpu_lane_destroy(c);
    return nullptr;
  }
  for (int i = 0; i < threads; i++) {
    pthread_attr_t at;
    if (pthread_attr_init(&at)) {
      cpu_lane_destroy(c);
      return nullptr;
    }
    bool ok = true;
    if (cores) {  // pinned from its first instruction: the attributes carry the CPU (one the kernel refuses: none)
      cpu_set_t set;
      CPU_ZERO(&set);
      ok = cores[i] >= 0 && cores[i] < CPU_SETSIZE;
      if (ok) CPU_SET(cores[i], &set);
      ok = ok && pthread_attr_setaffinity_np(&at, sizeof set, &set) == 0;
    }
    WorkerArg* a = ok ? new (std::nothrow) WorkerArg{c, i, cores ? cores[i] : -1} : nullptr;
    ok = a && pthread_create(&c->th[i], &at, worker, a) == 0;
    pthread_attr_destroy(&at);
    if (!ok) {
      delete a;
      cpu_lane_destroy(c);
      return nullptr;
    }
    c->n = i + 1;
  }
  return c;
}

extern "C" OSM_API void cpu_lane_destroy(CpuLane* c) {
  if (!c) return;
  cpu_lane_wait(c);
  pthread_mutex_lock(&c->mu);
  c->quit = true;
  pthread_cond_broadcast(&c->wake);
  pthread_mutex_unlock(&c->mu);
  for (int i = 0; i < c->n; i++) pthread_join(c->th[i], nullptr);
  pthread_mutex_destroy(&c->mu), pthread_cond_destroy(&c->wake), pthread_cond_destroy(&c->idle);
  std::free(c->q), std::free(c->qh), std::free(c->qd), std::free(c->qhd), std::free(c->g), std::free(c->u),
      std::free(c->h);
  delete c;
}

extern "C" OSM_API bool cpu_lane_submit(CpuLane* c, const CpuLaneJob* job) {
  if (!c || !job || !job_ok(c, job)) return false;
  pthread_mutex_lock(&c->mu);
  const bool free_ = !c->busy;
  if (free_) {
    c->job = *job, c->busy = true, c->gen++;
    c->failed.store(false, std::memory_order_relaxed);
    c->left.store(c->n, std::memory_order_release);
    pthread_cond_broadcast(&c->wake);
  }
  pthread_mutex_unlock(&c->mu);
  return free_;
}

extern "C" OSM_API bool cpu_lane_wait(CpuLane* c) {
  if (!c) return false;
  pthread_mutex_lock(&c->mu);
  while (c->busy) pthread_cond_wait(&c->idle, &c->mu);
  const bool ok = c->all_ok;
  c->all_ok = true;
  pthread_mutex_unlock(&c->mu);
  return ok;
}
