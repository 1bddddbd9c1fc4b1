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
// the pool (described where it is defined, below): a job cut into per-worker slices at submit, the phases joined by a
// counting latch. any split of the rows gives the same bits: each row's sums are its own.
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

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

// rows r0 .. r1 of a matrix (cols) against cnt rows of codes q / scales d: y[t ys + r]; false (nothing written) for
// a type that is not the lane's or cols not whole 256-value blocks
bool lane_rows(uint32_t type, const void* w, uint32_t cols, uint32_t r0, uint32_t r1, const int8_t* q, const float* d,
               uint32_t cnt, float* y, uint32_t ys) {
  if (!lane_type(type) || !cols || cols % 256 || r1 < r0) return false;
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
  return true;
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

// ---- the pool ----
//
// A job is cut into work before any worker sees it: cpu_lane_submit lays each phase's rows out as per-worker slices
// (the x rows and the activation rows as contiguous row ranges; the gate/up rows and the down rows as runs of
// (expert, first row, last row) over the experts' matrices laid end to end, balanced to within one row). The workers
// then only run their own slices. Between phases they meet at a counting latch: one atomic counts every worker's
// finished phases in this job, and phase p is over for everyone once it reaches (p + 1) * workers; the worker whose
// increment ends the last phase posts the job's value. Between jobs the workers sleep on a condition variable keyed
// by a job serial, which also orders the plan's writes before their reads.
namespace {

struct Slice {
  uint32_t e, r0, r1;  // rows r0 .. r1 of the job's expert e
};
struct WorkerPlan {
  uint32_t x0 = 0, x1 = 0;  // x rows to round (and, with ff, the activation rows to round)
  std::vector<Slice> gu, dn;
};

constexpr uint32_t kPhases = 4;  // x rounded; gate, up, SwiGLU; activations rounded; down

}  // namespace

struct CpuLane {
  uint32_t max_rows = 0, dim = 0, ff = 0;
  std::vector<int8_t> xq, hq;   // the job's x rows, then its activations, as int8 codes
  std::vector<float> xs, hs;    // their 32-value blocks' scales
  std::vector<float> gate, up, act;
  std::vector<std::thread> workers;
  std::vector<WorkerPlan> plan;
  CpuLaneJob job{};
  std::mutex mu;
  std::condition_variable start, done;
  uint64_t issued = 0, finished = 0;  // jobs (mu's)
  bool stopping = false, clean = true;  // (mu's) clean: no job failed since the last wait
  std::atomic<uint32_t> latch{0};
  std::atomic<bool> bad{false};
};

namespace {

// `total` rows of `rows`-row matrices laid end to end, cut into `n` runs of near-equal length: run w into plan[w]
void cut_rows(uint32_t n_e, uint32_t rows, std::vector<WorkerPlan>& plan, std::vector<Slice> WorkerPlan::*list) {
  const uint64_t total = (uint64_t) n_e * rows, n = plan.size();
  uint32_t e = 0, r = 0;
  for (uint64_t w = 0; w < n; w++) {
    std::vector<Slice>& out = plan[w].*list;
    out.clear();
    for (uint64_t want = total / n + (w < total % n ? 1 : 0); want;) {
      const uint32_t take = (uint32_t) std::min<uint64_t>(want, rows - r);
      out.push_back({e, r, r + take});
      want -= take, r += take;
      if (r == rows) e++, r = 0;
    }
  }
}

bool job_ok(const CpuLane* c, const CpuLaneJob* j) {
  if (!j->x || !j->scale || !j->e || !j->y || !j->seq || !j->n_e || !j->n_rows) return false;
  if (!cpu::lane_type(j->type_gu) || !cpu::lane_type(j->type_down)) return false;
  if (j->dim != c->dim || j->ff != c->ff || j->n_rows > c->max_rows) return false;
  for (const CpuLaneExpert* x = j->e; x != j->e + j->n_e; x++)
    if (!x->gate || !x->up || !x->down || !x->cnt || (uint64_t) x->row0 + x->cnt > j->n_rows) return false;
  return true;
}

// every worker has finished `phases` phases of this job
void meet(CpuLane* c, uint32_t phases) {
  const uint32_t goal = phases * (uint32_t) c->workers.size();
  c->latch.fetch_add(1, std::memory_order_acq_rel);
  while (c->latch.load(std::memory_order_acquire) < goal) {
#if defined(__x86_64__)
    __builtin_ia32_pause();
#endif
  }
}

void run_plan(CpuLane* c, const WorkerPlan& p) {
  const CpuLaneJob& j = c->job;
  const uint32_t D = j.dim, F = j.ff;
  bool ok = true;
  cpu::round_rows(j.x + (uint64_t) p.x0 * D, p.x1 - p.x0, D, c->xq.data() + (uint64_t) p.x0 * D,
                  c->xs.data() + (uint64_t) p.x0 * (D / 32));
  meet(c, 1);
  for (const Slice& s : p.gu) {
    const CpuLaneExpert& e = j.e[s.e];
    const uint64_t xo = (uint64_t) e.row0 * D, ho = (uint64_t) e.row0 * F;
    ok &= cpu::lane_rows(j.type_gu, e.gate, D, s.r0, s.r1, c->xq.data() + xo, c->xs.data() + xo / 32, e.cnt,
                         c->gate.data() + ho, F);
    ok &= cpu::lane_rows(j.type_gu, e.up, D, s.r0, s.r1, c->xq.data() + xo, c->xs.data() + xo / 32, e.cnt,
                         c->up.data() + ho, F);
    for (uint32_t t = 0; t < e.cnt; t++) {
      const float w = j.scale[e.row0 + t];
      for (uint64_t i = ho + (uint64_t) t * F + s.r0; i < ho + (uint64_t) t * F + s.r1; i++)
        c->act[i] = cpu::lane_swiglu(c->gate[i], c->up[i], j.lim, w);
    }
  }
  meet(c, 2);
  cpu::round_rows(c->act.data() + (uint64_t) p.x0 * F, p.x1 - p.x0, F, c->hq.data() + (uint64_t) p.x0 * F,
                  c->hs.data() + (uint64_t) p.x0 * (F / 32));
  meet(c, 3);
  for (const Slice& s : p.dn) {
    const CpuLaneExpert& e = j.e[s.e];
    const uint64_t ho = (uint64_t) e.row0 * F;
    ok &= cpu::lane_rows(j.type_down, e.down, F, s.r0, s.r1, c->hq.data() + ho, c->hs.data() + ho / 32, e.cnt,
                         j.y + (uint64_t) e.row0 * D, D);
  }
  if (!ok) c->bad.store(true, std::memory_order_relaxed);
}

void finish_job(CpuLane* c) {
  const bool failed = c->bad.load(std::memory_order_relaxed);
  __atomic_store_n(c->job.seq, c->job.value | (failed ? CPU_LANE_FAILED : 0u), __ATOMIC_RELEASE);
  std::lock_guard<std::mutex> lk(c->mu);
  c->clean = c->clean && !failed;
  c->finished++;
  c->done.notify_all();
}

void worker_main(CpuLane* c, size_t id) {
  for (uint64_t next = 1;; next++) {
    {
      std::unique_lock<std::mutex> lk(c->mu);
      c->start.wait(lk, [&] { return c->stopping || c->issued >= next; });
      if (c->stopping) return;
    }
    run_plan(c, c->plan[id]);
    const uint32_t all = kPhases * (uint32_t) c->workers.size();
    if (c->latch.fetch_add(1, std::memory_order_acq_rel) + 1 == all) finish_job(c);
  }
}

// the calling thread onto CPU `core` (before it runs anything else)
bool pin_self(int core) {
  if (core < 0 || core >= CPU_SETSIZE) return false;
  cpu_set_t set;
  CPU_ZERO(&set);
  CPU_SET(core, &set);
  return sched_setaffinity(0, sizeof set, &set) == 0;
}

}  // namespace

extern "C" OSM_API CpuLane* cpu_lane_create(int threads, const int* cores, uint32_t max_rows, uint32_t dim, uint32_t ff) {
  if (threads < 1 || threads > CPU_LANE_THREADS_MAX || !max_rows || !dim || dim % 256 || !ff || ff % 256) return nullptr;
  CpuLane* c = nullptr;
  // each worker pins itself first and reports; create returns only once all have (or one could not)
  std::mutex m;
  std::condition_variable cv;
  int reported = 0;
  bool pinned = true;
  try {
    c = new CpuLane;
    c->max_rows = max_rows, c->dim = dim, c->ff = ff;
    const uint64_t rd = (uint64_t) max_rows * dim, rf = (uint64_t) max_rows * ff;
    c->xq.resize(rd), c->hq.resize(rf), c->xs.resize(rd / 32), c->hs.resize(rf / 32);
    c->gate.resize(rf), c->up.resize(rf), c->act.resize(rf);
    c->plan.resize((size_t) threads);
    c->workers.reserve((size_t) threads);
    for (int i = 0; i < threads; i++)
      c->workers.emplace_back([c, i, cores, &m, &cv, &reported, &pinned] {
        const bool ok = !cores || pin_self(cores[i]);
        {
          std::lock_guard<std::mutex> lk(m);
          pinned = pinned && ok, reported++;
          cv.notify_all();
        }
        worker_main(c, (size_t) i);
      });
    std::unique_lock<std::mutex> lk(m);
    cv.wait(lk, [&] { return reported == threads; });
    if (!pinned) {
      lk.unlock();
      cpu_lane_destroy(c);
      return nullptr;
    }
    return c;
  } catch (...) {  // memory or a thread refused: the workers already started are joined
    if (c) {
      std::unique_lock<std::mutex> lk(m);
      cv.wait(lk, [&] { return reported == (int) c->workers.size(); });
      lk.unlock();
      cpu_lane_destroy(c);
    }
    return nullptr;
  }
}

extern "C" OSM_API void cpu_lane_destroy(CpuLane* c) {
  if (!c) return;
  cpu_lane_wait(c);
  {
    std::lock_guard<std::mutex> lk(c->mu);
    c->stopping = true;
    c->start.notify_all();
  }
  for (std::thread& t : c->workers) t.join();
  delete c;
}

extern "C" OSM_API bool cpu_lane_submit(CpuLane* c, const CpuLaneJob* job) {
  if (!c || !job || !job_ok(c, job)) return false;
  std::lock_guard<std::mutex> lk(c->mu);
  if (c->finished != c->issued) return false;  // a job under way
  try {
    const uint64_t n = c->plan.size();
    for (uint64_t w = 0; w < n; w++)
      c->plan[w].x0 = (uint32_t) (job->n_rows * w / n), c->plan[w].x1 = (uint32_t) (job->n_rows * (w + 1) / n);
    cut_rows(job->n_e, job->ff, c->plan, &WorkerPlan::gu);
    cut_rows(job->n_e, job->dim, c->plan, &WorkerPlan::dn);
  } catch (...) {
    return false;
  }
  c->job = *job;
  c->latch.store(0, std::memory_order_relaxed);
  c->bad.store(false, std::memory_order_relaxed);
  c->issued++;
  c->start.notify_all();
  return true;
}

extern "C" OSM_API bool cpu_lane_wait(CpuLane* c) {
  if (!c) return false;
  std::unique_lock<std::mutex> lk(c->mu);
  c->done.wait(lk, [&] { return c->finished == c->issued; });
  const bool ok = c->clean;
  c->clean = true;
  return ok;
}
