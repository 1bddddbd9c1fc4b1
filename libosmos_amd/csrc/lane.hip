// libosmos MI355X - the lane's int8 expert products (include/osmos/gpu/q8.h): q8_round, q8_group_tok, q8_gate_up.
//
// contract (reference kernels/lane.h:43-75, kernels/q8.h:133-212, include/osmos/gpu/q8.h:17-44): a row's 32-value
// blocks s go to logical lane s % L (L = 32 for cols >= 4096, else 16) in ascending order; per block each 16-value
// half's exact integer dot with the int8 activations (v_dot4_i32_i8), then ((d * s21) / 8) * isum per half, the halves
// added, fmaf'd with the block's activation scale onto the lane's sum; then the lanes' xor tree. the float steps and
// their order are the reference's, so each output's bits are the reference CPU path's.
//
// CDNA4 mapping: a wave64 holds 64 / L rows (4 at 16 lanes, 2 at 32), logical lane ll = lane % L of row lane / L -
// the tree's partners (ll ^ o, o < L) stay inside the row's aligned group of lanes. a workgroup is 4 waves.
#include "common.h"

extern "C" {
#include "../../include/osmos/gpu/mv.h"
#include "../../include/osmos/gpu/q8.h"
}

namespace osm {
namespace lane {

__constant__ Grids kGrids = make_grids();

constexpr int kWaves = 4;              // a workgroup's waves
constexpr int kThreads = kWave * kWaves;

// a 32-value block's int8 codes: 8 words (4 values each, value 4i + b in byte b of word i); per 8-value chunk k the
// IQ1 types' delta (+-1, codes 8 grid + delta) or 0; per 16-value half its scale integer s21 (Q2_K, Q4_K: 8 sc) and
// minimum m8 (8 m); the block scale d and minimum scale dmin. `bias`: a constant subtracted from every code (Q4_0's
// 8, Q3_K's 4), applied to the integer dot through x's sum - the same integer
struct Codes {
  int w[8];
  int delta[4];
  int s21[2];
  int m8[2];
  float d, dmin;
};

// 8 unsigned grid bytes, each negated where its sign bit is set: (v ^ m) + (m & 1) a byte, m = 0xFF where negative
__device__ inline void signed8(uint64_t grid, uint32_t signs, int& lo, int& hi) {
  uint32_t a = 0, b = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    a |= ((signs >> i) & 1u) * (0xFFu << (8 * i));
    b |= ((signs >> (4 + i)) & 1u) * (0xFFu << (8 * i));
  }
  lo = (int) (((uint32_t) grid ^ a) + (a & 0x01010101u));
  hi = (int) (((uint32_t) (grid >> 32) ^ b) + (b & 0x01010101u));
}

__device__ inline int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <uint32_t T> struct Traits {
  static constexpr bool iq1 = false, has_min = false, whole = false;
  static constexpr int bias = 0;  // subtracted from each code
};
template <> struct Traits<kIQ1_M> { static constexpr bool iq1 = true, has_min = false, whole = false; static constexpr int bias = 0; };
template <> struct Traits<kIQ1_S> { static constexpr bool iq1 = true, has_min = false, whole = false; static constexpr int bias = 0; };
template <> struct Traits<kQ2_K> { static constexpr bool iq1 = false, has_min = true, whole = false; static constexpr int bias = 0; };
template <> struct Traits<kQ4_0> { static constexpr bool iq1 = false, has_min = false, whole = true; static constexpr int bias = 8; };
template <> struct Traits<kQ4_K> { static constexpr bool iq1 = false, has_min = true, whole = true; static constexpr int bias = 0; };
template <> struct Traits<kQ3_K> { static constexpr bool iq1 = false, has_min = false, whole = false; static constexpr int bias = 4; };

template <uint32_t T> __device__ void codes(const uint8_t* b, int j, Codes& c);

// reference kernels/q8.h:46-55
template <> __device__ inline void codes<kIQ2_XXS>(const uint8_t* b, int j, Codes& c) {
  const uint8_t* q = b + 2 + 8 * j;
  const uint32_t aux = ld32(q + 4);
#pragma unroll
  for (int k = 0; k < 4; k++) signed8(kGrids.iq2xxs[q[k]], ksign((aux >> (7 * k)) & 0x7F), c.w[2 * k], c.w[2 * k + 1]);
  c.s21[0] = c.s21[1] = 2 * (int) (aux >> 28) + 1;
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:57-66
template <> __device__ inline void codes<kIQ2_XS>(const uint8_t* b, int j, Codes& c) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t q = ld16(b + 2 + 2 * (4 * j + k));
    signed8(kGrids.iq2xs[q & 511], ksign(q >> 9), c.w[2 * k], c.w[2 * k + 1]);
  }
  const uint32_t s = b[66 + j];
  c.s21[0] = 2 * (int) (s & 0x0F) + 1, c.s21[1] = 2 * (int) (s >> 4) + 1;
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:68-84
template <> __device__ inline void codes<kIQ1_M>(const uint8_t* b, int j, Codes& c) {
  const uint32_t sc0 = ld32(b + 48), sc1 = ld32(b + 52);
  const uint64_t sc = (uint64_t) sc0 | (uint64_t) sc1 << 32;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int kk = 4 * j + k;
    const uint32_t h = (b[32 + kk / 2] >> (4 * (kk % 2))) & 0x0F;
    const uint64_t g = kGrids.iq1s[b[kk] | (h & 0x07) << 8];
    c.w[2 * k] = (int) (uint32_t) g, c.w[2 * k + 1] = (int) (uint32_t) (g >> 32);
    c.delta[k] = h & 0x08 ? -1 : 1;
  }
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int kk = 4 * j + 2 * h;
    c.s21[h] = 2 * (int) ((sc >> (16 * (kk / 8) + 3 * ((kk / 2) % 4))) & 0x07) + 1;
  }
  const uint32_t s0 = sc0 & 0xFFFF, s1 = sc0 >> 16, s2 = sc1 & 0xFFFF, s3 = sc1 >> 16;
  c.d = f16((s0 >> 12) | ((s1 >> 8) & 0x00F0) | ((s2 >> 4) & 0x0F00) | (s3 & 0xF000));
}

// reference kernels/q8.h:86-95
template <> __device__ inline void codes<kIQ2_S>(const uint8_t* b, int j, Codes& c) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int kk = 4 * j + k;
    signed8(kGrids.iq2s[b[2 + kk] | ((b[66 + j] >> (2 * k)) & 0x03) << 8], b[34 + kk], c.w[2 * k], c.w[2 * k + 1]);
  }
  const uint32_t s = b[74 + j];
  c.s21[0] = 2 * (int) (s & 0x0F) + 1, c.s21[1] = 2 * (int) (s >> 4) + 1;
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:97-108
template <> __device__ inline void codes<kIQ3_XXS>(const uint8_t* b, int j, Codes& c) {
  const uint8_t* q = b + 2 + 8 * j;
  const uint32_t aux = ld32(b + 66 + 4 * j);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint64_t g = (uint64_t) kGrids.iq3xxs[q[2 * k]] | (uint64_t) kGrids.iq3xxs[q[2 * k + 1]] << 32;
    signed8(g, ksign((aux >> (7 * k)) & 0x7F), c.w[2 * k], c.w[2 * k + 1]);
  }
  c.s21[0] = c.s21[1] = 2 * (2 * (int) (aux >> 28) + 1);
  c.d = f16(ld16(b));
}

// reference kernels/q8.h:110-118
template <> __device__ inline void codes<kQ2_K>(const uint8_t* b, int j, Codes& c) {
  const uint8_t* qs = b + 16 + 32 * (j / 4);
  const int shift = 2 * (j % 4);
#pragma unroll
  for (int t = 0; t < 8; t++) c.w[t] = (int) ((ld32(qs + 4 * t) >> shift) & 0x03030303u);
#pragma unroll
  for (int h = 0; h < 2; h++) c.s21[h] = 8 * (b[2 * j + h] & 0x0F), c.m8[h] = 8 * (b[2 * j + h] >> 4);
  c.d = f16(ld16(b + 80)), c.dmin = f16(ld16(b + 82));
}

// reference kernels/q8.h:120-130
template <> __device__ inline void codes<kIQ1_S>(const uint8_t* b, int j, Codes& c) {
  const uint32_t h = ld16(b + 34 + 2 * j);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint64_t g = kGrids.iq1s[b[2 + 4 * j + k] | ((h >> (3 * k)) & 0x07) << 8];
    c.w[2 * k] = (int) (uint32_t) g, c.w[2 * k + 1] = (int) (uint32_t) (g >> 32);
    c.delta[k] = h & 0x8000 ? -1 : 1;
  }
  c.s21[0] = c.s21[1] = 2 * (int) ((h >> 12) & 0x07) + 1;
  c.d = f16(ld16(b));
}

// build-defined: ggml's Q4_0 (32 values: f16 d, 16 bytes of nibbles; value i < 16 byte i's low nibble, 16 + i its
// high), codes q - 8 (the 8 through `bias`), one part over the 32 with s21 8 - so d * isum exactly
template <> __device__ inline void codes<kQ4_0>(const uint8_t* b, int, Codes& c) {
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const uint32_t v = ld32(b + 2 + 4 * t);
    c.w[t] = (int) (v & 0x0F0F0F0Fu), c.w[4 + t] = (int) ((v >> 4) & 0x0F0F0F0Fu);
  }
  c.s21[0] = c.s21[1] = 8;
  c.d = f16(ld16(b));
}

// build-defined: Q4_K's group j (its 6-bit sc and m, reference kernels/quant.h:89-103's layout), codes q, one part
// with its minimum: ((d * 8 sc) / 8) * isum - ((dmin * 8 m) / 8) * xsum
template <> __device__ inline void codes<kQ4_K>(const uint8_t* b, int j, Codes& c) {
  const uint8_t* s = b + 4;
  const int sc = j < 4 ? s[j] & 0x3F : (s[j + 4] & 0x0F) | ((s[j - 4] >> 2) & 0x30);
  const int m = j < 4 ? s[j + 4] & 0x3F : (s[j + 4] >> 4) | ((s[j] >> 2) & 0x30);
  const uint8_t* qs = b + 16 + (j / 2) * 32;
  const int sh = 4 * (j % 2);
#pragma unroll
  for (int t = 0; t < 8; t++) c.w[t] = (int) ((ld32(qs + 4 * t) >> sh) & 0x0F0F0F0Fu);
  c.s21[0] = c.s21[1] = 8 * sc, c.m8[0] = c.m8[1] = 8 * m;
  c.d = f16(ld16(b)), c.dmin = f16(ld16(b + 2));
}

// build-defined: Q3_K's values 32 j .. 32 j + 31 (reference kernels/quant.h:264-284's layout): codes q2 + 4 h - 4
// (the 4 through `bias`), two halves, each s21 = 8 (sc - 32) of its 16-value group
template <> __device__ inline void codes<kQ3_K>(const uint8_t* b, int j, Codes& c) {
  const int n = j / 4, jj = j % 4;
  const uint8_t* qs = b + 32 + 32 * n;
#pragma unroll
  for (int t = 0; t < 8; t++) {
    const uint32_t q2 = (ld32(qs + 4 * t) >> (2 * jj)) & 0x03030303u;
    const uint32_t hb = (ld32(b + 4 * t) >> (4 * n + jj)) & 0x01010101u;
    c.w[t] = (int) (q2 + (hb << 2));
  }
  const uint8_t* sc = b + 96;
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int g = 2 * j + h, grp = g / 4, w = g % 4;
    const int low = ((grp & 1 ? sc[4 + w] : sc[w]) >> (grp & 2 ? 4 : 0)) & 0x0F;
    const int sc6 = low | ((sc[8 + w] >> (2 * grp)) & 0x03) << 4;
    c.s21[h] = 8 * (sc6 - 32);
  }
  c.d = f16(ld16(b + 108));
}

// the block's contribution before x's scale (reference kernels/q8.h:133-162)
template <uint32_t T>
__device__ inline float block_sum(const Codes& c, const int* x) {
  using Tr = Traits<T>;
  int isum[2], xsum[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    int s = 0, sx = 0;
#pragma unroll
    for (int k = 2 * h; k < 2 * h + 2; k++) {
      const int gx = dot4(c.w[2 * k + 1], x[2 * k + 1], dot4(c.w[2 * k], x[2 * k], 0));
      if constexpr (Tr::iq1 || Tr::has_min || Tr::bias) {
        const int xk = dot4(0x01010101, x[2 * k + 1], dot4(0x01010101, x[2 * k], 0));
        if constexpr (Tr::iq1) s += 8 * gx + c.delta[k] * xk;
        else s += gx - Tr::bias * xk;
        sx += xk;
      } else {
        s += gx;
      }
    }
    isum[h] = s, xsum[h] = sx;
  }
  if constexpr (Tr::whole) {
    const int is = isum[0] + isum[1];
    if constexpr (Tr::has_min)
      return __fsub_rn(lane_part(c.d, c.s21[0], is), lane_part(c.dmin, c.m8[0], xsum[0] + xsum[1]));
    else
      return lane_part(c.d, c.s21[0], is);
  } else if constexpr (Tr::has_min) {
    const float p0 = __fsub_rn(lane_part(c.d, c.s21[0], isum[0]), lane_part(c.dmin, c.m8[0], xsum[0]));
    const float p1 = __fsub_rn(lane_part(c.d, c.s21[1], isum[1]), lane_part(c.dmin, c.m8[1], xsum[1]));
    return __fadd_rn(p0, p1);
  } else {
    return __fadd_rn(lane_part(c.d, c.s21[0], isum[0]), lane_part(c.d, c.s21[1], isum[1]));
  }
}

// a launch's NT input rows for output rows r0 .. r0 + NT - 1 (reference kernels/q8.h:164-173): row r's own (xin
// NULL), else row xin[r]; the rows past the count read as the count's last - summed, never stored
template <int NT>
__device__ inline void in_rows(const int32_t* xin, uint32_t r0, uint32_t cnt, uint64_t* xr) {
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const uint32_t r = r0 + ((uint32_t) t < cnt ? (uint32_t) t : cnt - 1);
    xr[t] = xin ? (uint64_t) (uint32_t) xin[r] : r;
  }
}

__device__ inline void load_x(const int8_t* q, uint64_t at, int* x) {
  const int4* xp = (const int4*) (q + at);
  const int4 a = xp[0], b = xp[1];
  x[0] = a.x, x[1] = a.y, x[2] = a.z, x[3] = a.w, x[4] = b.x, x[5] = b.y, x[6] = b.z, x[7] = b.w;
}

// the lanes' xor tree over the row's L logical lanes: acc[l] + acc[l ^ o], o = L/2 .. 1 (reference kernels/q8.h:209)
template <int L>
__device__ inline float tree(float v) {
#pragma unroll
  for (int o = L / 2; o > 0; o >>= 1) v = __fadd_rn(v, __shfl_xor(v, o, kWave));
  return v;
}

// matrix blockIdx.y: 64 / L rows a wave; logical lane ll its blocks ll, ll + L, ... for each of NT tokens
template <uint32_t T, int NT, int L>
__global__ __launch_bounds__(kThreads) void group_tok_kernel(const uint8_t* const* __restrict__ w,
                                                             const int32_t* __restrict__ cnt,
                                                             const int32_t* __restrict__ xrow,
                                                             const int32_t* __restrict__ xin, uint32_t rows,
                                                             uint32_t cols, const int8_t* __restrict__ q,
                                                             const float* __restrict__ d, float* __restrict__ y,
                                                             uint32_t ys) {
  constexpr int G = kWave / L, per = (int) (Block<T>::values / 32);
  const int lane = threadIdx.x % kWave, ll = lane % L;
  const uint32_t m = blockIdx.y, row = (blockIdx.x * kWaves + threadIdx.x / kWave) * G + lane / L;
  const uint32_t n = (uint32_t) cnt[m];
  if (!n) return;  // an entry past a device-built table's live ones (osmos_lane_tables): nothing read or written
  const uint32_t nblk = cols / 32, r0 = (uint32_t) xrow[m];
  const uint8_t* rb = w[m] + (uint64_t) (row < rows ? row : 0) * row_bytes<T>(cols);
  uint64_t xr[NT];
  in_rows<NT>(xin, r0, n, xr);
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = 0.0f;
#pragma unroll 2
  for (uint32_t s = ll; s < nblk; s += L) {
    Codes c;
    codes<T>(rb + (s / per) * Block<T>::bytes, (int) (s % per), c);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      int x[8];
      load_x(q, xr[t] * cols + (uint64_t) s * 32, x);
      acc[t] = __builtin_fmaf(d[xr[t] * nblk + s], block_sum<T>(c, x), acc[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const float v = tree<L>(acc[t]);
    if (ll == 0 && row < rows && (uint32_t) t < n) y[(uint64_t) (r0 + t) * ys + row] = v;
  }
}

// gate and up at once, then the activation (reference kernels/q8.h:214-261)
template <uint32_t T, int NT, int L>
__global__ __launch_bounds__(kThreads) void gate_up_kernel(const uint8_t* const* __restrict__ wg,
                                                           const uint8_t* const* __restrict__ wu,
                                                           const int32_t* __restrict__ cnt,
                                                           const int32_t* __restrict__ xrow,
                                                           const int32_t* __restrict__ xin,
                                                           const int32_t* __restrict__ win, uint32_t rows,
                                                           uint32_t cols, const int8_t* __restrict__ q,
                                                           const float* __restrict__ d,
                                                           const float* __restrict__ scale, float lim,
                                                           float* __restrict__ h, uint32_t hs) {
  constexpr int G = kWave / L, per = (int) (Block<T>::values / 32);
  const int lane = threadIdx.x % kWave, ll = lane % L;
  const uint32_t m = blockIdx.y, row = (blockIdx.x * kWaves + threadIdx.x / kWave) * G + lane / L;
  const uint32_t n = (uint32_t) cnt[m];
  if (!n) return;  // as group_tok_kernel
  const uint32_t nblk = cols / 32, r0 = (uint32_t) xrow[m];
  const uint64_t off = (uint64_t) (row < rows ? row : 0) * row_bytes<T>(cols);
  const uint8_t *rg = wg[m] + off, *ru = wu[m] + off;
  uint64_t xr[NT];
  in_rows<NT>(xin, r0, n, xr);
  float ag[NT], au[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) ag[t] = au[t] = 0.0f;
#pragma unroll 2
  for (uint32_t s = ll; s < nblk; s += L) {
    Codes cg, cu;
    const uint64_t at = (s / per) * Block<T>::bytes;
    codes<T>(rg + at, (int) (s % per), cg);
    codes<T>(ru + at, (int) (s % per), cu);
#pragma unroll
    for (int t = 0; t < NT; t++) {
      int x[8];
      load_x(q, xr[t] * cols + (uint64_t) s * 32, x);
      const float xd = d[xr[t] * nblk + s];
      ag[t] = __builtin_fmaf(xd, block_sum<T>(cg, x), ag[t]);
      au[t] = __builtin_fmaf(xd, block_sum<T>(cu, x), au[t]);
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const float vg = tree<L>(ag[t]), vu = tree<L>(au[t]);
    if (ll == 0 && row < rows && (uint32_t) t < n)
      h[(uint64_t) (r0 + t) * hs + row] = lane_swiglu(vg, vu, lim, scale[win ? win[r0 + t] : r0 + t]);
  }
}

// rows of x to int8 a block at a time (reference kernels/q8.h:263-277): half a wave a block, lane i its value i; the
// block's largest magnitude by the half-wave's tree (max is exact in any order)
__global__ __launch_bounds__(kThreads) void round_kernel(const float* __restrict__ x, uint32_t rows, uint32_t cols,
                                                         uint32_t xs, int8_t* __restrict__ q, float* __restrict__ d) {
  const uint32_t nblk = cols / 32;
  const uint64_t blk = (uint64_t) blockIdx.x * (kThreads / 32) + threadIdx.x / 32;
  const int i = threadIdx.x % 32;
  if (blk >= (uint64_t) rows * nblk) return;  // a whole half-wave
  const uint32_t r = (uint32_t) (blk / nblk), s = (uint32_t) (blk % nblk);
  const float v = x[(uint64_t) r * xs + (uint64_t) s * 32 + i];
  float a = fabsf(v);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
  const float inv = a > 0.0f ? __fdiv_rn(127.0f, a) : 0.0f;
  q[(uint64_t) r * cols + (uint64_t) s * 32 + i] = (int8_t) (int) rintf(__fmul_rn(v, inv));
  if (i == 0) d[(uint64_t) r * nblk + s] = __fdiv_rn(a, 127.0f);
}

// ---- dispatch ----
struct Args {
  const void* const *wg, *const *wu;
  const int32_t *cnt, *xrow, *xin, *win;
  uint32_t n, rows, cols;
  const int8_t* q;
  const float *d, *scale;
  float lim;
  float* y;
  uint32_t ys;
};

template <uint32_t T, int NT, int L>
bool launch(const Args& a, bool fused, hipStream_t s) {
  constexpr uint32_t per_block = kWaves * (kWave / L);
  const dim3 grid((a.rows + per_block - 1) / per_block, a.n);
  if (fused)
    gate_up_kernel<T, NT, L><<<grid, kThreads, 0, s>>>((const uint8_t* const*) a.wg, (const uint8_t* const*) a.wu,
                                                         a.cnt, a.xrow, a.xin, a.win, a.rows, a.cols, a.q, a.d,
                                                         a.scale, a.lim, a.y, a.ys);
  else
    group_tok_kernel<T, NT, L><<<grid, kThreads, 0, s>>>((const uint8_t* const*) a.wg, a.cnt, a.xrow, a.xin, a.rows,
                                                           a.cols, a.q, a.d, a.y, a.ys);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T, int NT>
bool by_lanes(const Args& a, bool fused, hipStream_t s) {
  return a.cols >= 4096 ? launch<T, NT, 32>(a, fused, s) : launch<T, NT, 16>(a, fused, s);
}

template <uint32_t T>
bool by_tokens(const Args& a, uint32_t max_cnt, bool fused, hipStream_t s) {
  if (a.cols % Block<T>::values) return false;
  switch (max_cnt) {
    case 1: return by_lanes<T, 1>(a, fused, s);
    case 2: return by_lanes<T, 2>(a, fused, s);
    case 3: return by_lanes<T, 3>(a, fused, s);
    case 4: return by_lanes<T, 4>(a, fused, s);
    case 5: return by_lanes<T, 5>(a, fused, s);
    case 6: return by_lanes<T, 6>(a, fused, s);
    case 7: return by_lanes<T, 7>(a, fused, s);
    case 8: return by_lanes<T, 8>(a, fused, s);
    default: return false;
  }
}

bool dispatch(uint32_t type, const Args& a, uint32_t max_cnt, bool fused, hipStream_t s) {
  switch (type) {
    case kIQ2_XXS: return by_tokens<kIQ2_XXS>(a, max_cnt, fused, s);
    case kIQ2_XS: return by_tokens<kIQ2_XS>(a, max_cnt, fused, s);
    case kIQ1_M: return by_tokens<kIQ1_M>(a, max_cnt, fused, s);
    case kIQ1_S: return by_tokens<kIQ1_S>(a, max_cnt, fused, s);
    case kIQ2_S: return by_tokens<kIQ2_S>(a, max_cnt, fused, s);
    case kIQ3_XXS: return by_tokens<kIQ3_XXS>(a, max_cnt, fused, s);
    case kQ2_K: return by_tokens<kQ2_K>(a, max_cnt, fused, s);
    case kQ4_0: return by_tokens<kQ4_0>(a, max_cnt, fused, s);
    case kQ4_K: return by_tokens<kQ4_K>(a, max_cnt, fused, s);
    case kQ3_K: return by_tokens<kQ3_K>(a, max_cnt, fused, s);
    default: return false;
  }
}

}  // namespace lane
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool q8_round(const float* x, uint32_t rows, uint32_t cols, uint32_t xs, int8_t* q, float* d,
                         void* stream) {
  if (!x || !q || !d || !rows || !cols || cols % 32 || xs < cols) return false;
  const uint64_t blocks = (uint64_t) rows * (cols / 32), per = lane::kThreads / 32;
  lane::round_kernel<<<(unsigned) ((blocks + per - 1) / per), lane::kThreads, 0, (hipStream_t) stream>>>(x, rows, cols,
                                                                                                        xs, q, d);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool q8_group_tok(uint32_t type, const void* const* w, const int32_t* cnt, const int32_t* xrow,
                             const int32_t* xin, uint32_t n, uint32_t max_cnt, uint32_t rows, uint32_t cols,
                             const int8_t* q, const float* d, float* y, uint32_t ys, void* stream) {
  if (!w || !cnt || !xrow || !q || !d || !y || !n || n > MV_MAX_GROUP || !rows || !max_cnt ||
      max_cnt > MV_MAX_TOKENS || !cols || cols % 32)
    return false;
  const lane::Args a = {w, nullptr, cnt, xrow, xin, nullptr, n, rows, cols, q, d, nullptr, 0.0f, y, ys};
  return lane::dispatch(type, a, max_cnt, false, (hipStream_t) stream);
}

extern "C" OSM_API bool q8_gate_up(uint32_t type, const void* const* wg, const void* const* wu, const int32_t* cnt,
                           const int32_t* xrow, const int32_t* xin, const int32_t* win, uint32_t n, uint32_t max_cnt,
                           uint32_t rows, uint32_t cols, const int8_t* q, const float* d, const float* scale,
                           float lim, float* h, uint32_t hs, void* stream) {
  if (!wg || !wu || !cnt || !xrow || !q || !d || !h || !n || n > MV_MAX_GROUP || !rows || !max_cnt ||
      max_cnt > MV_MAX_TOKENS || !cols || cols % 32 || !scale || hs < rows)
    return false;
  const lane::Args a = {wg, wu, cnt, xrow, xin, win, n, rows, cols, q, d, scale, lim, h, hs};
  return lane::dispatch(type, a, max_cnt, true, (hipStream_t) stream);
}
