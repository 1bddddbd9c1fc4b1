// libosmos MI355X - the decode's fp32-activation matvec (include/osmos/gpu/mv.h): mv_run, mv_strided, mv_group,
// mv_group_tok.
//
// contract (reference kernels/mv.h:1-70, include/osmos/gpu/mv.h:31-62): a row's 8-value chunks c go to logical lane
// c % 32 in ascending order, each chunk's 8 values fmaf'd onto the lane's sum in order (the value decode.h gives, the
// reference's bits), then the 32 lanes' xor tree. any tiling of rows and tokens gives the same bits.
//
// CDNA4 mapping: each half of a wave64 is one 32-lane row group holding R rows; a workgroup is 4 waves = 8 R rows.
// tokens past MV_MAX_TOKENS are tiled 8 at a time over blockIdx.y.
#include "decode.h"

extern "C" {
#include "../../include/osmos/gpu/mv.h"
}

namespace osm {
namespace mv {

__constant__ DecodeTables kDec = make_decode_tables();

constexpr int kWaves = 4, kThreads = kWave * kWaves, kHalf = 32;

// R rows of one half-wave over NT tokens: x rows xs floats apart (token t's at x + t xs), y's ys apart; rows past
// `rows` decode row 0 and store nothing; tokens at or past `live` read the last live token and store nothing
// STG (one row a half-wave, the row a whole number of 16-byte words, at most kStgMax bytes, the matrix 16-aligned): the
// half-wave first copies its row into its own LDS slot with 16-byte loads (a row's bytes in a few wide loads rather
// than a few bytes a chunk), then decodes the same bytes from there - the same values, so the same bits
constexpr uint32_t kStgMax = 2048;
// the types whose decode reads a chunk's bytes in many small pieces (K-quant scale fields, IQ grid indices, sign and
// scale bytes); measured on 8192 x 2048 at one token, staged / not (us): Q2_K 6.3 / 7.3, IQ2_XXS 7.0 / 7.6, IQ2_XS
// 6.9 / 8.0, IQ2_S 7.2 / 10.0, IQ3_XXS 8.4 / 9.8, IQ4_XS 12.8 / 14.9 and IQ4_NL 13.0 / 15.6 with the IQ4 table in
// memory (7.1 and 8.0 staged with it as byte permutes); Q4_K staged 7.6; Q4_0 (8.2 / 7.7) and Q6_K (11.1 / 9.8) were
// slower staged, Q3_K and Q8_0 even
template <uint32_t T> constexpr bool stages() {
  return T == kQ2_K || T == kQ4_K || T == kQ5_K || T == kIQ2_XXS || T == kIQ2_XS || T == kIQ2_S || T == kIQ3_XXS ||
         T == kIQ1_S || T == kIQ1_M || T == kIQ4_XS || T == kIQ4_NL;
}
// XL (one token): x already copied into the workgroup's LDS (xl): the 8 rows of a workgroup read it there, not each
// from L2 - the same values, so the same bits
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(3))) f32x4v lds_f4;
constexpr uint32_t kXlMax = 4096;  // x floats a workgroup copies at most
// the types that take it: measured at one token on 8192 x 2048 (us, x from L2 / from LDS): Q4_0 6.43 / 5.69, BF16
// 8.44 / 8.16; slower for the rest (F32 14.1 / 14.1, Q8_0 8.11 / 8.25, Q3_K 8.18 / 10.85, Q4_K 7.22 / 9.16, Q6_K
// 9.81 / 13.32, IQ2_XXS 7.23 / 7.46, IQ4_NL 7.72 / 9.94 ...: the compiler keeps fewer of their weight loads in flight)
template <uint32_t T> constexpr bool x_in_lds() { return T == kQ4_0 || T == kBF16; }
template <uint32_t T, int NT, int R, bool STG = false, bool XL = false>
__device__ inline void rows_of(const uint8_t* __restrict__ w, uint32_t rows, uint32_t cols, const float* __restrict__ x,
                               uint32_t xs, float* __restrict__ y, uint32_t ys, uint32_t live,
                               lds_f4* xl = nullptr) {
  const int lane = threadIdx.x % kHalf;
  const uint32_t row0 = ((blockIdx.x * kWaves + threadIdx.x / kWave) * 2 + (threadIdx.x % kWave) / kHalf) * R;
  // SW (an even token tile): the two half-waves hold the same chunks of different rows, so each loads half of the
  // tokens' x and the halves swap them (v_permlane32_swap): half the vector-memory work for x, which bounds the
  // multi-token matvec (2048 -> 6144 at 64 tokens, us: Q4_K 82.5 -> 60.5, Q3_K 99.8 -> 73.9). both halves then stay
  // to the end - a row past `rows` decodes row 0 and stores nothing
  constexpr bool SW = NT >= 2 && NT % 2 == 0;
  if (!SW && row0 >= rows) return;  // the whole half-wave: its tree's partners are its own
  const uint8_t* base[R];
#pragma unroll
  for (int q = 0; q < R; q++) base[q] = row_base<T>(w, row0 + q < rows ? row0 + q : 0, cols);
  if constexpr (STG) {
    static_assert(T != kQ5_KR, "a Q5_KR row is not contiguous");
    static_assert(R == 1, "a staged half-wave holds one row");
    __shared__ __attribute__((aligned(16))) uint8_t stg[2 * kWaves][kStgMax];
    uint8_t* slot = stg[threadIdx.x / kHalf];
    const uint32_t words = (uint32_t) row_bytes<T>(cols) / 16;
    const uint4* src = (const uint4*) base[0];
    uint4 r[kStgMax / 16 / kHalf];
#pragma unroll
    for (int i = 0; i < (int) (kStgMax / 16 / kHalf); i++)
      r[i] = src[min((uint32_t) (lane + i * kHalf), words - 1)];  // (every load made: a conditional one puts r in scratch)
#pragma unroll
    for (int i = 0; i < (int) (kStgMax / 16 / kHalf); i++)
      if (lane + i * kHalf < (int) words) ((uint4*) slot)[lane + i * kHalf] = r[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // (the slot is the half-wave's own: no workgroup barrier)
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    base[0] = slot;
  }
  const float* xt[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) xt[t] = x + (uint64_t) ((uint32_t) t < live ? t : live - 1) * xs;
  const uint32_t chunks = cols / kChunk;
  float acc[R][NT];
#pragma unroll
  for (int q = 0; q < R; q++)
#pragma unroll
    for (int t = 0; t < NT; t++) acc[q][t] = 0.0f;
#pragma unroll(NT == 1 ? 8 : SW ? 1 : 2)  // (one token: the lane's chunks' loads all in flight at once; the swaps
                                          // are convergent, so a loop holding them stays rolled)
  for (uint32_t c = lane; c < chunks; c += kHalf) {
    float v[R][kChunk];
#pragma unroll
    for (int q = 0; q < R; q++) {
      int k;
      const uint8_t* b = chunk_of<T>(base[q], row0 + q < rows ? row0 + q : 0, c, &k);
      decode<T>(kDec, b, k, v[q]);
    }
    float xv[NT][kChunk];
    if constexpr (SW) {
      // half h loads tokens h NT / 2 ..; one swap of a word gives every lane the lower half's value (first) and the
      // upper half's (second): tokens t and NT / 2 + t
      const uint32_t h = (threadIdx.x % kWave) / kHalf;
#pragma unroll
      for (int t = 0; t < NT / 2; t++) {
        const uint32_t tok = h * (NT / 2) + t;
        const float* p = x + (uint64_t) (tok < live ? tok : live - 1) * xs + (uint64_t) c * kChunk;
        const float4 a = ((const float4*) p)[0], b = ((const float4*) p)[1];
        const float w[kChunk] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < kChunk; e++) {
          const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(w[e]), __float_as_uint(w[e]), false, false);
          xv[t][e] = __uint_as_float(r[0]), xv[NT / 2 + t][e] = __uint_as_float(r[1]);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        float4 a, b;
        if constexpr (XL) {
          static_assert(NT == 1, "x in LDS: one token");
          const f32x4v va = xl[2 * c], vb = xl[2 * c + 1];
          a = make_float4(va.x, va.y, va.z, va.w), b = make_float4(vb.x, vb.y, vb.z, vb.w);
        } else {
          a = ((const float4*) (xt[t] + (uint64_t) c * kChunk))[0];
          b = ((const float4*) (xt[t] + (uint64_t) c * kChunk))[1];
        }
        xv[t][0] = a.x, xv[t][1] = a.y, xv[t][2] = a.z, xv[t][3] = a.w;
        xv[t][4] = b.x, xv[t][5] = b.y, xv[t][6] = b.z, xv[t][7] = b.w;
      }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
      const float4 a = make_float4(xv[t][0], xv[t][1], xv[t][2], xv[t][3]);
      const float4 b = make_float4(xv[t][4], xv[t][5], xv[t][6], xv[t][7]);
#pragma unroll
      for (int q = 0; q < R; q++) {
        float s = acc[q][t];
        s = __builtin_fmaf(v[q][0], a.x, s), s = __builtin_fmaf(v[q][1], a.y, s);
        s = __builtin_fmaf(v[q][2], a.z, s), s = __builtin_fmaf(v[q][3], a.w, s);
        s = __builtin_fmaf(v[q][4], b.x, s), s = __builtin_fmaf(v[q][5], b.y, s);
        s = __builtin_fmaf(v[q][6], b.z, s), s = __builtin_fmaf(v[q][7], b.w, s);
        acc[q][t] = s;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < R; q++)
#pragma unroll
    for (int t = 0; t < NT; t++) {
      float s = acc[q][t];
#pragma unroll
      for (int o = kHalf / 2; o > 0; o >>= 1) s = __fadd_rn(s, __shfl_xor(s, o, kWave));
      if (lane == 0 && row0 + q < rows && (uint32_t) t < live) y[(uint64_t) t * ys + row0 + q] = s;
    }
}

// one matrix, n_tok tokens in tiles of NT over blockIdx.y
template <uint32_t T, int NT, int R, bool STG>
__device__ __forceinline__ void tokens_item(const uint8_t* __restrict__ w, uint32_t rows, uint32_t cols,
                                            const float* __restrict__ x, uint32_t xs, uint32_t n_tok,
                                            float* __restrict__ y, uint32_t ys) {
  const uint32_t t0 = blockIdx.y * NT, live = n_tok - t0 < (uint32_t) NT ? n_tok - t0 : NT;
  if constexpr (NT == 1 && x_in_lds<T>()) {
    if (cols <= kXlMax) {  // (uniform) the token's row into LDS: every load first, then the stores
      __shared__ __attribute__((aligned(16))) float xsm[kXlMax];
      constexpr int U = (int) (kXlMax / 4 / kThreads);
      const float4* src = (const float4*) (x + (uint64_t) t0 * xs);
      const uint32_t nw = cols / 4;
      float4 r[U];
#pragma unroll
      for (int u = 0; u < U; u++) r[u] = src[min(threadIdx.x + u * kThreads, nw - 1)];
#pragma unroll
      for (int u = 0; u < U; u++)
        if (threadIdx.x + u * kThreads < nw) ((float4*) xsm)[threadIdx.x + u * kThreads] = r[u];
      __syncthreads();
      rows_of<T, NT, R, STG, true>(w, rows, cols, x + (uint64_t) t0 * xs, xs, y + (uint64_t) t0 * ys, ys, live,
                                   (lds_f4*) xsm);
      return;
    }
  }
  rows_of<T, NT, R, STG>(w, rows, cols, x + (uint64_t) t0 * xs, xs, y + (uint64_t) t0 * ys, ys, live);
}

template <uint32_t T, int NT, int R, bool STG = false>
__global__ __launch_bounds__(kThreads) void kernel(const uint8_t* __restrict__ w, uint32_t rows, uint32_t cols,
                                                   const float* __restrict__ x, uint32_t xs, uint32_t n_tok,
                                                   float* __restrict__ y, uint32_t ys) {
  tokens_item<T, NT, R, STG>(w, rows, cols, x, xs, n_tok, y, ys);
}
// the same with the compiler's register budget set for 4 waves a SIMD (a one-token launch has about that many): it
// then keeps more of a lane's chunk loads in flight. measured at one token (us, 8192 x 2048 / 6144 x 2048): Q4_0
// 5.68 / 5.29 -> 5.10 / 4.68, F32 14.1 / 11.3 -> 13.0 / 10.5, Q8_0 6.94 -> 6.42 (6144), Q3_K 6.99 -> 6.70, the IQ2 / IQ1 /
// K types 1-3 % faster; IQ4_NL 7.64 -> 9.47, Q6_K 9.78 -> 9.96 and IQ2_XS 5.79 -> 5.93 (6144) slower, so they keep
// the first
template <uint32_t T> constexpr bool budget4() { return T != kIQ4_NL && T != kQ6_K && T != kIQ2_XS; }
template <uint32_t T, int NT, int R, bool STG = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void kernel4(
    const uint8_t* __restrict__ w, uint32_t rows, uint32_t cols, const float* __restrict__ x, uint32_t xs,
    uint32_t n_tok, float* __restrict__ y, uint32_t ys) {
  tokens_item<T, NT, R, STG>(w, rows, cols, x, xs, n_tok, y, ys);
}

// n matrices of one shape (blockIdx.y the matrix): x at x + (m / x_div) x_mat, y at y + m rows
template <uint32_t T, int R>
__global__ __launch_bounds__(kThreads) void group_kernel(const uint8_t* const* __restrict__ w, uint32_t rows,
                                                         uint32_t cols, const float* __restrict__ x, uint32_t x_mat,
                                                         uint32_t x_div, float* __restrict__ y) {
  const uint32_t m = blockIdx.y;
  const uint8_t* wm = table_at(w, m);
  const float* xm = x + (uint64_t) (m / x_div) * x_mat;
  if constexpr (stages<T>() && R == 1) {  // (the matrix's alignment is known only here: a uniform choice per matrix)
    const uint32_t rb = (uint32_t) row_bytes<T>(cols);
    if (rb % 16 == 0 && rb <= kStgMax && (uintptr_t) wm % 16 == 0) {
      rows_of<T, 1, R, true>(wm, rows, cols, xm, cols, y + (uint64_t) m * rows, rows, 1);
      return;
    }
  }
  rows_of<T, 1, R>(wm, rows, cols, xm, cols, y + (uint64_t) m * rows, rows, 1);
}

// matrices each over their own cnt[m] tokens from row xrow[m] (0: skipped)
template <uint32_t T, int NT, int R>
__global__ __launch_bounds__(kThreads) void group_tok_kernel(const uint8_t* const* __restrict__ w,
                                                             const int32_t* __restrict__ cnt,
                                                             const int32_t* __restrict__ xrow, uint32_t rows,
                                                             uint32_t cols, const float* __restrict__ x, uint32_t xs,
                                                             float* __restrict__ y, uint32_t ys) {
  const uint32_t m = blockIdx.y, n = (uint32_t) cnt[m];
  if (!n) return;
  const uint64_t r0 = (uint64_t) xrow[m];
  rows_of<T, NT, R>(table_at(w, m), rows, cols, x + r0 * xs, xs, y + r0 * ys, ys, n < (uint32_t) NT ? n : NT);
}

// rows a half-wave: the tiling alone, never the bits (one token: a row a half-wave, for as many waves as the rows give)
template <int NT> constexpr int rows_per() { return NT == 1 ? 1 : 2; }

template <uint32_t T, int NT>
bool run_nt(const void* w, uint32_t rows, uint32_t cols, const float* x, uint32_t xs, uint32_t n_tok, float* y,
            uint32_t ys, hipStream_t s) {
  const uint32_t rb = (uint32_t) row_bytes<T>(cols);
  auto grid = [&](uint32_t r) { return dim3((rows + kWaves * 2 * r - 1) / (kWaves * 2 * r), (n_tok + NT - 1) / NT); };
  // (the staged row copy at tiles of up to 4 tokens, one row a half-wave: 2048 -> 6144 Q4_K at 8 tokens 22.1 -> 15.5
  // us; at tiles of 8 it lost, 60 -> 70 us at 64 tokens)
  constexpr bool B4 = NT == 1 && budget4<T>();
  if constexpr (stages<T>()) {
    if (NT <= 4 && rb % 16 == 0 && rb <= kStgMax && (uintptr_t) w % 16 == 0) {
      if constexpr (B4)
        kernel4<T, NT, 1, true><<<grid(1), kThreads, 0, s>>>((const uint8_t*) w, rows, cols, x, xs, n_tok, y, ys);
      else
        kernel<T, NT, 1, true><<<grid(1), kThreads, 0, s>>>((const uint8_t*) w, rows, cols, x, xs, n_tok, y, ys);
      return hipGetLastError() == hipSuccess;
    }
  }
  if constexpr (B4)
    kernel4<T, NT, rows_per<NT>()><<<grid(rows_per<NT>()), kThreads, 0, s>>>((const uint8_t*) w, rows, cols, x, xs,
                                                                              n_tok, y, ys);
  else
    kernel<T, NT, rows_per<NT>()><<<grid(rows_per<NT>()), kThreads, 0, s>>>((const uint8_t*) w, rows, cols, x, xs,
                                                                             n_tok, y, ys);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool by_tokens(const void* w, uint32_t rows, uint32_t cols, const float* x, uint32_t xs, uint32_t n_tok, float* y,
               uint32_t ys, hipStream_t s) {
  if (!w || !x || !y || !rows || !cols || cols % Block<T>::values || cols % kChunk || !n_tok) return false;
  if (T == kQ5_KR && rows % 16) return false;  // (whole tiles of 16 rows: quant_repack_q5k's)
  if ((n_tok > 1 && (xs < cols || ys < rows)) || xs % kChunk) return false;
  switch (n_tok) {
    case 1: return run_nt<T, 1>(w, rows, cols, x, xs, n_tok, y, ys, s);
    case 2: return run_nt<T, 2>(w, rows, cols, x, xs, n_tok, y, ys, s);
    case 3: return run_nt<T, 3>(w, rows, cols, x, xs, n_tok, y, ys, s);
    case 4: return run_nt<T, 4>(w, rows, cols, x, xs, n_tok, y, ys, s);
    case 5: case 6: case 7: case 8:  // (tiles of 4: twice the waves for the few tokens' rows)
      return run_nt<T, 4>(w, rows, cols, x, xs, n_tok, y, ys, s);
    default:  // 9 .. any: tiles of 8 (Q3_K took tiles of 4 before the x exchange: 2048 -> 6144 at 64 tokens 74 -> 59 us)
      return run_nt<T, 8>(w, rows, cols, x, xs, n_tok, y, ys, s);
  }
}

template <uint32_t T>
bool group(const void* const* w, uint32_t n, uint32_t rows, uint32_t cols, const float* x, uint32_t x_mat,
           uint32_t x_div, float* y, hipStream_t s) {
  if (!w || !x || !y || cols % Block<T>::values || cols % kChunk || x_mat % kChunk || !x_div) return false;
  constexpr uint32_t per = kWaves * 2 * rows_per<1>();
  group_kernel<T, rows_per<1>()><<<dim3((rows + per - 1) / per, n), kThreads, 0, s>>>((const uint8_t* const*) w, rows, cols, x,
                                                                            x_mat, x_div, y);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T, int NT>
bool group_tok_nt(const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n, uint32_t rows,
                  uint32_t cols, const float* x, uint32_t xs, float* y, uint32_t ys, hipStream_t s) {
  constexpr uint32_t per = kWaves * 2 * rows_per<NT>();
  group_tok_kernel<T, NT, rows_per<NT>()><<<dim3((rows + per - 1) / per, n), kThreads, 0, s>>>(
      (const uint8_t* const*) w, cnt, xrow, rows, cols, x, xs, y, ys);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool group_tok(const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n, uint32_t max_cnt,
               uint32_t rows, uint32_t cols, const float* x, uint32_t xs, float* y, uint32_t ys, hipStream_t s) {
  if (!w || !cnt || !xrow || !x || !y || cols % Block<T>::values || cols % kChunk || xs < cols || xs % kChunk)
    return false;
  switch (max_cnt) {
    case 1: return group_tok_nt<T, 1>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    case 2: return group_tok_nt<T, 2>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    case 3: return group_tok_nt<T, 3>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    case 4: return group_tok_nt<T, 4>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    case 5: return group_tok_nt<T, 5>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    case 6: return group_tok_nt<T, 6>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    case 7: return group_tok_nt<T, 7>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    case 8: return group_tok_nt<T, 8>(w, cnt, xrow, n, rows, cols, x, xs, y, ys, s);
    default: return false;
  }
}

#define OSM_MV_TYPES(X) \
  X(kF32) X(kBF16) X(kQ8_0) X(kQ4_0) X(kIQ4_NL) X(kQ2_K) X(kQ3_K) X(kQ4_K) X(kQ5_K) X(kQ6_K) X(kIQ2_XXS) X(kIQ2_XS) \
  X(kIQ2_S) X(kIQ3_XXS) X(kIQ1_S) X(kIQ1_M) X(kIQ4_XS)

}  // namespace mv
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool mv_strided(uint32_t type, const void* w, uint32_t rows, uint32_t cols, const float* x, uint32_t xs,
                           uint32_t n_tok, float* y, uint32_t ys, void* stream) {
  const hipStream_t s = (hipStream_t) stream;
  switch (type) {
#define X(t) \
  case t: return mv::by_tokens<t>(w, rows, cols, x, xs, n_tok, y, ys, s);
    OSM_MV_TYPES(X) X(kQ5_KR)  // (Q5_KR the one-matrix product's alone, as the reference's kernels/mv.hip:277)
#undef X
    default: return false;
  }
}

extern "C" OSM_API bool mv_run(uint32_t type, const void* w, uint32_t rows, uint32_t cols, const float* x, uint32_t n_tok,
                       float* y, void* stream) {
  if (n_tok > MV_MAX_TOKENS) return false;
  return mv_strided(type, w, rows, cols, x, cols, n_tok, y, rows, stream);
}

extern "C" OSM_API bool mv_group(uint32_t type, const void* const* w, uint32_t n, uint32_t rows, uint32_t cols, const float* x,
                         uint32_t x_mat, uint32_t x_div, float* y, void* stream) {
  if (!n || n > MV_MAX_GROUP || !rows) return false;
  const hipStream_t s = (hipStream_t) stream;
  switch (type) {
#define X(t) \
  case t: return mv::group<t>(w, n, rows, cols, x, x_mat, x_div, y, s);
    OSM_MV_TYPES(X)
#undef X
    default: return false;
  }
}

extern "C" OSM_API bool mv_group_tok(uint32_t type, const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n,
                             uint32_t max_cnt, uint32_t rows, uint32_t cols, const float* x, uint32_t xs, float* y,
                             uint32_t ys, void* stream) {
  if (!n || n > MV_MAX_GROUP || !rows || !max_cnt || max_cnt > MV_MAX_TOKENS) return false;
  const hipStream_t s = (hipStream_t) stream;
  switch (type) {
#define X(t) \
  case t: return mv::group_tok<t>(w, cnt, xrow, n, max_cnt, rows, cols, x, xs, y, ys, s);
    OSM_MV_TYPES(X)
#undef X
    default: return false;
  }
}
