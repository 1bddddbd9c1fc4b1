// libosmos MI355X - the quantized weights' f16 matrix products (include/osmos/gpu/mm.h): mm_known, mm_fits,
// mm_col_tiles, mm_x16, mm_x16_rows, mm_run, mm_group.
//
// contract (reference include/osmos/gpu/mm.h:119-200, kernels/mm.h): y = W x over each weight's exact value rounded
// to f16 (RNE) and the f16 activations, products exact in F32 and summed in F32 by the matrix cores.
//
// CDNA4 mapping: a wave owns 16 rows; each 32-value K step it decodes its A operand straight into registers - lane l
// the 8 values 8 (l / 16) .. + 7 of row l % 16 (decode.h's chunk, the mv contract's exact values), then f16 - and runs
// v_mfma_f32_16x16x32_f16 against up to CT token tiles of x16 (lane l's B operand the same 8 columns of token l % 16:
// one 16-byte load from the tiled layout). A and B fill the same lane slots with the same columns, so the product is
// the dot product whatever order the unit takes K in; the accumulator of a token depends on that token's column
// alone, the K steps always in ascending order - the same bits at any batch size, tile count or grouping.
#include "decode.h"
#include "x16.h"

extern "C" {
#include "../../include/osmos/gpu/mm.h"
}

namespace osm {
namespace mm {

__constant__ DecodeTables kDec = make_decode_tables();

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4, kThreads = kWave * kWaves;
constexpr uint32_t kTile = kX16Tile, kRowsWave = 16, kRowsWg = kRowsWave * kWaves, kStep = 32;

struct Args {
  const uint8_t* w0;            // mm_run's matrix (wt NULL)
  const uint8_t* const* wt;     // mm_group's matrices, with cnt / xoff / yoff
  const int32_t* cnt;
  const uint32_t* xoff;
  const uint32_t* yoff;
  uint32_t n, rows, cols, xts, ys;
  const _Float16* x16;
  float* y;
};

// blockIdx.x: 64 rows; blockIdx.y: the matrix; blockIdx.z: CT token tiles
template <uint32_t T, int CT>
__global__ __launch_bounds__(kThreads) void kernel(Args a) {
  const uint32_t m = blockIdx.y;
  const uint8_t* w = a.w0;
  const _Float16* x16 = a.x16;
  float* y = a.y;
  uint32_t n = a.n;
  if (a.wt) {
    w = a.wt[m], n = (uint32_t) a.cnt[m];
    x16 += a.xoff[m], y += a.yoff[m];
  }
  const uint32_t t0 = blockIdx.z * kTile * CT, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const uint32_t row0 = blockIdx.x * kRowsWg + wave * kRowsWave;
  if (t0 >= n || row0 >= a.rows) return;  // (uniform: the block's, then the wave's)
  const uint32_t q = lane / 16;           // the lane's 8-value chunk of each 32-value step
  const uint8_t* wr = w + (uint64_t) (row0 + lane % 16) * row_bytes<T>(a.cols);
  const _Float16* xb = x16 + x16_at(t0 + lane % 16, 8 * q, a.xts);
  f32x4 acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ct++) acc[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t k0 = 0; k0 < a.cols; k0 += kStep) {
    float v[kChunk];
    int k;
    const uint8_t* b = chunk_at<T>(wr, k0 / kChunk + q, &k);
    decode<T>(kDec, b, k, v);
    half8 av;
#pragma unroll
    for (int i = 0; i < kChunk; i++) av[i] = (_Float16) v[i];  // nearest, ties to even
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
      if (t0 + ct * kTile < n) {  // (uniform) the tiles that exist
        const half8 bv = *(const half8*) (xb + (uint64_t) ct * kTile * a.xts + (k0 / 16) * 256);
        acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[ct], 0, 0, 0);
      }
  }
  // the accumulator: lane l holds rows 4 (l / 16) + i of the wave's 16, token l % 16 of the tile
#pragma unroll
  for (int ct = 0; ct < CT; ct++) {
    const uint32_t t = t0 + ct * kTile + lane % 16;
    if (t < n)
#pragma unroll
      for (int i = 0; i < 4; i++) y[(uint64_t) t * a.ys + row0 + 4 * q + i] = acc[ct][i];
  }
}

// F32 rows to the tiled f16: a thread 8 columns of one token (16 bytes out); rows at or past n zero. Rows: token t is
// row idx[t] of x (-1: zero), read as two float4s
template <bool Rows>
__global__ __launch_bounds__(256) void x16_kernel(const float* __restrict__ x, uint32_t xs, const int32_t* __restrict__ idx,
                                                  uint32_t n, uint32_t cols, _Float16* __restrict__ x16,
                                                  int32_t* __restrict__ overflow) {
  const uint32_t g = blockIdx.x * 256 + threadIdx.x, groups = cols / 8;
  const uint32_t t = g / groups, c = (g % groups) * 8;
  const uint32_t n16 = (n + kTile - 1) / kTile * kTile;
  if (t >= n16) return;
  const float* src = nullptr;
  if (t < n) {
    if constexpr (Rows) {
      const int32_t r = idx[t];
      if (r >= 0) src = x + (uint64_t) r * xs + c;
    } else {
      src = x + (uint64_t) t * xs + c;
    }
  }
  half8 h;
  bool over = false;
  if (src) {
    float v[8];
    if constexpr (Rows) {
      const float4 a = ((const float4*) src)[0], b = ((const float4*) src)[1];
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = src[i];
    }
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = x16_round(v[i], over);
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = (_Float16) 0.0f;
  }
  *(half8*) (x16 + x16_at(t, c, cols)) = h;
  if (over && overflow) *overflow = 1;
}

constexpr uint32_t col_tiles(uint32_t n) {
  const uint32_t t = (n + kTile - 1) / kTile;
  return t >= 4 ? 4 : t >= 2 ? 2 : 1;
}

template <uint32_t T, int CT>
bool launch(const Args& a, uint32_t n_mat, uint32_t max_n, hipStream_t s) {
  const dim3 grid((a.rows + kRowsWg - 1) / kRowsWg, n_mat, (max_n + kTile * CT - 1) / (kTile * CT));
  kernel<T, CT><<<grid, kThreads, 0, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool fits(uint32_t rows, uint32_t cols) {
  return rows && cols && rows % kTile == 0 && cols % Block<T>::values == 0 && cols % kStep == 0;
}

template <uint32_t T>
bool run_by(const Args& a, uint32_t n_mat, uint32_t max_n, hipStream_t s) {
  if (!fits<T>(a.rows, a.cols)) return false;
  switch (col_tiles(max_n)) {
    case 1: return launch<T, 1>(a, n_mat, max_n, s);
    case 2: return launch<T, 2>(a, n_mat, max_n, s);
    default: return launch<T, 4>(a, n_mat, max_n, s);
  }
}

#define OSM_MM_TYPES(X) \
  X(kQ8_0) X(kQ4_0) X(kIQ4_NL) X(kQ2_K) X(kQ3_K) X(kQ4_K) X(kQ5_K) X(kQ6_K) X(kIQ2_XXS) X(kIQ2_XS) X(kIQ2_S) \
  X(kIQ3_XXS) X(kIQ1_S) X(kIQ1_M) X(kIQ4_XS)

bool run(uint32_t type, const Args& a, uint32_t n_mat, uint32_t max_n, hipStream_t s) {
  switch (type) {
#define X(t) \
  case t: return run_by<t>(a, n_mat, max_n, s);
    OSM_MM_TYPES(X)
#undef X
    default: return false;
  }
}

bool known(uint32_t type) {
  switch (type) {
#define X(t) case t:
    OSM_MM_TYPES(X)
#undef X
    return true;
    default: return false;
  }
}

bool fits_type(uint32_t type, uint32_t rows, uint32_t cols) {
  switch (type) {
#define X(t) \
  case t: return fits<t>(rows, cols);
    OSM_MM_TYPES(X)
#undef X
    default: return false;
  }
}

}  // namespace mm
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool mm_known(uint32_t type) { return mm::known(type); }

extern "C" OSM_API bool mm_fits(uint32_t type, uint32_t rows, uint32_t cols) { return mm::fits_type(type, rows, cols); }

extern "C" OSM_API uint32_t mm_col_tiles(uint32_t type, uint32_t n) {
  return mm::known(type) && n ? mm::col_tiles(n) : 0;
}

extern "C" OSM_API bool mm_x16(const float* x, uint32_t xs, uint32_t n, uint32_t cols, void* x16, int32_t* overflow,
                               void* stream) {
  if (!x || !x16 || (uintptr_t) x16 % 16 || !n || n > MM_MAX_TOKENS || !cols || cols % 16 || xs < cols) return false;
  const uint64_t threads = (uint64_t) (n + 15) / 16 * 16 * (cols / 8);
  mm::x16_kernel<false><<<(uint32_t) ((threads + 255) / 256), 256, 0, (hipStream_t) stream>>>(
      x, xs, nullptr, n, cols, (_Float16*) x16, overflow);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool mm_x16_rows(const float* x, uint32_t xs, const int32_t* idx, uint32_t slots, uint32_t cols,
                                    void* x16, int32_t* overflow, void* stream) {
  if (!x || !idx || !x16 || (uintptr_t) x16 % 16 || !slots || !cols || cols % 16 || xs < cols || xs % 4 ||
      (uintptr_t) x % 16)
    return false;
  const uint64_t threads = (uint64_t) (slots + 15) / 16 * 16 * (cols / 8);
  mm::x16_kernel<true><<<(uint32_t) ((threads + 255) / 256), 256, 0, (hipStream_t) stream>>>(
      x, xs, idx, slots, cols, (_Float16*) x16, overflow);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool mm_run(uint32_t type, const void* w, uint32_t rows, uint32_t cols, const void* x16, uint32_t n,
                               float* y, uint32_t ys, void* stream) {
  if (!w || !x16 || (uintptr_t) x16 % 16 || !y || !n || n > MM_MAX_TOKENS || (n > 1 && ys < rows)) return false;
  const mm::Args a = {(const uint8_t*) w, nullptr, nullptr, nullptr, nullptr, n, rows, cols, cols, ys,
                      (const _Float16*) x16, y};
  return mm::run(type, a, 1, n, (hipStream_t) stream);
}

extern "C" OSM_API bool mm_group(uint32_t type, const void* const* w, const int32_t* cnt, uint32_t n_mat,
                                 uint32_t max_cnt, uint32_t rows, uint32_t cols, const void* x16, const uint32_t* xoff,
                                 uint32_t xts, float* y, const uint32_t* yoff, uint32_t ys, void* stream) {
  if (!w || !cnt || !x16 || (uintptr_t) x16 % 16 || !xoff || !y || !yoff || !n_mat || n_mat > MM_MAX_GROUP || !max_cnt ||
      max_cnt > MM_MAX_TOKENS || xts < cols || xts % 16 || (max_cnt > 1 && ys < rows))
    return false;
  const mm::Args a = {nullptr, (const uint8_t* const*) w, cnt, xoff, yoff, 0, rows, cols, xts, ys,
                      (const _Float16*) x16, y};
  return mm::run(type, a, n_mat, max_cnt, (hipStream_t) stream);
}
