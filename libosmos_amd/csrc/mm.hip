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
#include <type_traits>

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

// the codebook a type's decoder reads (Dec<T>::run's `tables`), held in LDS: only the members that type reads
template <uint32_t T> struct LdsTab { struct { } g; };
template <> struct LdsTab<kIQ2_XXS> { struct { uint64_t iq2xxs[256]; } g; };
template <> struct LdsTab<kIQ2_XS> { struct { uint64_t iq2xs[512]; } g; };
template <> struct LdsTab<kIQ2_S> { struct { uint64_t iq2s[1024]; } g; };
template <> struct LdsTab<kIQ3_XXS> { struct { uint32_t iq3xxs[256]; } g; };
template <> struct LdsTab<kIQ1_S> { struct { uint64_t iq1s[2048]; } g; };
template <> struct LdsTab<kIQ1_M> { struct { uint64_t iq1s[2048]; } g; };
template <> struct LdsTab<kIQ4_NL> { struct { } g; alignas(4) int8_t iq4nl[16]; };
template <> struct LdsTab<kIQ4_XS> { struct { } g; alignas(4) int8_t iq4nl[16]; };

template <uint32_t T>
__device__ inline void fill_tab(LdsTab<T>& t) {  // every thread of the workgroup, from the constant tables
  const uint32_t* src = nullptr;
  uint32_t words = 0;
  uint32_t* dst = (uint32_t*) &t;
  if constexpr (T == kIQ2_XXS) src = (const uint32_t*) kDec.g.iq2xxs, words = sizeof t / 4;
  else if constexpr (T == kIQ2_XS) src = (const uint32_t*) kDec.g.iq2xs, words = sizeof t / 4;
  else if constexpr (T == kIQ2_S) src = (const uint32_t*) kDec.g.iq2s, words = sizeof t / 4;
  else if constexpr (T == kIQ3_XXS) src = (const uint32_t*) kDec.g.iq3xxs, words = sizeof t / 4;
  else if constexpr (T == kIQ1_S || T == kIQ1_M) src = (const uint32_t*) kDec.g.iq1s, words = sizeof t / 4;
  else if constexpr (T == kIQ4_NL || T == kIQ4_XS) src = (const uint32_t*) kDec.iq4nl, words = 4, dst = (uint32_t*) t.iq4nl;
  for (uint32_t i = threadIdx.x; i < words; i += kThreads) dst[i] = src[i];
}

// values a staged chunk of a row: whole blocks, about 256 bytes of a row (16 KB for the workgroup's 64 rows)
template <uint32_t T>
constexpr uint32_t chunk_values() {
  constexpr uint32_t v = Block<T>::values, b = Block<T>::bytes, per256 = 256 / v * b;
  return v == 1 ? 64 : per256 <= 72 ? 1024 : per256 <= 144 ? 512 : 256;
}

// blockIdx.x: 64 rows (a wave 16); blockIdx.y: the matrix; blockIdx.z: CT token tiles. the rows' bytes go through LDS a
// chunk at a time (double-buffered: the next chunk's loads in flight while this one is decoded), W bytes a load (4
// where every row's chunk is 4-aligned, else 2); the type's codebook is copied into LDS once. each wave decodes its 16
// rows from LDS and runs the K steps in ascending order, as the unstaged kernel did: the same sums, the same bits
template <uint32_t T, int CT, int W>
__global__ __launch_bounds__(kThreads) void kernel(Args a) {
  typedef typename std::conditional<W == 4, uint32_t, uint16_t>::type word;
  constexpr uint32_t kCv = chunk_values<T>(), kCb = kCv / Block<T>::values * Block<T>::bytes;  // a row's chunk
  constexpr uint32_t kWords = kRowsWg * kCb / W, kPer = (kWords + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) uint8_t wbuf[2][kRowsWg * kCb];
  __shared__ LdsTab<T> tab;
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
  const uint32_t rbase = blockIdx.x * kRowsWg, row0 = rbase + wave * kRowsWave;
  if (t0 >= n) return;  // (uniform: the whole workgroup)
  const bool live = row0 < a.rows;  // (a wave past the rows stages and meets the barriers, computes nothing)
  const uint32_t rb = (uint32_t) row_bytes<T>(a.cols), q = lane / 16;
  // this thread's staged words: word i of the chunk is row i / (kCb / W), word i % (kCb / W) of it; its source a 32-bit
  // byte offset from the matrix (one expert's matrix is far under 4 GB) plus the chunk's
  constexpr uint32_t kWr = kCb / W;  // words a row's chunk
  uint32_t woff[kPer];
#pragma unroll
  for (int u = 0; u < kPer; u++) {
    const uint32_t i = min((uint32_t) (u * kThreads) + threadIdx.x, kWords - 1);
    const uint32_t gr = min(rbase + i / kWr, a.rows - 1);  // (rows past the matrix: its last, staged and not used)
    woff[u] = gr * rb + (i % kWr) * W;
  }
  word wr[kPer];
  const uint32_t nch = (a.cols + kCv - 1) / kCv;
  auto load = [&](uint32_t c) __attribute__((always_inline)) {
    // (a short last chunk: the words past its end read its last word instead - loaded, never decoded)
    const uint32_t lim = (a.cols - c * kCv) / Block<T>::values * Block<T>::bytes;  // the chunk's bytes a row
    const uint8_t* base = w + (uint64_t) c * kCb;
#pragma unroll
    for (int u = 0; u < kPer; u++) {
      const uint32_t o = (u * kThreads + threadIdx.x) % kWr * W;
      wr[u] = *(const word*) (base + woff[u] - (o < lim ? 0 : o - (lim - W)));
    }
  };
  auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < kPer; u++)
      if (u * kThreads + threadIdx.x < kWords) ((word*) wbuf[buf])[u * kThreads + threadIdx.x] = wr[u];
  };
  fill_tab<T>(tab);
  load(0);
  store(0);
  if (nch > 1) load(1);
  __syncthreads();
  const _Float16* xb = x16 + x16_at(t0 + lane % 16, 8 * q, a.xts);
  f32x4 acc[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ct++) acc[ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t c = 0; c < nch; c++) {
    const int buf = (int) (c % 2);
    if (c + 1 < nch) store(buf ^ 1);  // (buffer buf ^ 1's last reads were before the previous barrier)
    if (c + 2 < nch) load(c + 2);
    const uint32_t k_end = min(kCv, a.cols - c * kCv);
    const uint8_t* row = wbuf[buf] + (wave * kRowsWave + lane % 16) * kCb;
    if (live) {
      for (uint32_t k0 = 0; k0 < k_end; k0 += kStep) {
        float v[kChunk];
        int k;
        const uint8_t* b = chunk_at<T>(row, k0 / kChunk + q, &k);
        decode<T>(tab, b, k, v);
        half8 av;
#pragma unroll
        for (int i = 0; i < kChunk; i++) av[i] = (_Float16) v[i];  // nearest, ties to even
        const uint32_t kk = c * kCv + k0;
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
          if (t0 + ct * kTile < n) {  // (uniform) the tiles that exist
            const half8 bv = *(const half8*) (xb + (uint64_t) ct * kTile * a.xts + (kk / 16) * 256);
            acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[ct], 0, 0, 0);
          }
      }
    }
    __syncthreads();  // chunk c read by every wave; chunk c + 1 stored
  }
  if (!live) return;
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
  // 4-byte staging loads where every row's chunk starts 4-aligned (the row bytes and the chunk bytes multiples of 4:
  // the weights themselves come from hipMalloc, 256-aligned, or a caller's whole-block slice of them)
  constexpr uint32_t cb = chunk_values<T>() / Block<T>::values * Block<T>::bytes;
  const bool w4 = row_bytes<T>(a.cols) % 4 == 0 && cb % 4 == 0;
  if (w4)
    kernel<T, CT, 4><<<grid, kThreads, 0, s>>>(a);
  else
    kernel<T, CT, 2><<<grid, kThreads, 0, s>>>(a);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool fits(uint32_t rows, uint32_t cols) {  // (a matrix under 4 GB: the staging's 32-bit offsets)
  return rows && cols && rows % kTile == 0 && cols % Block<T>::values == 0 && cols % kStep == 0 &&
         (uint64_t) rows * row_bytes<T>(cols) <= 0xFFFFFFFFull;
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
