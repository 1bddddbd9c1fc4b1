// libosmos MI355X - the quantized weights' f16 matrix products (include/osmos/gpu/mm.h): mm_known, mm_fits,
// mm_col_tiles, mm_x16, mm_x16_rows, mm_run, mm_group.
//
// contract (reference include/osmos/gpu/mm.h:87-200, kernels/mm.hip:24-73, kernels/mm.h:84-90): y = W x over each
// weight's exact value rounded to f16 (RNE) and the f16 activations, products exact in F32; K split the reference's
// way for the type and width - W partitions, partition p the slabs p, p + W, ... (SL values each), one chain of
// matrix-core steps from zero each, then the partitions summed in order. a token's sums its own: the same bits at any
// batch, tiling or grouping.
//
// CDNA4 mapping: a workgroup is 16 rows x W waves, wave p partition p; each step is v_mfma_f32_16x16x32_f16 (32
// values: the gfx950 f16 MMA's K, the reference's WMMA takes 16) - A the lane's row's 8 decoded values, B the same 8
// columns of its token.
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
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kTile = kX16Tile, kStep = 32;

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

// the IQ2 / IQ3 grids as f16 (each grid byte's value as f16 bits) and the 8-value sign masks as f16 sign bits
// (0x8000 in each negated value): sign7 by a 7-bit sign index (its parity bit folded in, gguf's ksigns), sign8 by
// the 8 sign bits themselves
constexpr uint16_t half_bits(uint32_t n) {  // a small positive integer's f16 bits
  int e = 0;
  while ((n >> (e + 1)) != 0) e++;
  return (uint16_t) ((15 + e) << 10 | ((n << (10 - e)) & 0x3FFu));
}
struct alignas(16) HalfGrids {
  uint16_t iq2xxs[256][8], iq2xs[512][8], iq2s[1024][8], iq3xxs[256][4], sign7[128][8], sign8[256][8];
};
constexpr HalfGrids make_half_grids() {
  const Grids g = make_grids();
  HalfGrids h{};
  for (int i = 0; i < 256; i++)
    for (int j = 0; j < 8; j++) h.iq2xxs[i][j] = half_bits((uint32_t) (g.iq2xxs[i] >> (8 * j)) & 0xFF);
  for (int i = 0; i < 512; i++)
    for (int j = 0; j < 8; j++) h.iq2xs[i][j] = half_bits((uint32_t) (g.iq2xs[i] >> (8 * j)) & 0xFF);
  for (int i = 0; i < 1024; i++)
    for (int j = 0; j < 8; j++) h.iq2s[i][j] = half_bits((uint32_t) (g.iq2s[i] >> (8 * j)) & 0xFF);
  for (int i = 0; i < 256; i++)
    for (int j = 0; j < 4; j++) h.iq3xxs[i][j] = half_bits((g.iq3xxs[i] >> (8 * j)) & 0xFF);
  for (int i = 0; i < 256; i++) {
    int par = 0;
    for (int j = 0; j < 7; j++) par ^= (i >> j) & 1;
    const int s7 = (i & 127) | par << 7;
    for (int j = 0; j < 8; j++) {
      if (i < 128) h.sign7[i][j] = (uint16_t) (((s7 >> j) & 1) << 15);
      h.sign8[i][j] = (uint16_t) (((i >> j) & 1) << 15);
    }
  }
  return h;
}
__constant__ HalfGrids kHalf = make_half_grids();

// the codebook a type's decoder reads, held in LDS: for the generic decoder (decode.h's Layout<T>::at `tables`) only
// the members that type reads; for the f16 path of the IQ2 / IQ3 types (decode_h below) the f16 grid and sign masks
template <uint32_t T> struct LdsTab { struct { } g; };
template <> struct LdsTab<kIQ2_XXS> { uint16_t grid[256][8], sign[128][8]; };
template <> struct LdsTab<kIQ2_XS> { uint16_t grid[512][8], sign[128][8]; };
template <> struct LdsTab<kIQ2_S> { uint16_t grid[1024][8], sign[256][8]; };
template <> struct LdsTab<kIQ3_XXS> { uint16_t grid[256][4], sign[128][8]; };
template <> struct LdsTab<kIQ1_S> { struct { uint64_t iq1s[2048]; } g; };
template <> struct LdsTab<kIQ1_M> { struct { uint64_t iq1s[2048]; } g; };
template <> struct LdsTab<kIQ4_NL> { struct { } g; alignas(4) int8_t iq4nl[16]; };
template <> struct LdsTab<kIQ4_XS> { struct { } g; alignas(4) int8_t iq4nl[16]; };

template <uint32_t T>
__device__ inline void fill_tab(LdsTab<T>& t) {  // every thread of the workgroup, from the constant tables
  const uint32_t* src = nullptr;
  const uint32_t* src2 = nullptr;
  uint32_t words = 0, words2 = 0;
  uint32_t* dst = (uint32_t*) &t;
  uint32_t* dst2 = nullptr;
  if constexpr (T == kIQ2_XXS || T == kIQ2_XS || T == kIQ2_S || T == kIQ3_XXS) {
    if constexpr (T == kIQ2_XXS) src = (const uint32_t*) kHalf.iq2xxs;
    else if constexpr (T == kIQ2_XS) src = (const uint32_t*) kHalf.iq2xs;
    else if constexpr (T == kIQ2_S) src = (const uint32_t*) kHalf.iq2s;
    else src = (const uint32_t*) kHalf.iq3xxs;
    src2 = T == kIQ2_S ? (const uint32_t*) kHalf.sign8 : (const uint32_t*) kHalf.sign7;
    words = sizeof t.grid / 4, words2 = sizeof t.sign / 4, dst = (uint32_t*) t.grid, dst2 = (uint32_t*) t.sign;
  } else if constexpr (T == kIQ1_S || T == kIQ1_M) src = (const uint32_t*) kDec.g.iq1s, words = sizeof t / 4;
  else if constexpr (T == kIQ4_NL || T == kIQ4_XS) src = (const uint32_t*) kDec.iq4nl, words = 4, dst = (uint32_t*) t.iq4nl;
  for (uint32_t i = threadIdx.x; i < words; i += blockDim.x) dst[i] = src[i];
  for (uint32_t i = threadIdx.x; i < words2; i += blockDim.x) dst2[i] = src2[i];
}

// the IQ2 / IQ3 types straight to f16: their values are (scale) x (+-grid byte) with the product exact in F32
// (scale d (0.5 + s) / 4 or / 2: at most 16 significant bits; a grid byte at most 6), so each value is the f16 grid
// byte, its sign bit xored in, times the F32 scale and rounded once to f16 - decode.h's exact value rounded to f16,
// the same bits, with no integer-to-float step
template <uint32_t T>
constexpr bool half_path() {
  return T == kIQ2_XXS || T == kIQ2_XS || T == kIQ2_S || T == kIQ3_XXS;
}
template <uint32_t T>
__device__ inline half8 decode_h(const LdsTab<T>& t, const uint8_t* b, int k) {
  uint4 g, sg;
  float scale;
  if constexpr (T == kIQ2_XXS) {
    const uint8_t* g8 = b + 2 + 8 * (k >> 2);
    const uint32_t aux = ld32(g8 + 4);
    scale = mul(mul(half_at(b), 0.5f + (float) (aux >> 28)), 0.25f);
    g = *(const uint4*) t.grid[g8[k & 3]], sg = *(const uint4*) t.sign[(aux >> (7 * (k & 3))) & 127u];
  } else if constexpr (T == kIQ2_XS) {
    const uint32_t e = ld16(b + 2 + 2 * k), s = (b[66 + (k >> 2)] >> (4 * ((k >> 1) & 1))) & 15u;
    scale = mul(mul(half_at(b), 0.5f + (float) s), 0.25f);
    g = *(const uint4*) t.grid[e & 511u], sg = *(const uint4*) t.sign[e >> 9];
  } else if constexpr (T == kIQ2_S) {
    const uint32_t s = (b[74 + (k >> 2)] >> (4 * ((k >> 1) & 1))) & 15u;
    const uint32_t idx = b[2 + k] | ((b[66 + (k >> 2)] >> (2 * (k & 3))) & 3u) << 8;
    scale = mul(mul(half_at(b), 0.5f + (float) s), 0.25f);
    g = *(const uint4*) t.grid[idx], sg = *(const uint4*) t.sign[b[34 + k]];
  } else {  // IQ3_XXS: two 4-value grid entries a chunk
    const uint8_t* idx = b + 2 + 2 * k;
    const uint32_t aux = ld32(b + 66 + 4 * (k >> 2));
    scale = mul(mul(half_at(b), 0.5f + (float) (aux >> 28)), 0.5f);
    const uint2 g0 = *(const uint2*) t.grid[idx[0]], g1 = *(const uint2*) t.grid[idx[1]];
    g = uint4{g0.x, g0.y, g1.x, g1.y}, sg = *(const uint4*) t.sign[(aux >> (7 * (k & 3))) & 127u];
  }
  const uint32_t w[4] = {g.x ^ sg.x, g.y ^ sg.y, g.z ^ sg.z, g.w ^ sg.w};
  // each word's two values times the scale, rounded to f16 into the low and the high half of one register (the mixed
  // fma: an F32 and an f16 operand, exact product, plus -0 so that a -0 product stays -0, one rounding to f16; the
  // low form keeps the high half and the high form the low one, so the pair needs no packing)
  uint32_t p[4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#if __HIP_DEVICE_COMPILE__  // (the instruction exists on the device only; the host pass never runs this)
    asm("v_fma_mixlo_f16 %0, %1, %2, neg(0) op_sel_hi:[0,1,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %2, neg(0) op_sel:[0,1,0] op_sel_hi:[0,1,0]"
        : "=&v"(p[i])
        : "v"(scale), "v"(w[i]));
#else
    p[i] = w[i] ^ __float_as_uint(scale);
#endif
  return __builtin_bit_cast(half8, u32x4{p[0], p[1], p[2], p[3]});
}

// a type's K split (reference kernels/mm.hip:24-73, the Tuned / Short / Odd shapes): SL values a slab, W partitions.
// partition p takes the slabs p, p + W, ... of a row; each partition one chain of MMAs from zero in K order; then the
// partitions' sums added in order, s = part 0, s += part 1, ... a matrix's shape is its type's and its width's, never
// its tokens': a token's bits are the same at any batch
struct KSplit {
  uint32_t sl, w;
};
template <uint32_t T> constexpr KSplit tuned() {
  switch (T) {
    case kQ5_K: case kQ5_KR: return {32, 8};  // (Q5_KR: Q5_K's, a round one block - one 2880-byte piece a tile)
    case kQ4_K: return {32, 16};
    case kIQ1_M: case kIQ1_S: case kIQ2_XXS: case kIQ2_XS: case kIQ2_S: return {128, 4};
    case kIQ4_NL: case kIQ4_XS: case kQ4_0: return {64, 4};
    case kQ2_K: case kQ3_K: return {64, 8};
    default: return {128, 8};  // Q8_0, Q6_K, IQ3_XXS
  }
}
constexpr uint32_t kShortCols = 2048;  // under it mm_run takes the type's short shape (Q6_K: 64 x 8)
template <uint32_t T> constexpr KSplit short_shape() { return T == kQ6_K ? KSplit{64, 8} : tuned<T>(); }
// a width the slab does not divide: Q8_0's 64 x 2 (others: none - mm_fits refuses)
template <uint32_t T> constexpr KSplit odd_shape() { return T == kQ8_0 ? KSplit{64, 2} : short_shape<T>(); }
// mm_run's shape for a width (group: mm_group's - the tuned shape whatever the width)
template <uint32_t T> KSplit shape_of(uint32_t cols, bool group) {
  if (group) return tuned<T>();
  const KSplit s = cols < kShortCols ? short_shape<T>() : tuned<T>();
  return cols % s.sl ? odd_shape<T>() : s;
}

// blockIdx.x: RT tiles of 16 rows; blockIdx.y: the matrix; blockIdx.z: CT token tiles. W waves, wave p the partition
// p. the rows go through LDS a round at a time (a round: W slabs, whole blocks - every partition's next slab),
// double-buffered: the next round's loads in flight while this one is decoded; the type's codebook in LDS once. in a
// round wave p decodes its slab of each row tile (lane l: row l % 16, the 8 values 8 (l / 16) .. of each 32-value
// step, decode.h's exact values rounded to f16) into its A operands and runs v_mfma_f32_16x16x32_f16 against each
// token tile (B: the same 8 columns of token l % 16, one 16-byte load of the tiled x16) - A and B fill the same lane
// slots with the same columns, so each step is its 32 values' dot product whatever order the unit takes them in.
// then the partitions' tiles are summed in order through LDS. RT and CT are the tiling alone: the same sums
template <uint32_t T, uint32_t SL, int W, int CT, int RT, int WB>
// (IQ2_XXS on 4-byte staging words held to 128 VGPRs, 4 waves a SIMD: config 5's gate 761-783 -> 733 us, no spills;
// the other instances spill at that budget)
__global__ __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(T == kIQ2_XXS && WB == 4 ? 4 : 1)))
void kernel(Args a) {
  typedef typename std::conditional<WB == 4, uint32_t, uint16_t>::type word;
  constexpr int kThreads = W * kWave;
  constexpr uint32_t kRows = kTile * RT;                                // the workgroup's rows
  constexpr uint32_t kRv = SL * W;                                      // a round's values a row
  constexpr uint32_t kRb = kRv / Block<T>::values * Block<T>::bytes;    // its bytes
  static_assert(kRv % Block<T>::values == 0, "a round whole blocks");
  constexpr uint32_t kWords = kRows * kRb / WB, kPer = (kWords + kThreads - 1) / kThreads, kWr = kRb / WB;
  constexpr uint32_t kStage = 2 * kRows * kRb, kPart = W * 4 * kWave * 4;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kStage > kPart ? kStage : kPart];
  __shared__ LdsTab<T> tab;
  const uint32_t m = blockIdx.y;
  const uint8_t* w = a.w0;
  const _Float16* x16 = a.x16;
  float* y = a.y;
  uint32_t n = a.n;
  if (a.wt) {
    w = table_at(a.wt, m), n = (uint32_t) a.cnt[m];
    x16 += a.xoff[m], y += a.yoff[m];
  }
  const uint32_t t0 = blockIdx.z * kTile * CT, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, q = lane / 16;
  const uint32_t row0 = blockIdx.x * kRows;
  if (t0 >= n) return;  // (uniform: the whole workgroup)
  const int tiles = (int) ((n - t0 + kTile - 1) / kTile) < CT ? (int) ((n - t0 + kTile - 1) / kTile) : CT;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.cols);
  // this thread's staged words: word i of a round is row i / kWr's word i % kWr, at a 32-bit offset from the matrix
  // (rows past the matrix: its last, staged and not stored). Q5_KR: a round is one block, its tile's 16 rows' 2880
  // bytes side by side in the matrix - word i is tile i / kWt's word i % kWt, and a tile's rows lie in LDS as there
  constexpr bool kTiled = T == kQ5_KR;
  static_assert(!kTiled || kRv == Block<T>::values, "a Q5_KR round one block");
  constexpr uint32_t kWt = kTile * kRb / WB;
  uint32_t woff[kPer];
#pragma unroll
  for (uint32_t u = 0; u < kPer; u++) {
    const uint32_t i = min(u * kThreads + threadIdx.x, kWords - 1);
    if constexpr (kTiled) woff[u] = min(row0 / kTile + i / kWt, a.rows / kTile - 1) * kTile * rb + (i % kWt) * WB;
    else woff[u] = min(row0 + i / kWr, a.rows - 1) * rb + (i % kWr) * WB;
  }
  word wr[kPer];
  const uint32_t nr = (a.cols + kRv - 1) / kRv;  // rounds (the last may be short: its missing slabs skipped)
  auto load = [&](uint32_t r) __attribute__((always_inline)) {
    if constexpr (kTiled) {  // (every round whole: cols a multiple of the block)
      const uint8_t* base = w + (uint64_t) r * kTile * kRb;
#pragma unroll
      for (uint32_t u = 0; u < kPer; u++) wr[u] = gload<word>(base + woff[u]);
    } else {
      const uint32_t lim = (a.cols - r * kRv) / Block<T>::values * Block<T>::bytes;  // the round's bytes a row
      const uint8_t* base = w + (uint64_t) r * kRb;
#pragma unroll
      for (uint32_t u = 0; u < kPer; u++) {
        const uint32_t o = (u * kThreads + threadIdx.x) % kWr * WB;
        wr[u] = gload<word>(base + woff[u] - (o < lim ? 0 : o - (lim - WB)));  // (past a short round: its last word)
      }
    }
  };
  auto store = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (uint32_t u = 0; u < kPer; u++)
      if (u * kThreads + threadIdx.x < kWords) ((word*) (smem + buf * kRows * kRb))[u * kThreads + threadIdx.x] = wr[u];
  };
  fill_tab<T>(tab);
  load(0);
  store(0);
  load(nr > 1 ? 1 : 0);  // (every load made: the in-flight count exact on every path)
  __syncthreads();
  const _Float16* xb = x16 + x16_at(t0 + lane % 16, 8 * q, a.xts);
  f32x4 acc[RT][CT];
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) acc[rt][ct] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // the activations of the wave's next step (its 32 columns of each token tile), loaded a step ahead: every load made
  // (a tile past the live ones reads tile 0 again, a step past the matrix this step's columns), so the loads in flight
  // are counted exactly and each wait is for that one
  // (not for the shapes whose registers it would spill: Q8_0's and Q4_K's four row tiles by two token tiles)
  constexpr bool kXPre = !(RT == 4 && CT == 2 && (T == kQ8_0 || T == kQ4_K));
  half8 bn[CT];
  auto xload = [&](uint32_t kk) __attribute__((always_inline)) {
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
      bn[ct] = gload<half8>(xb + (uint64_t) (ct < tiles ? ct : 0) * kTile * a.xts + (kk / 16) * 256);
  };
  if constexpr (kXPre) xload(wave * SL < a.cols ? wave * SL : 0);
  for (uint32_t r = 0; r < nr; r++) {
    const int buf = (int) (r % 2);
    if (r + 1 < nr) store(buf ^ 1);  // (buffer buf ^ 1's last reads were before the previous barrier)
    load(r + 2 < nr ? r + 2 : nr - 1);  // (past the last round: the last again, not stored)
    const uint32_t k_slab = r * kRv + wave * SL;  // this wave's slab of the round
    if (k_slab < a.cols) {  // (uniform in the wave)
#pragma unroll
      for (uint32_t k0 = 0; k0 < SL; k0 += kStep) {
        half8 av[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
          int k;
          const uint8_t* b;
          if constexpr (kTiled)  // (the tile's block, row lane % 16's chunk in it)
            b = chunk_of<T>(smem + buf * kRows * kRb + rt * kTile * kRb, lane % 16, (wave * SL + k0) / kChunk + q, &k);
          else
            b = chunk_at<T>(smem + buf * kRows * kRb + (rt * kTile + lane % 16) * kRb, (wave * SL + k0) / kChunk + q, &k);
          if constexpr (half_path<T>()) {
            av[rt] = decode_h<T>(tab, b, k);
          } else {
            float v[kChunk];
            decode<T>(tab, b, k, v);
#pragma unroll
            for (int i = 0; i < kChunk; i++) av[rt][i] = (_Float16) v[i];  // nearest, ties to even
          }
        }
        const uint32_t kk = k_slab + k0;
        half8 bc[CT];
        if constexpr (kXPre) {
#pragma unroll
          for (int ct = 0; ct < CT; ct++) bc[ct] = bn[ct];
          const uint32_t nx = k0 + kStep < SL ? kk + kStep : k_slab + kRv;  // the wave's next step
          xload(nx < a.cols ? nx : kk);
        }
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
          if (ct < tiles) {  // (uniform) the tiles that exist
            half8 bv;
            if constexpr (kXPre) bv = bc[ct];
            else bv = gload<half8>(xb + (uint64_t) ct * kTile * a.xts + (kk / 16) * 256);
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
              acc[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[rt], bv, acc[rt][ct], 0, 0, 0);
          }
      }
    }
    __syncthreads();  // round r read by every wave; round r + 1 stored
  }
  // the partitions' sums in order, a tile at a time through LDS (the staging buffers free now): lane l of wave p holds
  // partition p's rows 4 (l / 16) + i, token l % 16 of the tile; register i's outputs are summed by wave i % W
  float* part = (float*) smem;
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      if (ct >= tiles) break;  // (uniform)
      if (rt || ct) __syncthreads();  // the tile before summed
#pragma unroll
      for (int i = 0; i < 4; i++) part[(wave * 4 + i) * kWave + lane] = acc[rt][ct][i];
      __syncthreads();
      const uint32_t t = t0 + ct * kTile + lane % 16, r = row0 + rt * kTile + 4 * q;
      for (int i = (int) wave; i < 4; i += W) {
        float sum = part[i * kWave + lane];
#pragma unroll
        for (int p = 1; p < W; p++) sum = __fadd_rn(sum, part[(p * 4 + i) * kWave + lane]);
        if (t < n && r + i < a.rows) y[(uint64_t) t * a.ys + r + i] = sum;
      }
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

// token tiles a decoded step feeds (the reference's most: 8): the accumulators are 4 VGPRs a tile
constexpr uint32_t col_tiles(uint32_t n) {
  const uint32_t t = (n + kTile - 1) / kTile;
  return t >= 8 ? 8 : t >= 4 ? 4 : t >= 2 ? 2 : 1;
}

// token tiles a workgroup at most: 2 for a 128-value slab's shapes, 4 for the others. at 8 the 128-value shapes need
// more than 256 VGPRs (the 128 x 8 of Q8_0 / Q6_K / IQ3_XXS spills, the 128 x 4 of IQ1 / IQ2 runs a wave a SIMD);
// measured on 2048 -> 7168 at 512 tokens (us, caps 8 / 4 / 2): IQ3_XXS 692 / 147 / 81, IQ2_XXS 318 / 105 / 74,
// Q8_0 704 / 144 / 104, Q4_K 83 / 69 / 96, Q4_0 88 / 59 / 72, IQ4_XS 88 / 57 / 65. the 128 x 8 shape on 2-byte
// staging words also spills at 4 row tiles (Q8_0 / Q6_K), so it takes one
template <uint32_t SL> constexpr int ct_max() { return SL == 128 ? 2 : 4; }
template <uint32_t SL, int W> constexpr bool heavy() { return SL == 128 && W == 8; }
template <uint32_t T, uint32_t SL, int W, int CT, int RT>
bool launch_s(const Args& a, uint32_t n_mat, uint32_t max_n, hipStream_t s) {
  const dim3 grid((a.rows + kTile * RT - 1) / (kTile * RT), n_mat, (max_n + kTile * CT - 1) / (kTile * CT));
  // 4-byte staging loads where every row's round starts 4-aligned (the row bytes and the round bytes multiples of 4:
  // the weights themselves come from hipMalloc, 256-aligned, or a caller's whole-block slice of them)
  constexpr uint32_t rbr = SL * W / Block<T>::values * Block<T>::bytes;
  if (row_bytes<T>(a.cols) % 4 == 0 && rbr % 4 == 0)
    kernel<T, SL, W, CT, RT, 4><<<grid, W * kWave, 0, s>>>(a);
  else if constexpr (RT == 1 || !heavy<SL, W>() || T == kIQ3_XXS)  // (launch_ct never takes the others)
    kernel<T, SL, W, CT, RT, 2><<<grid, W * kWave, 0, s>>>(a);
  else
    return false;
  return hipGetLastError() == hipSuccess;
}

// the tiling: a workgroup's row tiles RT (4 where the launch has row blocks enough for the chip at 64 rows - many
// matrices, or a tall one - else 1) and token tiles CT (at most ct_max, and 2 with 4 row tiles)
template <uint32_t T, uint32_t SL, int W>
bool launch_ct(const Args& a, uint32_t n_mat, uint32_t max_n, hipStream_t s) {
  constexpr uint32_t rbr = SL * W / Block<T>::values * Block<T>::bytes;
  const bool words2 = row_bytes<T>(a.cols) % 4 != 0 || rbr % 4 != 0;
  const bool tall = (uint64_t) n_mat * (a.rows / 64) >= 1024 && !(heavy<SL, W>() && T != kIQ3_XXS && words2);
  const uint32_t ct = col_tiles(max_n);
  if (tall) {
    if (ct == 1) return launch_s<T, SL, W, 1, 4>(a, n_mat, max_n, s);
    return launch_s<T, SL, W, 2, 4>(a, n_mat, max_n, s);
  }
  switch (ct) {
    case 1: return launch_s<T, SL, W, 1, 1>(a, n_mat, max_n, s);
    case 2: return launch_s<T, SL, W, 2, 1>(a, n_mat, max_n, s);
    default: return launch_s<T, SL, W, ct_max<SL>(), 1>(a, n_mat, max_n, s);
  }
}

template <uint32_t T>
bool fits_shape(uint32_t rows, uint32_t cols, bool group) {  // (a matrix under 4 GB: the staging's 32-bit offsets)
  if (!rows || !cols || rows % kTile || cols % Block<T>::values || (uint64_t) rows * row_bytes<T>(cols) > 0xFFFFFFFFull)
    return false;
  if (group && cols % 128) return false;  // (mm_group: whole 128-value slabs, the reference's rule)
  return cols % shape_of<T>(cols, group).sl == 0;
}
template <uint32_t T>
bool fits(uint32_t rows, uint32_t cols) { return fits_shape<T>(rows, cols, false); }

template <uint32_t T>
bool run_by(const Args& a, uint32_t n_mat, uint32_t max_n, hipStream_t s) {
  const bool group = a.wt != nullptr;
  if (!fits_shape<T>(a.rows, a.cols, group)) return false;
  const KSplit k = shape_of<T>(a.cols, group);
  constexpr KSplit t = tuned<T>(), sh = short_shape<T>(), od = odd_shape<T>();
  if (k.sl == t.sl && k.w == t.w) return launch_ct<T, t.sl, (int) t.w>(a, n_mat, max_n, s);
  if (k.sl == sh.sl && k.w == sh.w) return launch_ct<T, sh.sl, (int) sh.w>(a, n_mat, max_n, s);
  return launch_ct<T, od.sl, (int) od.w>(a, n_mat, max_n, s);
}

#define OSM_MM_TYPES(X) \
  X(kQ8_0) X(kQ4_0) X(kIQ4_NL) X(kQ2_K) X(kQ3_K) X(kQ4_K) X(kQ5_K) X(kQ6_K) X(kIQ2_XXS) X(kIQ2_XS) X(kIQ2_S) \
  X(kIQ3_XXS) X(kIQ1_S) X(kIQ1_M) X(kIQ4_XS) X(kQ5_KR)

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
