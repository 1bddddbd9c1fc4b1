// libosmos MI355X - the lane contract at prefill scale on the int8 matrix cores (include/osmos_mi355x.h:
// osmos_lane_group): q8_group_tok's sums for any token count, the same bits.
//
// contract (reference kernels/lane.h:43-75, kernels/q8.h:133-212, src/cpu/q8.c:383-407): a row's 32-value blocks s go to
// logical lane ll = s % L (L = 32 for cols >= 4096, else 16) in ascending order; per block each 16-value half's exact
// integer dot with the int8 activations, then ((d s21) / 8) isum per half, the halves added, fmaf'd with the block's
// activation scale onto the lane's sum; then the lanes' xor tree (pairs ll, ll ^ L/2 first, then ll ^ L/4, ...).
//
// CDNA4 mapping: a wave owns 16 rows x CT tiles of 16 tokens. the integer half-dots are MFMAs: each 32-value block's
// codes (lane l: row l % 16, values 8 (l / 16) .. + 7, decoded straight into its A operand - the IQ1 types' 8 grid +
// delta folded into one int8 per value) go to two v_mfma_i32_16x16x32_i8, one with the second half's lanes zeroed,
// one with the first's: the two halves' exact dots for 16 rows x 16 tokens. the float steps then run per output in the
// contract's order. a logical lane's chain is one accumulator: the chains are run one after another, in bit-reversed
// lane order, so the xor tree becomes a post-order walk that keeps at most log2(L) partial sums - the same additions
// as the tree, operand for operand (fadd commutes exactly).
#include "lanedec.h"

extern "C" {
#include "../../include/osmos_mi355x.h"
}

namespace osm {
namespace lgemm {

using namespace lane;

constexpr int kWaves = 4, kThreads = kWave * kWaves;
constexpr uint32_t kTile = 16;
typedef int v4i __attribute__((ext_vector_type(4)));

// a lane's chunk k (values 8k .. 8k + 7) of block j of a 256-value super-block: two words of int8 codes (IQ1: 8 grid +
// delta), as codes<T> (lanedec.h) gives them for that chunk
template <uint32_t T>
__device__ inline void chunk(const uint8_t* b, int j, int k, const typename GridOf<T>::E* grid, uint32_t& w0,
                             uint32_t& w1);
// the block's scale and each half's s21
template <uint32_t T>
__device__ inline void scales(const uint8_t* b, int j, float& d, int& s0, int& s1);

// 8 v + delta a byte, v in {-1, 0, 1} (0xFF, 0, 1): a byte permute from a pool of the three results
__device__ inline uint32_t iq1_codes(uint32_t w, int delta) {
  const uint32_t pool = (uint32_t) (uint8_t) delta | (uint32_t) (uint8_t) (8 + delta) << 8 |
                        (uint32_t) (uint8_t) (-8 + delta) << 24;
  return __builtin_amdgcn_perm(0u, pool, w & 0x03030303u);  // v's low 2 bits: 0 -> byte 0, 1 -> 1, 3 (-1) -> 3
}

// reference kernels/q8.h:46-55
template <>
__device__ inline void chunk<kIQ2_XXS>(const uint8_t* b, int j, int k, const GridOf<kIQ2_XXS>::E* grid, uint32_t& w0,
                                       uint32_t& w1) {
  const uint8_t* q = b + 2 + 8 * j;
  int lo, hi;
  signed8(grid[q[k]], ksign((ld32(q + 4) >> (7 * k)) & 0x7F), lo, hi);
  w0 = (uint32_t) lo, w1 = (uint32_t) hi;
}
template <>
__device__ inline void scales<kIQ2_XXS>(const uint8_t* b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (int) (ld32(b + 2 + 8 * j + 4) >> 28) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:57-66
template <>
__device__ inline void chunk<kIQ2_XS>(const uint8_t* b, int j, int k, const GridOf<kIQ2_XS>::E* grid, uint32_t& w0,
                                      uint32_t& w1) {
  const uint32_t q = ld16(b + 2 + 2 * (4 * j + k));
  int lo, hi;
  signed8(grid[q & 511], ksign(q >> 9), lo, hi);
  w0 = (uint32_t) lo, w1 = (uint32_t) hi;
}
template <>
__device__ inline void scales<kIQ2_XS>(const uint8_t* b, int j, float& d, int& s0, int& s1) {
  const uint32_t s = b[66 + j];
  s0 = 2 * (int) (s & 0x0F) + 1, s1 = 2 * (int) (s >> 4) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:86-95
template <>
__device__ inline void chunk<kIQ2_S>(const uint8_t* b, int j, int k, const GridOf<kIQ2_S>::E* grid, uint32_t& w0,
                                     uint32_t& w1) {
  const int kk = 4 * j + k;
  int lo, hi;
  signed8(grid[b[2 + kk] | ((b[66 + j] >> (2 * k)) & 0x03) << 8], b[34 + kk], lo, hi);
  w0 = (uint32_t) lo, w1 = (uint32_t) hi;
}
template <>
__device__ inline void scales<kIQ2_S>(const uint8_t* b, int j, float& d, int& s0, int& s1) {
  const uint32_t s = b[74 + j];
  s0 = 2 * (int) (s & 0x0F) + 1, s1 = 2 * (int) (s >> 4) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:97-108, through the signed table (lanedec.h)
template <>
__device__ inline void chunk<kIQ3_XXS>(const uint8_t* b, int j, int k, const GridOf<kIQ3_XXS>::E* grid, uint32_t& w0,
                                       uint32_t& w1) {
  const uint8_t* q = b + 2 + 8 * j;
  const uint32_t sg = (ld32(b + 66 + 4 * j) >> (7 * k)) & 0x7F, par = __builtin_popcount(sg) & 1u;
  w0 = grid[16 * q[2 * k] + (sg & 15)];
  w1 = grid[16 * q[2 * k + 1] + ((sg >> 4) | par << 3)];
}
template <>
__device__ inline void scales<kIQ3_XXS>(const uint8_t* b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (2 * (int) (ld32(b + 66 + 4 * j) >> 28) + 1);
  d = f16(ld16(b));
}
// reference kernels/q8.h:120-130
template <>
__device__ inline void chunk<kIQ1_S>(const uint8_t* b, int j, int k, const GridOf<kIQ1_S>::E* grid, uint32_t& w0,
                                     uint32_t& w1) {
  const uint32_t h = ld16(b + 34 + 2 * j);
  const uint64_t g = grid[b[2 + 4 * j + k] | ((h >> (3 * k)) & 0x07) << 8];
  const int delta = h & 0x8000 ? -1 : 1;
  w0 = iq1_codes((uint32_t) g, delta), w1 = iq1_codes((uint32_t) (g >> 32), delta);
}
template <>
__device__ inline void scales<kIQ1_S>(const uint8_t* b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (int) ((ld16(b + 34 + 2 * j) >> 12) & 0x07) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:68-84
template <>
__device__ inline void chunk<kIQ1_M>(const uint8_t* b, int j, int k, const GridOf<kIQ1_M>::E* grid, uint32_t& w0,
                                     uint32_t& w1) {
  const int kk = 4 * j + k;
  const uint32_t h = (b[32 + kk / 2] >> (4 * (kk % 2))) & 0x0F;
  const uint64_t g = grid[b[kk] | (h & 0x07) << 8];
  const int delta = h & 0x08 ? -1 : 1;
  w0 = iq1_codes((uint32_t) g, delta), w1 = iq1_codes((uint32_t) (g >> 32), delta);
}
template <>
__device__ inline void scales<kIQ1_M>(const uint8_t* b, int j, float& d, int& s0, int& s1) {
  const uint32_t sc0 = ld32(b + 48), sc1 = ld32(b + 52);
  const uint64_t sc = (uint64_t) sc0 | (uint64_t) sc1 << 32;
  const int k0 = 4 * j, k1 = 4 * j + 2;
  s0 = 2 * (int) ((sc >> (16 * (k0 / 8) + 3 * ((k0 / 2) % 4))) & 0x07) + 1;
  s1 = 2 * (int) ((sc >> (16 * (k1 / 8) + 3 * ((k1 / 2) % 4))) & 0x07) + 1;
  const uint32_t a0 = sc0 & 0xFFFF, a1 = sc0 >> 16, a2 = sc1 & 0xFFFF, a3 = sc1 >> 16;
  d = f16((a0 >> 12) | ((a1 >> 8) & 0x00F0) | ((a2 >> 4) & 0x0F00) | (a3 & 0xF000));
}

// blockIdx.x: 64 rows (a wave 16); blockIdx.y: the matrix, its cnt[m] tokens from row xrow[m] of q / d, CT tiles of
// 16 at a time
template <uint32_t T, int L, int CT>
__global__ __launch_bounds__(kThreads) void kernel(const uint8_t* const* __restrict__ w, const int32_t* __restrict__ cnt,
                                                   const int32_t* __restrict__ xrow, uint32_t rows, uint32_t cols,
                                                   const int8_t* __restrict__ q, const float* __restrict__ d,
                                                   float* __restrict__ y, uint32_t ys) {
  constexpr int per = (int) (Block<T>::values / 32), kLog = L == 32 ? 5 : 4;
  __shared__ float scl[kWaves][2][kTile];  // a block's 16 rows' ((d s21) / 8) of each half, a wave's own
  const uint32_t m = blockIdx.y, n = (uint32_t) cnt[m];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, col = lane % 16, quad = lane / 16;
  const uint32_t row0 = blockIdx.x * kTile * kWaves + wave * kTile;
  if (!n || row0 >= rows) return;  // (uniform: the matrix's, then the wave's; no workgroup barrier follows)
  const uint32_t nblk = cols / 32, r0 = (uint32_t) xrow[m];
  const uint8_t* arow = w[m] + (uint64_t) (row0 + col) * row_bytes<T>(cols);  // this lane's A row
  const auto* grid = const_grid<T>();
  for (uint32_t c0 = 0; c0 < n; c0 += kTile * CT) {
    // this lane's B token in each tile (past the count: the last token, summed, never stored)
    const int8_t* xb[CT];
    const float* xd[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      const uint32_t t = c0 + ct * kTile + col, tt = t < n ? t : n - 1;
      xb[ct] = q + (uint64_t) (r0 + tt) * cols + 8 * quad;
      xd[ct] = d + (uint64_t) (r0 + tt) * nblk;
    }
    float stack[kLog][CT][4];  // the tree's pending left subtrees, level by level
    float root[CT][4];
    for (int p = 0; p < L; p++) {  // (uniform) chains in bit-reversed lane order
      const uint32_t ll = __builtin_bitreverse32((uint32_t) p) >> (32 - kLog);
      float acc[CT][4];
#pragma unroll
      for (int ct = 0; ct < CT; ct++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[ct][i] = 0.0f;
      for (uint32_t s = ll; s < nblk; s += L) {
        const uint8_t* blk = arow + (uint64_t) (s / per) * Block<T>::bytes;
        const int j = (int) (s % per);
        uint32_t w0, w1;
        chunk<T>(blk, j, quad, grid, w0, w1);
        const long a = (long) (((uint64_t) w1 << 32) | w0);
        const long a0 = quad < 2 ? a : 0, a1 = quad < 2 ? 0 : a;  // the first half's lanes, the second's
        if (quad == 0) {  // lanes 0 .. 15: row col's ((d s21) / 8) per half (lane_part's first two products)
          float dd;
          int s0, s1;
          scales<T>(blk, j, dd, s0, s1);
          scl[wave][0][col] = __fmul_rn(__fmul_rn(dd, (float) s0), 0.125f);
          scl[wave][1][col] = __fmul_rn(__fmul_rn(dd, (float) s1), 0.125f);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float f0[4], f1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) f0[i] = scl[wave][0][4 * quad + i], f1[i] = scl[wave][1][4 * quad + i];
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
          if (c0 + ct * kTile < n) {  // (uniform) the tiles that exist
            const long bx = *(const long*) (xb[ct] + (uint64_t) s * 32);
            const v4i I0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a0, bx, v4i{0, 0, 0, 0}, 0, 0, 0);
            const v4i I1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a1, bx, v4i{0, 0, 0, 0}, 0, 0, 0);
            const float xs = xd[ct][s];
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const float sub = __fadd_rn(__fmul_rn(f0[i], (float) I0[i]), __fmul_rn(f1[i], (float) I1[i]));
              acc[ct][i] = __builtin_fmaf(xs, sub, acc[ct][i]);
            }
          }
        }
        __builtin_amdgcn_wave_barrier();  // the table read by every lane before the next block's is written
      }
      // the chain's sum into the tree: position p's leaf, merged with each complete left sibling
#pragma unroll
      for (int ct = 0; ct < CT; ct++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float v = acc[ct][i];
          bool open = true;
#pragma unroll
          for (int lv = 0; lv < kLog; lv++)
            if (open) {
              if ((p >> lv) & 1) v = __fadd_rn(stack[lv][ct][i], v);
              else stack[lv][ct][i] = v, open = false;
            }
          if (open) root[ct][i] = v;  // p = L - 1: the whole tree
        }
    }
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {
      const uint32_t t = c0 + ct * kTile + col;
      if (t < n)
#pragma unroll
        for (int i = 0; i < 4; i++) y[(uint64_t) (r0 + t) * ys + row0 + 4 * quad + i] = root[ct][i];
    }
  }
}

template <uint32_t T, int L>
bool by_tiles(const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n_mat, uint32_t max_cnt,
              uint32_t rows, uint32_t cols, const int8_t* q, const float* d, float* y, uint32_t ys, hipStream_t s) {
  const dim3 grid((rows + kTile * kWaves - 1) / (kTile * kWaves), n_mat);
  if (max_cnt <= kTile)
    kernel<T, L, 1><<<grid, kThreads, 0, s>>>((const uint8_t* const*) w, cnt, xrow, rows, cols, q, d, y, ys);
  else
    kernel<T, L, 2><<<grid, kThreads, 0, s>>>((const uint8_t* const*) w, cnt, xrow, rows, cols, q, d, y, ys);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool by_lanes(const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n_mat, uint32_t max_cnt,
              uint32_t rows, uint32_t cols, const int8_t* q, const float* d, float* y, uint32_t ys, hipStream_t s) {
  if (cols % Block<T>::values) return false;
  return cols >= 4096 ? by_tiles<T, 32>(w, cnt, xrow, n_mat, max_cnt, rows, cols, q, d, y, ys, s)
                      : by_tiles<T, 16>(w, cnt, xrow, n_mat, max_cnt, rows, cols, q, d, y, ys, s);
}

}  // namespace lgemm
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool osmos_lane_group(uint32_t type, const void* const* w, const int32_t* cnt, const int32_t* xrow,
                                         uint32_t n_mat, uint32_t max_cnt, uint32_t rows, uint32_t cols,
                                         const int8_t* q, const float* d, float* y, uint32_t ys, void* stream) {
  if (!w || !cnt || !xrow || !q || !d || !y || !n_mat || n_mat > 65535 || !max_cnt || max_cnt > OSMOS_LANE_MAX_TOKENS ||
      !rows || rows % lgemm::kTile || !cols || cols % 256 || ys < rows)
    return false;
  const hipStream_t s = (hipStream_t) stream;
  switch (type) {
#define X(t) \
  case t: return lgemm::by_lanes<t>(w, cnt, xrow, n_mat, max_cnt, rows, cols, q, d, y, ys, s);
    X(kIQ2_XXS) X(kIQ2_XS) X(kIQ2_S) X(kIQ3_XXS) X(kIQ1_S) X(kIQ1_M)
#undef X
    default: return false;
  }
}
