// libosmos MI355X - the lane contract at prefill scale on the int8 matrix cores (include/osmos_mi355x.h:
// osmos_lane_group): q8_group_tok's sums for any token count, the same bits.
//
// contract (reference kernels/lane.h:43-75, kernels/q8.h:133-212, src/cpu/q8.c:383-407): a row's 32-value blocks s go to
// logical lane ll = s % L (L = 32 for cols >= 4096, else 16) in ascending order; per block each 16-value half's exact
// integer dot with the int8 activations, then ((d s21) / 8) isum per half, the halves added, fmaf'd with the block's
// activation scale onto the lane's sum; then the lanes' xor tree (pairs ll, ll ^ L/2 first, then ll ^ L/4, ...).
//
// CDNA4 mapping: a workgroup owns 16 rows (their whole slab and the codebook staged in LDS once) x CT tiles of 16
// tokens a pass. the integer half-dots are MFMAs: each 32-value block's codes (lane l: row l % 16, values 8 (l / 16) ..
// + 7, decoded from LDS straight into its B operand - the IQ1 types' 8 grid + delta folded into one int8 per value;
// the tokens' codes the A operand) go to two v_mfma_i32_16x16x32_i8, one with the second half's lanes zeroed, one
// with the first's: the two halves' exact dots, D[token][row] - lane l holds tokens 4 (l / 16) + i of its own row
// l % 16, so it applies that row's half scales itself. the float steps then run per output in the contract's order. the 4 waves split
// the logical lanes (wave w the chains ll = w mod 4, blocks s = w mod 4), so a wave keeps L / 4 chains an output in
// registers; the xor tree is finished across the waves through LDS with the same additions (fadd commutes exactly).
#include "lanedec.h"

extern "C" {
#include "../../include/osmos_mi355x.h"
}

namespace osm {
namespace lgemm {

using namespace lane;

constexpr uint32_t kTile = 16;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// (the block bytes are in LDS: lbytes, their 2-aligned words read 16 bits at a time)
// a lane's chunk k (values 8k .. 8k + 7) of block j of a 256-value super-block: two words of int8 codes (IQ1: 8 grid +
// delta), as codes<T> (lanedec.h) gives them for that chunk
template <uint32_t T>
__device__ inline void chunk(lbytes b, int j, int k, const typename GridOf<T>::E* grid, const uint64_t* sm,
                             uint32_t& w0, uint32_t& w1);
// the block's scale and each half's s21
template <uint32_t T>
__device__ inline void scales(lbytes b, int j, float& d, int& s0, int& s1);

// 8 v + delta a byte, v in {-1, 0, 1} (0xFF, 0, 1): a byte permute from a pool of the three results
__device__ inline uint32_t iq1_codes(uint32_t w, int delta) {
  const uint32_t pool = (uint32_t) (uint8_t) delta | (uint32_t) (uint8_t) (8 + delta) << 8 |
                        (uint32_t) (uint8_t) (-8 + delta) << 24;
  return __builtin_amdgcn_perm(0u, pool, w & 0x03030303u);  // v's low 2 bits: 0 -> byte 0, 1 -> 1, 3 (-1) -> 3
}

// 8 unsigned grid bytes negated where the byte mask m is 0xFF: (v ^ m) + (m & 1) a byte (signed8's arithmetic, the
// mask read from a table of the 128 7-bit sign fields' masks, parity bit included)
__device__ inline void signs8(uint64_t g, uint64_t m, uint32_t& w0, uint32_t& w1) {
  const uint32_t m0 = (uint32_t) m, m1 = (uint32_t) (m >> 32);
  w0 = ((uint32_t) g ^ m0) + (m0 & 0x01010101u), w1 = ((uint32_t) (g >> 32) ^ m1) + (m1 & 0x01010101u);
}
// the table: entry i, ksign(i)'s 8 bits as bytes of 0xFF (set) or 0
__device__ inline uint64_t sign_mask(uint32_t i) {
  const uint32_t s = ksign(i);
  uint64_t m = 0;
#pragma unroll
  for (int b = 0; b < 8; b++) m |= (uint64_t) ((s >> b) & 1u) * (0xFFull << (8 * b));
  return m;
}

// reference kernels/q8.h:46-55
template <>
__device__ inline void chunk<kIQ2_XXS>(lbytes b, int j, int k, const GridOf<kIQ2_XXS>::E* grid, const uint64_t* sm,
                                       uint32_t& w0,
                                       uint32_t& w1) {
  const auto q = b + 2 + 8 * j;
  signs8(grid[q[k]], sm[(ld32s(q + 4) >> (7 * k)) & 0x7F], w0, w1);
}
template <>
__device__ inline void scales<kIQ2_XXS>(lbytes b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (int) (ld32s(b + 2 + 8 * j + 4) >> 28) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:57-66
template <>
__device__ inline void chunk<kIQ2_XS>(lbytes b, int j, int k, const GridOf<kIQ2_XS>::E* grid, const uint64_t* sm,
                                       uint32_t& w0,
                                      uint32_t& w1) {
  const uint32_t q = ld16(b + 2 + 2 * (4 * j + k));
  signs8(grid[q & 511], sm[q >> 9], w0, w1);
}
template <>
__device__ inline void scales<kIQ2_XS>(lbytes b, int j, float& d, int& s0, int& s1) {
  const uint32_t s = b[66 + j];
  s0 = 2 * (int) (s & 0x0F) + 1, s1 = 2 * (int) (s >> 4) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:86-95
template <>
__device__ inline void chunk<kIQ2_S>(lbytes b, int j, int k, const GridOf<kIQ2_S>::E* grid, const uint64_t* sm,
                                       uint32_t& w0,
                                     uint32_t& w1) {
  const int kk = 4 * j + k;
  int lo, hi;
  signed8(grid[b[2 + kk] | ((b[66 + j] >> (2 * k)) & 0x03) << 8], b[34 + kk], lo, hi);
  w0 = (uint32_t) lo, w1 = (uint32_t) hi;
}
template <>
__device__ inline void scales<kIQ2_S>(lbytes b, int j, float& d, int& s0, int& s1) {
  const uint32_t s = b[74 + j];
  s0 = 2 * (int) (s & 0x0F) + 1, s1 = 2 * (int) (s >> 4) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:97-108, through the signed table (lanedec.h)
template <>
__device__ inline void chunk<kIQ3_XXS>(lbytes b, int j, int k, const GridOf<kIQ3_XXS>::E* grid, const uint64_t* sm,
                                       uint32_t& w0,
                                       uint32_t& w1) {
  const auto q = b + 2 + 8 * j;
  const uint32_t sg = (ld32s(b + 66 + 4 * j) >> (7 * k)) & 0x7F, par = __builtin_popcount(sg) & 1u;
  w0 = grid[16 * q[2 * k] + (sg & 15)];
  w1 = grid[16 * q[2 * k + 1] + ((sg >> 4) | par << 3)];
}
template <>
__device__ inline void scales<kIQ3_XXS>(lbytes b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (2 * (int) (ld32s(b + 66 + 4 * j) >> 28) + 1);
  d = f16(ld16(b));
}
// reference kernels/q8.h:120-130
template <>
__device__ inline void chunk<kIQ1_S>(lbytes b, int j, int k, const GridOf<kIQ1_S>::E* grid, const uint64_t* sm,
                                       uint32_t& w0,
                                     uint32_t& w1) {
  const uint32_t h = ld16(b + 34 + 2 * j);
  const uint64_t g = grid[b[2 + 4 * j + k] | ((h >> (3 * k)) & 0x07) << 8];
  const int delta = h & 0x8000 ? -1 : 1;
  w0 = iq1_codes((uint32_t) g, delta), w1 = iq1_codes((uint32_t) (g >> 32), delta);
}
template <>
__device__ inline void scales<kIQ1_S>(lbytes b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (int) ((ld16(b + 34 + 2 * j) >> 12) & 0x07) + 1;
  d = f16(ld16(b));
}
// reference kernels/q8.h:68-84
template <>
__device__ inline void chunk<kIQ1_M>(lbytes b, int j, int k, const GridOf<kIQ1_M>::E* grid, const uint64_t* sm,
                                       uint32_t& w0,
                                     uint32_t& w1) {
  const int kk = 4 * j + k;
  const uint32_t h = (b[32 + kk / 2] >> (4 * (kk % 2))) & 0x0F;
  const uint64_t g = grid[b[kk] | (h & 0x07) << 8];
  const int delta = h & 0x08 ? -1 : 1;
  w0 = iq1_codes((uint32_t) g, delta), w1 = iq1_codes((uint32_t) (g >> 32), delta);
}
template <>
__device__ inline void scales<kIQ1_M>(lbytes b, int j, float& d, int& s0, int& s1) {
  const uint32_t sc0 = ld32s(b + 48), sc1 = ld32s(b + 52);
  const uint64_t sc = (uint64_t) sc0 | (uint64_t) sc1 << 32;
  const int k0 = 4 * j, k1 = 4 * j + 2;
  s0 = 2 * (int) ((sc >> (16 * (k0 / 8) + 3 * ((k0 / 2) % 4))) & 0x07) + 1;
  s1 = 2 * (int) ((sc >> (16 * (k1 / 8) + 3 * ((k1 / 2) % 4))) & 0x07) + 1;
  const uint32_t a0 = sc0 & 0xFFFF, a1 = sc0 >> 16, a2 = sc1 & 0xFFFF, a3 = sc1 >> 16;
  d = f16((a0 >> 12) | ((a1 >> 8) & 0x00F0) | ((a2 >> 4) & 0x0F00) | (a3 & 0xF000));
}

// token tiles a pass and waves a workgroup at 16 / 32 logical lanes: the waves split the logical lanes, so a wave holds
// L / W chains x CT tiles x 4 accumulators (64 / 32 VGPRs), and each decoded block serves CT tiles. measured on config
// 5's IQ2_XXS gate (32 lanes): 4 waves and one tile 1.98 ms; 8 waves (so four tiles fit) 3.2 ms, 8 waves and two
// tiles 2.2 ms - most of its experts hold one tile, and the larger workgroups halve the occupancy
constexpr int kCT16 = 4, kCT32 = 1, kW16 = 4, kW32 = 4;

template <uint32_t T>
constexpr uint32_t grid_bytes_of() {
  return GridOf<T>::n * sizeof(typename GridOf<T>::E);
}

// dynamic LDS: the workgroup's 16 weight rows (the whole slab), the codebook, the sign masks, the waves' scale tables
// and their partial trees
template <uint32_t T, int CT, int W>
struct Lds {
  uint32_t slab, grid, sm, part, total;
  __host__ __device__ Lds(uint32_t rb) {
    slab = 0;
    grid = (16 * rb + 15) / 16 * 16;
    sm = grid + grid_bytes_of<T>();
    part = sm + 128 * 8;
    total = part + W * CT * 4 * kWave * 4;
  }
};

// blockIdx.x: 16 rows; blockIdx.y: the matrix, its cnt[m] tokens from row xrow[m] of q / d, CT tiles of 16 a pass.
// wave w takes the blocks s = w (mod W): its chains are the logical lanes ll = w (mod W), L / W accumulators an
// output; the xor tree's levels L/2 .. W pair chains of one wave (in registers), its levels W/2 .. 1 pair the waves
// (through LDS) - the same additions as the tree
template <uint32_t T, int L, int CT, int W>
__global__ __launch_bounds__(W * kWave) void kernel(const uint8_t* const* __restrict__ w, const int32_t* __restrict__ cnt,
                                                   const int32_t* __restrict__ xrow, uint32_t cols,
                                                   const int8_t* __restrict__ q, const float* __restrict__ d,
                                                   float* __restrict__ y, uint32_t ys) {
  constexpr int kWaves = W, kThreads = W * kWave;
  constexpr int per = (int) (Block<T>::values / 32), C = L / kWaves;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t m = blockIdx.y, n = (uint32_t) cnt[m];
  if (!n) return;  // (the whole workgroup)
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, col = lane % 16, quad = lane / 16;
  const uint32_t row0 = blockIdx.x * kTile, nblk = cols / 32, r0 = (uint32_t) xrow[m];
  const uint32_t rb = (uint32_t) row_bytes<T>(cols);
  const Lds<T, CT, W> L_(rb);
  // the slab (16 rows x rb: contiguous, 16-aligned) and the codebook into LDS
  {
    const u32x4* src = (const u32x4*) (w[m] + (uint64_t) row0 * rb);
    const uint32_t nw = 16 * rb / 16;
    for (uint32_t i = threadIdx.x; i < nw; i += kThreads) ((u32x4*) (smem + L_.slab))[i] = src[i];
    constexpr uint32_t ng = grid_bytes_of<T>() / 16;
    const u32x4* gs = (const u32x4*) const_grid<T>();
    for (uint32_t i = threadIdx.x; i < ng; i += kThreads) ((u32x4*) (smem + L_.grid))[i] = gs[i];
    if (threadIdx.x < 128) ((uint64_t*) (smem + L_.sm))[threadIdx.x] = sign_mask(threadIdx.x);
  }
  __syncthreads();
  const auto* grid = (const typename GridOf<T>::E*) (smem + L_.grid);
  const uint64_t* sm = (const uint64_t*) (smem + L_.sm);
  float* part = (float*) (smem + L_.part);                    // [wave][ct][i][lane]
  const uint8_t* arow = smem + L_.slab + col * rb;            // this lane's A row
  for (uint32_t c0 = 0; c0 < n; c0 += kTile * CT) {
    // (the matrix's first token row as a scalar base, each lane's token as a 32-bit offset from it: tokens under
    // OSMOS_LANE_MAX_TOKENS, so tt cols fits)
    const int8_t* qb = q + (uint64_t) r0 * cols;
    const float* db = d + (uint64_t) r0 * nblk;
    uint32_t xb[CT], xd[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ct++) {  // this lane's B token (past the count: the last, summed, never stored)
      const uint32_t t = c0 + ct * kTile + col, tt = t < n ? t : n - 1;
      xb[ct] = tt * cols + 8 * quad;
      xd[ct] = tt * nblk;
    }
    const int tiles = (int) ((n - c0 + kTile - 1) / kTile) < CT ? (int) ((n - c0 + kTile - 1) / kTile) : CT;
    float acc[C][CT][4];
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
      for (int ct = 0; ct < CT; ct++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[c][ct][i] = 0.0f;
    // the activations of the wave's next block, loaded one block ahead (global memory's latency behind the MFMAs)
    long bxn[CT];
    float xsn[CT];
    auto xload = [&](uint32_t s) __attribute__((always_inline)) {
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        const uint32_t sc = s < nblk ? s : 0;
        bxn[ct] = *(const long*) (qb + (xb[ct] + sc * 32));
        xsn[ct] = db[xd[ct] + sc];
      }
    };
    xload((uint32_t) wave);
    for (uint32_t s0 = (uint32_t) wave; s0 < nblk; s0 += L) {
#pragma unroll
      for (int c = 0; c < C; c++) {
        const uint32_t s = s0 + kWaves * c;  // logical lane wave + 4 c
        if (s >= nblk) break;                // (uniform)
        long bx[CT];
        float xs[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ct++) bx[ct] = bxn[ct], xs[ct] = xsn[ct];
        xload(s + kWaves);
        const uint8_t* blk = arow + (s / per) * Block<T>::bytes;
        const int j = (int) (s % per);
        uint32_t w0, w1;
        chunk<T>((lbytes) blk, j, quad, grid, sm, w0, w1);
        const long a = (long) (((uint64_t) w1 << 32) | w0);
        const long a0 = quad < 2 ? a : 0, a1 = quad < 2 ? 0 : a;  // the first half's lanes, the second's
        // row col's ((d s21) / 8) per half (lane_part's first two products): every lane its own row's
        float dd;
        int s0_, s1_;
        scales<T>((lbytes) blk, j, dd, s0_, s1_);
        const float f0 = __fmul_rn(__fmul_rn(dd, (float) s0_), 0.125f), f1 = __fmul_rn(__fmul_rn(dd, (float) s1_), 0.125f);
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
          if (ct < tiles) {
            // tokens the A operand, weight rows the B: D[token 4 quad + i][row col]
            const v4i I0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(bx[ct], a0, v4i{0, 0, 0, 0}, 0, 0, 0);
            const v4i I1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(bx[ct], a1, v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) {
              // token 4 quad + i's block scale, from the lane that loaded it (lane 4 quad + i: token col)
              const float xt = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * quad + i) * 4, __float_as_int(xs[ct])));
              const float sub = __fadd_rn(__fmul_rn(f0, (float) I0[i]), __fmul_rn(f1, (float) I1[i]));
              acc[c][ct][i] = __builtin_fmaf(xt, sub, acc[c][ct][i]);
            }
          }
        }
      }
    }
    // the tree's levels L/2 .. 4 within the wave: chains c and c ^ o4 (logical lanes ll and ll ^ 4 o4)
#pragma unroll
    for (int o4 = C / 2; o4 > 0; o4 >>= 1)
#pragma unroll
      for (int c = 0; c < o4; c++)
#pragma unroll
        for (int ct = 0; ct < CT; ct++)
#pragma unroll
          for (int i = 0; i < 4; i++) acc[c][ct][i] = __fadd_rn(acc[c][ct][i], acc[c + o4][ct][i]);
#pragma unroll
    for (int ct = 0; ct < CT; ct++)
#pragma unroll
      for (int i = 0; i < 4; i++) part[((wave * CT + ct) * 4 + i) * kWave + lane] = acc[0][ct][i];
    __syncthreads();
    // levels W/2 .. 1 across the waves (T_w: wave w's subtree, logical lanes w mod W): each pass pairs w with
    // w + o for w < o, as the tree pairs logical lanes ll and ll ^ o. the CT 4 outputs of a lane are shared out
    // over the waves: wave v finishes outputs v, v + W, ...
    {
      const uint32_t wv = CT * 4 * kWave;  // a wave's stride
      for (int oi = (int) wave; oi < CT * 4; oi += kWaves) {
        const int ct = oi / 4, i = oi % 4;
        const float* pp = part + (ct * 4 + i) * kWave + lane;
        float t[kWaves];
#pragma unroll
        for (int v = 0; v < kWaves; v++) t[v] = pp[v * wv];
#pragma unroll
        for (int o = kWaves / 2; o > 0; o >>= 1)
#pragma unroll
          for (int v = 0; v < o; v++) t[v] = __fadd_rn(t[v], t[v + o]);
        const uint32_t tk = c0 + ct * kTile + 4 * quad + i;  // (D: token 4 quad + i, row col)
        if (tk < n) y[(uint64_t) (r0 + tk) * ys + row0 + col] = t[0];
      }
    }
    __syncthreads();  // the partial trees read before the next pass writes them
  }
}

template <uint32_t T, int L, int CT, int W>
bool launch(const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n_mat, uint32_t rows,
            uint32_t cols, const int8_t* q, const float* d, float* y, uint32_t ys, hipStream_t s) {
  const Lds<T, CT, W> l((uint32_t) row_bytes<T>(cols));
  if (l.total > 160 * 1024) return false;
  auto k = kernel<T, L, CT, W>;
  if (l.total > 64 * 1024 &&
      hipFuncSetAttribute((const void*) k, hipFuncAttributeMaxDynamicSharedMemorySize, (int) l.total) != hipSuccess)
    return false;
  k<<<dim3(rows / kTile, n_mat), W * kWave, l.total, s>>>((const uint8_t* const*) w, cnt, xrow, cols, q, d, y, ys);
  return hipGetLastError() == hipSuccess;
}

template <uint32_t T>
bool by_lanes(const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n_mat, uint32_t max_cnt,
              uint32_t rows, uint32_t cols, const int8_t* q, const float* d, float* y, uint32_t ys, hipStream_t s) {
  if (cols % Block<T>::values) return false;
  (void) max_cnt;
  return cols >= 4096 ? launch<T, 32, kCT32, kW32>(w, cnt, xrow, n_mat, rows, cols, q, d, y, ys, s)
                      : launch<T, 16, kCT16, kW16>(w, cnt, xrow, n_mat, rows, cols, q, d, y, ys, s);
}

}  // namespace lgemm
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool osmos_lane_group(uint32_t type, const void* const* w, const int32_t* cnt, const int32_t* xrow,
                                         uint32_t n_mat, uint32_t max_cnt, uint32_t rows, uint32_t cols,
                                         const int8_t* q, const float* d, float* y, uint32_t ys, void* stream) {
  if (!w || !cnt || !xrow || !q || !d || !y || !n_mat || n_mat > 65535 || !max_cnt || max_cnt > OSMOS_LANE_MAX_TOKENS ||
      !rows || rows % lgemm::kTile || !cols || cols % 256 || ys < rows || (uint64_t) max_cnt * cols >= (1ull << 31))
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
