// libosmos MI355X - the experts' matmul on the int8 matrix cores (include/osmos/gpu/mmq.h): mmq_x8_rows, mmq_group,
// mmq_known.
//
// contract (reference include/osmos/gpu/mmq.h:37-55, kernels/mmq.hip:33-151): activations int8 a 32-value group
// (dx = amax / 127, q = clamp(rint(x / dx)), sx = dx * sum q) in 16-slot tiles; Q4_K's 32-value group g of a weight row
// contributes (d sc) dx I - (dmin m) sx with I the group's exact integer dot, applied as v = (d sc) * dx;
// acc = fmaf(v, I, acc); acc = fmaf(dmin m, -sx, acc); K split into 4 partitions by 256-value block (partition p its
// blocks p, p + 4, ...), each its groups in order, then the partitions summed in order. every output the reference's
// bits, whatever the batch.
//
// CDNA4 mapping: one v_mfma_i32_16x16x32_i8 is exactly one group's 16 rows x 16 tokens of integer dots (K = 32 = the
// contract's group), so the epilogue applies per MFMA with no reassociation. a wave owns 16 rows and keeps the 4 K
// partitions' sums side by side in registers, for CT tiles of 16 tokens at a time, walking all of its expert's tiles;
// a workgroup is 4 such waves (64 rows) of one expert, so an expert with no tokens costs one empty workgroup a row
// block, not one a token tile.
// A operand: lane l holds row l % 16's 8 codes 8 (l / 16) .. + 7 of the group (one 64-bit load of packed nibbles for
// a pair of groups); B: token l % 16's 8 int8 at the same K (one 64-bit load from the slot tile); D: rows
// 4 (l / 16) + i, token l % 16.
#include "common.h"

extern "C" {
#include "../../include/osmos/gpu/mmq.h"
}

namespace osm {
namespace mmq {

constexpr int kWaves = 4;  // the contract's K partitions
constexpr int kThreads = kWave * kWaves, kTile = 16, kGroups = 8, kBlockBytes = 144;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // (native: stays in registers)

// a half-wave a group: its 32 values' max |x| and the codes' sum by the half-wave's tree (reference kernels/mmq.hip:33-52)
__global__ __launch_bounds__(256) void x8_rows_kernel(const float* __restrict__ x, uint32_t xs,
                                                      const int32_t* __restrict__ idx, uint32_t slots, uint32_t cols,
                                                      int8_t* __restrict__ x8, float* __restrict__ dx,
                                                      float* __restrict__ sx) {
  const uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t) slots * cols) return;  // whole groups: slots * cols a multiple of 32, a half-wave's
  const uint32_t s = (uint32_t) (i / cols), c = (uint32_t) (i % cols);
  const int32_t r = idx[s];
  const float v = r >= 0 ? x[(uint64_t) r * xs + c] : 0.0f;
  float a = fabsf(v);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
  const float d = __fdiv_rn(a, 127.0f);
  const int q = a == 0.0f ? 0 : (int) fminf(fmaxf(rintf(__fdiv_rn(v, d)), -127.0f), 127.0f);
  int sum = q;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 32);
  x8[mmq_x8_at(s, c, cols)] = (int8_t) q;
  if (c % MMQ_GROUP == 0) {
    const uint64_t g = mmq_dx_at(s, c / MMQ_GROUP, cols / MMQ_GROUP);
    const float dd = a == 0.0f ? 0.0f : d;
    dx[g] = dd;
    sx[g] = __fmul_rn(dd, (float) sum);
  }
}

// the same with 4 lanes a group, 8 values a lane (two 16-byte loads of the token's row, one 8-byte store): for x rows
// 16-aligned. each value's code and the group's dx / sx exactly as above (max and the integer sum in any order)
__global__ __launch_bounds__(256) void x8_rows8_kernel(const float* __restrict__ x, uint32_t xs,
                                                       const int32_t* __restrict__ idx, uint32_t slots, uint32_t cols,
                                                       int8_t* __restrict__ x8, float* __restrict__ dx,
                                                       float* __restrict__ sx) {
  const uint32_t groups = cols / MMQ_GROUP;
  const uint64_t gi = ((uint64_t) blockIdx.x * 256 + threadIdx.x) / 4, ng = (uint64_t) slots * groups;
  const uint32_t c8 = 8 * (threadIdx.x % 4);
  const uint64_t gc = gi < ng ? gi : ng - 1;  // (past the end: the last group again, nothing stored)
  const uint32_t s = (uint32_t) (gc / groups), g = (uint32_t) (gc % groups);
  const int32_t r = idx[s];
  float v[8];
  if (r >= 0) {
    const float4* src = (const float4*) (x + (uint64_t) r * xs + (uint64_t) g * MMQ_GROUP + c8);
    const float4 lo = src[0], hi = src[1];
    v[0] = lo.x, v[1] = lo.y, v[2] = lo.z, v[3] = lo.w, v[4] = hi.x, v[5] = hi.y, v[6] = hi.z, v[7] = hi.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = 0.0f;
  }
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) a = fmaxf(a, fabsf(v[i]));
  a = fmaxf(a, __shfl_xor(a, 1, 4));
  a = fmaxf(a, __shfl_xor(a, 2, 4));
  const float dd = __fdiv_rn(a, 127.0f);
  int sum = 0;
  uint64_t w = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int qv = a == 0.0f ? 0 : (int) fminf(fmaxf(rintf(__fdiv_rn(v[i], dd)), -127.0f), 127.0f);
    sum += qv;
    w |= (uint64_t) (uint8_t) (int8_t) qv << (8 * i);
  }
  sum += __shfl_xor(sum, 1, 4);
  sum += __shfl_xor(sum, 2, 4);
  if (gi < ng) {
    *(uint64_t*) (x8 + mmq_x8_at(s, g * MMQ_GROUP + c8, cols)) = w;
    if (c8 == 0) {
      const uint64_t at = mmq_dx_at(s, g, groups);
      const float d0 = a == 0.0f ? 0.0f : dd;
      dx[at] = d0;
      sx[at] = __fmul_rn(d0, (float) sum);
    }
  }
}

// a workgroup: 64 rows (a wave 16) of matrix blockIdx.y over all of its cnt tokens, CT tiles of 16 at a time. each
// wave keeps the 4 K partitions' sums side by side in registers (partition p the 256-blocks b with b % 4 == p, each
// partition's groups in ascending order, then the 4 sums added in order - the contract's). a block's activations
// for the CT tiles (x8 4 KB a tile, dx and sx 512 B a tile: contiguous in the slot layout) are staged in LDS by the
// whole workgroup, the next block's loads in flight while this one's MFMAs run; lanes 0 .. 15 of each wave write the
// block's per-row (d sc, dmin m) into the wave's table, which every lane reads for its 4 output rows
template <int CT>
__global__ __launch_bounds__(kThreads) void q4k_kernel(const uint8_t* const* __restrict__ wt,
                                                       const int32_t* __restrict__ cnt, uint32_t rows, uint32_t cols,
                                                       const int8_t* __restrict__ x8, const float* __restrict__ dx,
                                                       const float* __restrict__ sx, const uint32_t* __restrict__ soff,
                                                       float* __restrict__ ya, const uint32_t* __restrict__ yoff,
                                                       uint32_t ys) {
  constexpr uint32_t kX8Tile = kGroups * MMQ_SLOTS * MMQ_GROUP;  // a tile's block of x8: 4 KB
  constexpr uint32_t kDxTile = kGroups * MMQ_SLOTS;              // a tile's block of dx (or sx): 128 floats
  constexpr int kXPer = CT * kX8Tile / 16 / kThreads;            // 16-byte words of x8 a thread stages (1, 2, 4)
  constexpr int kDPer = (2 * CT * kDxTile + kThreads - 1) / kThreads;  // dx / sx values a thread stages
  __shared__ __attribute__((aligned(16))) int8_t xs8[CT * kX8Tile];
  __shared__ __attribute__((aligned(16))) float xds[2][CT * kDxTile];  // [0] dx, [1] sx
  __shared__ float scl[kWaves][kGroups][2][kTile];  // a block's 16 rows' (d sc, dmin m) by group, a wave's own
  const uint32_t m = blockIdx.y, n = (uint32_t) cnt[m];
  if (n <= blockIdx.z * kTile * CT) return;  // (the whole workgroup: no pass of its own)
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave, col = lane % kTile, quad = lane / kTile;
  const uint32_t row0 = blockIdx.x * kTile * kWaves + wave * kTile;
  const bool live_rows = row0 < rows;  // (a wave past the rows still stages and meets the barriers)
  const uint32_t nb = cols / 256, rb = nb * kBlockBytes, groups = cols / MMQ_GROUP;
  const uint8_t* arow = wt[m] + (uint64_t) (live_rows ? row0 + col : 0) * rb;  // this lane's A row
  float* y = ya + yoff[m];
  for (uint32_t c0 = blockIdx.z * kTile * CT; c0 < n; c0 += gridDim.z * kTile * CT) {  // (passes over blockIdx.z)
    const uint32_t s0 = soff[m] + c0;  // the pass's first slot: a multiple of 16
    const int live = (int) ((n - c0 + kTile - 1) / kTile), tiles = live < CT ? live : CT;
    // a block's activations for the live tiles, into registers
    u32x4 xr[kXPer];
    float dr[kDPer];
    auto load = [&](uint32_t b) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kXPer; u++) {
        const uint32_t wd = threadIdx.x + u * kThreads, ct = wd / (kX8Tile / 16), off = wd % (kX8Tile / 16);
        if ((int) ct < tiles)
          xr[u] = *(const u32x4*) (x8 + mmq_x8_at(s0 + ct * kTile, b * kGroups * MMQ_GROUP, cols) + off * 16);
      }
#pragma unroll
      for (int u = 0; u < kDPer; u++) {  // dx then sx, CT tiles each
        const uint32_t e = threadIdx.x + u * kThreads, which = e / (CT * kDxTile), f = e % (CT * kDxTile);
        if (which < 2 && (int) (f / kDxTile) < tiles)
          dr[u] = (which ? sx : dx)[mmq_dx_at(s0 + (f / kDxTile) * kTile, b * kGroups, groups) + f % kDxTile];
      }
    };
    auto store = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kXPer; u++) ((u32x4*) xs8)[threadIdx.x + u * kThreads] = xr[u];
#pragma unroll
      for (int u = 0; u < kDPer; u++) {
        const uint32_t e = threadIdx.x + u * kThreads, which = e / (CT * kDxTile), f = e % (CT * kDxTile);
        if (which < 2) xds[which][f] = dr[u];
      }
    };
    float acc[4][CT][4];
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
      for (int ct = 0; ct < CT; ct++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[p][ct][i] = 0.0f;
    // this lane's weights of a block: its row's codes 8 quad .. of the 4 group pairs, and (lanes 0 .. 15) its header
    u32x4 wa, wb, hd;
    auto wload = [&](uint32_t b) __attribute__((always_inline)) {
      const uint8_t* blk = arow + (uint64_t) b * kBlockBytes;
      const uint2 r0 = *(const uint2*) (blk + 16 + 8 * quad), r1 = *(const uint2*) (blk + 48 + 8 * quad);
      const uint2 r2 = *(const uint2*) (blk + 80 + 8 * quad), r3 = *(const uint2*) (blk + 112 + 8 * quad);
      wa = u32x4{r0.x, r0.y, r1.x, r1.y}, wb = u32x4{r2.x, r2.y, r3.x, r3.y};
      if (quad == 0) hd = *(const u32x4*) blk;
    };
    load(0);
    wload(0);
    for (uint32_t b0 = 0; b0 < nb; b0 += 4) {
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const uint32_t b = b0 + (uint32_t) p;
        if (b >= nb) break;  // (uniform)
        __syncthreads();  // the previous block's activations read by every wave
        store();
        const uint2 raw0 = {wa.x, wa.y}, raw1 = {wa.z, wa.w}, raw2 = {wb.x, wb.y}, raw3 = {wb.z, wb.w};
        const u32x4 hdc = hd;
        if (b + 1 < nb) load(b + 1), wload(b + 1);  // in flight during this block's MFMAs
        if (quad == 0) {  // lanes 0 .. 15: row col's header -> 8 groups' (d sc, dmin m)
          const u32x4 hd = hdc;
          const float d = f16(hd.x & 0xFFFF), dmin = f16(hd.x >> 16);
          const uint32_t sw[3] = {hd.y, hd.z, hd.w};
          auto sb = [&](int i) { return (int) ((sw[i / 4] >> (8 * (i % 4))) & 0xFF); };
#pragma unroll
          for (int g = 0; g < kGroups; g++) {
            const int sc = g < 4 ? sb(g) & 0x3F : (sb(g + 4) & 0x0F) | ((sb(g - 4) >> 2) & 0x30);
            const int mn = g < 4 ? sb(g + 4) & 0x3F : (sb(g + 4) >> 4) | ((sb(g) >> 2) & 0x30);
            scl[wave][g][0][col] = __fmul_rn(d, (float) sc);
            scl[wave][g][1][col] = __fmul_rn(dmin, (float) mn);
          }
        }
        __syncthreads();  // this block's activations and tables written
#pragma unroll
        for (int g = 0; g < kGroups; g++) {
          // this lane's 8 codes 8 quad .. + 7 of group g: nibbles (g % 2) of bytes 16 + 32 (g / 2) + 8 quad ..
          const uint2 raw = g / 2 == 0 ? raw0 : g / 2 == 1 ? raw1 : g / 2 == 2 ? raw2 : raw3;
          const uint32_t sh = 4u * (uint32_t) (g % 2);
          const long a = (long) (((uint64_t) ((raw.y >> sh) & 0x0F0F0F0Fu) << 32) | ((raw.x >> sh) & 0x0F0F0F0Fu));
          float ds[4], dm[4];
#pragma unroll
          for (int i = 0; i < 4; i++) ds[i] = scl[wave][g][0][4 * quad + i], dm[i] = scl[wave][g][1][4 * quad + i];
#pragma unroll
          for (int ct = 0; ct < CT; ct++) {
            if (ct < tiles) {
              const long bb = *(const long*) (xs8 + ct * kX8Tile + g * (MMQ_SLOTS * MMQ_GROUP) + col * MMQ_GROUP + 8 * quad);
              const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bb, v4i{0, 0, 0, 0}, 0, 0, 0);
              const float dxt = xds[0][ct * kDxTile + g * MMQ_SLOTS + col];
              const float nsx = -xds[1][ct * kDxTile + g * MMQ_SLOTS + col];
#pragma unroll
              for (int i = 0; i < 4; i++) {
                const float v = __fmul_rn(ds[i], dxt);
                acc[p][ct][i] = __builtin_fmaf(v, (float) I[i], acc[p][ct][i]);
                acc[p][ct][i] = __builtin_fmaf(dm[i], nsx, acc[p][ct][i]);
              }
            }
          }
        }
      }
    }
    __syncthreads();  // the last block's activations read before the next pass stages its own
    if (live_rows) {
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        const uint32_t t = c0 + ct * kTile + col;
        if (ct < tiles && t < n)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float s = __fadd_rn(__fadd_rn(__fadd_rn(acc[0][ct][i], acc[1][ct][i]), acc[2][ct][i]), acc[3][ct][i]);
            y[(uint64_t) t * ys + row0 + 4 * quad + i] = s;
          }
      }
    }
  }
}

// the token passes of a matrix spread over blockIdx.z: enough workgroups for the chip when few matrices hold many
// tokens (one expert at 512 tokens: 112 row blocks x 8), each workgroup a pass in every Z
template <int CT>
bool q4k_launch(const void* const* w, const int32_t* cnt, uint32_t n_mat, uint32_t max_cnt, uint32_t rows,
                uint32_t cols, const int8_t* x8, const float* dx, const float* sx, const uint32_t* soff, float* y,
                const uint32_t* yoff, uint32_t ys, hipStream_t s) {
  const uint32_t per = kTile * kWaves, bx = (rows + per - 1) / per, passes = (max_cnt + kTile * CT - 1) / (kTile * CT);
  uint32_t z = 1;
  while (z < passes && (uint64_t) bx * n_mat * z < 2048) z *= 2;  // (about 8 workgroups a CU at most)
  q4k_kernel<CT><<<dim3(bx, n_mat, min(z, passes)), kThreads, 0, s>>>((const uint8_t* const*) w, cnt, rows, cols,
                                                                        x8, dx, sx, soff, y, yoff, ys);
  return hipGetLastError() == hipSuccess;
}

}  // namespace mmq
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool mmq_known(uint32_t type) { return type == kQ4_K; }

extern "C" OSM_API bool mmq_x8_rows(const float* x, uint32_t xs, const int32_t* idx, uint32_t slots, uint32_t cols,
                                    int8_t* x8, float* dx, float* sx, void* stream) {
  if (!x || !idx || !x8 || !dx || !sx || !slots || !cols || cols % MMQ_GROUP || xs < cols) return false;
  const uint64_t work = (uint64_t) slots * cols;
  if ((uintptr_t) x % 16 == 0 && xs % 4 == 0 && (uintptr_t) x8 % 8 == 0) {  // (the vector form where it is aligned)
    mmq::x8_rows8_kernel<<<(unsigned) ((work / 8 + 255) / 256), 256, 0, (hipStream_t) stream>>>(x, xs, idx, slots, cols,
                                                                                                x8, dx, sx);
    return hipGetLastError() == hipSuccess;
  }
  mmq::x8_rows_kernel<<<(unsigned) ((work + 255) / 256), 256, 0, (hipStream_t) stream>>>(x, xs, idx, slots, cols, x8,
                                                                                          dx, sx);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool mmq_group(uint32_t type, const void* const* w, const int32_t* cnt, uint32_t n_mat,
                                  uint32_t max_cnt, uint32_t rows, uint32_t cols, const int8_t* x8, const float* dx,
                                  const float* sx, const uint32_t* soff, float* y, const uint32_t* yoff, uint32_t ys,
                                  void* stream) {
  if (!mmq_known(type) || !w || !cnt || !x8 || !dx || !sx || !soff || !y || !yoff || !n_mat || !max_cnt || !rows ||
      rows % mmq::kTile || !cols || cols % 256 || ys < rows)
    return false;
  const hipStream_t s = (hipStream_t) stream;
  // (at most 2 tiles a pass: 4 hold 186 VGPRs, occupancy 2, and run the batch-512 down 1.45x slower, the dense
  // 512-token expert 1.3x slower)
  if (max_cnt <= mmq::kTile)
    return mmq::q4k_launch<1>(w, cnt, n_mat, max_cnt, rows, cols, x8, dx, sx, soff, y, yoff, ys, s);
  return mmq::q4k_launch<2>(w, cnt, n_mat, max_cnt, rows, cols, x8, dx, sx, soff, y, yoff, ys, s);
}
