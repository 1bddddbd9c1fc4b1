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
// contract's group), so the epilogue applies per MFMA with no reassociation. a workgroup is 16 rows x up to CT tiles
// of 16 tokens; its 4 waves are the contract's 4 K partitions, their partial sums added in wave order through LDS.
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

template <int CT>
__global__ __launch_bounds__(kThreads) void q4k_kernel(const uint8_t* const* __restrict__ wt,
                                                       const int32_t* __restrict__ cnt, uint32_t cols,
                                                       const int8_t* __restrict__ x8, const float* __restrict__ dx,
                                                       const float* __restrict__ sx, const uint32_t* __restrict__ soff,
                                                       float* __restrict__ ya, const uint32_t* __restrict__ yoff,
                                                       uint32_t ys) {
  __shared__ float scl[kWaves][kGroups][2][kTile];     // a block's 16 rows' (d sc, dmin m) by group, a wave's own
  __shared__ float part[kWaves][CT][4][kWave];         // the partitions' sums, for the ordered total
  const uint32_t m = blockIdx.y, n = (uint32_t) cnt[m], row0 = blockIdx.x * kTile, c0 = blockIdx.z * kTile * CT;
  if (c0 >= n) return;  // the whole workgroup: no barrier is reached by part of it
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, col = lane % kTile, quad = lane / kTile;
  const uint32_t nb = cols / 256, groups = cols / MMQ_GROUP;
  const uint64_t rb = (uint64_t) nb * kBlockBytes;
  const uint8_t* w = wt[m] + (uint64_t) row0 * rb;
  const uint32_t s0 = soff[m] + c0;  // the first slot: a multiple of 16
  float* y = ya + yoff[m];
  const int live_tiles = (int) ((n - c0 + kTile - 1) / kTile), tiles = live_tiles < CT ? live_tiles : CT;
  float acc[CT][4];
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[ct][i] = 0.0f;
  const uint8_t* arow = w + (uint64_t) col * rb;  // this lane's A row
  for (uint32_t b = wave; b < nb; b += kWaves) {
    const uint8_t* blk = arow + (uint64_t) b * kBlockBytes;
    if (quad == 0) {  // lanes 0 .. 15: row col's header -> 8 groups' (d sc, dmin m)
      const uint4 hd = *(const uint4*) blk;
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
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll 1
    for (int gp = 0; gp < kGroups / 2; gp++) {
      // 8 bytes of this lane's row: codes 8 quad .. + 7 of groups 2 gp (low nibbles) and 2 gp + 1 (high)
      const uint2 raw = *(const uint2*) (blk + 16 + gp * 32 + 8 * quad);
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int g = 2 * gp + e;
        const uint32_t sh = 4u * (uint32_t) e;
        const uint2 av = {(raw.x >> sh) & 0x0F0F0F0Fu, (raw.y >> sh) & 0x0F0F0F0Fu};
        const long a = (long) (((uint64_t) av.y << 32) | av.x);
        const uint32_t gg = b * kGroups + (uint32_t) g;
        float ds[4], dm[4];
#pragma unroll
        for (int i = 0; i < 4; i++) ds[i] = scl[wave][g][0][4 * quad + i], dm[i] = scl[wave][g][1][4 * quad + i];
#pragma unroll
        for (int ct = 0; ct < CT; ct++) {
          if (ct < tiles) {
            const uint32_t slot = s0 + ct * kTile + col;
            const uint2 bv = *(const uint2*) (x8 + mmq_x8_at(slot, gg * MMQ_GROUP + 8 * quad, cols));
            const long bb = (long) (((uint64_t) bv.y << 32) | bv.x);
            const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bb, v4i{0, 0, 0, 0}, 0, 0, 0);
            const uint64_t at = mmq_dx_at(slot, gg, groups);
            const float dxt = dx[at], nsx = -sx[at];
#pragma unroll
            for (int i = 0; i < 4; i++) {
              const float v = __fmul_rn(ds[i], dxt);
              acc[ct][i] = __builtin_fmaf(v, (float) I[i], acc[ct][i]);
              acc[ct][i] = __builtin_fmaf(dm[i], nsx, acc[ct][i]);
            }
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();  // the block's table read before the next block's is written
  }
#pragma unroll
  for (int ct = 0; ct < CT; ct++)
#pragma unroll
    for (int i = 0; i < 4; i++) part[wave][ct][i][lane] = acc[ct][i];
  __syncthreads();
  if (wave) return;
#pragma unroll
  for (int ct = 0; ct < CT; ct++) {
    const uint32_t t = c0 + ct * kTile + col;
    if (ct < tiles && t < n)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float s = part[0][ct][i][lane];
#pragma unroll
        for (int p = 1; p < kWaves; p++) s = __fadd_rn(s, part[p][ct][i][lane]);
        y[(uint64_t) t * ys + row0 + 4 * quad + i] = s;
      }
  }
}

template <int CT>
bool q4k_launch(const void* const* w, const int32_t* cnt, uint32_t n_mat, uint32_t max_cnt, uint32_t rows,
                uint32_t cols, const int8_t* x8, const float* dx, const float* sx, const uint32_t* soff, float* y,
                const uint32_t* yoff, uint32_t ys, hipStream_t s) {
  const uint32_t z = (max_cnt + kTile * CT - 1) / (kTile * CT);
  q4k_kernel<CT><<<dim3(rows / kTile, n_mat, z), kThreads, 0, s>>>((const uint8_t* const*) w, cnt, cols, x8, dx, sx,
                                                                   soff, y, yoff, ys);
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
  if (max_cnt <= mmq::kTile) return mmq::q4k_launch<1>(w, cnt, n_mat, max_cnt, rows, cols, x8, dx, sx, soff, y, yoff, ys, s);
  if (max_cnt <= 2 * mmq::kTile)
    return mmq::q4k_launch<2>(w, cnt, n_mat, max_cnt, rows, cols, x8, dx, sx, soff, y, yoff, ys, s);
  return mmq::q4k_launch<MMQ_MAX_TILES>(w, cnt, n_mat, max_cnt, rows, cols, x8, dx, sx, soff, y, yoff, ys, s);
}
