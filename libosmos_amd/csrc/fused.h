// libosmos MI355X - the routed layer's two fused kernels (osmos_lane_layer, layer.hip), bit for bit the lane
// contract's sums in the reference's layer order (src/cpu/lane.c:98-118, src/run/hip_lane.c:164-220):
//
// gu_kernel (gate/up): a workgroup is (an expert, a tile of 16 of its ff rows). its expert's first pick owns it: the
//   picks that chose the same expert (at most one a token) are its tokens, read once for all of them. it stages the
//   tile's gate and up rows in LDS with 16-byte loads (every load issued before any is waited on), copies the type's
//   codebook to LDS, rounds its tokens' x rows itself (q8_round's bits), then each row's lane sums, the tree and
//   lane_swiglu(gate, up, lim, w[pick]) into h[pick][row].
// dn_kernel (down): a workgroup is (a token, a tile of 8 of the dim rows). it rounds h of the token's k picks into LDS
//   (q8_round's bits), stages the k experts' tile rows, sums each (expert, row) in the lane order, then each row's k
//   sums in ascending expert id (the reference's ops_gather_sum_add order) and add[t][row] after.
#pragma once
#include "lanedec.h"

namespace osm {
namespace fused {

using namespace lane;

constexpr int kThreads = 256, kWaves = 4;
constexpr uint32_t kGuRows = 16, kDnRows = 8, kMaxTok = 64, kMaxK = 32;

__host__ __device__ constexpr uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

// gu_kernel's LDS: the gate and up tiles, NT tokens' int8 x and scales, the codebook, the expert's tokens
struct GuLds {
  uint32_t wg, wu, q, d, grid, toks, ids, total;
};
__host__ __device__ inline GuLds gu_lds(uint32_t row_bytes, uint32_t dim, int nt, uint32_t grid_bytes, uint32_t n) {
  GuLds l;
  uint32_t at = 0;
  l.wg = at, at += align16(kGuRows * row_bytes);
  l.wu = at, at += align16(kGuRows * row_bytes);
  l.q = at, at += align16((uint32_t) nt * dim);
  l.d = at, at += align16((uint32_t) nt * (dim / 32) * 4);
  l.grid = at, at += align16(grid_bytes);
  l.toks = at, at += align16((2 * kMaxTok + 1) * 4);
  l.ids = at, at += align16(n * 4);
  l.total = at;
  return l;
}

// dn_kernel's LDS: the k experts' tiles, the k rounded h rows and scales, the k row sums, the sorted picks
struct DnLds {
  uint32_t w, q, d, grid, ye, picks, total;
};
__host__ __device__ inline DnLds dn_lds(uint32_t row_bytes, uint32_t ff, uint32_t k, uint32_t grid_bytes) {
  DnLds l;
  uint32_t at = 0;
  l.w = at, at += align16(k * kDnRows * row_bytes);
  l.q = at, at += align16(k * ff);
  l.d = at, at += align16(k * (ff / 32) * 4);
  l.grid = at, at += align16(grid_bytes);
  l.ye = at, at += align16(k * kDnRows * 4);
  l.picks = at, at += align16(2 * kMaxK * 4);
  l.total = at;
  return l;
}

template <uint32_t T> constexpr uint32_t grid_bytes() { return (uint32_t) (GridOf<T>::n * sizeof(typename GridOf<T>::E)); }

struct GuArgs {
  const float* x;       // n_tok rows of dim
  const int32_t* ids;   // n_tok x k picks
  const float* w;       // their router weights
  uint32_t n_tok, k, dim, ff;
  const uint8_t *gate, *up;
  uint64_t gate_bytes, up_bytes;  // an expert's
  float lim;
  float* h;             // n_tok k rows of ff
};

struct DnArgs {
  const float* h;
  const int32_t* ids;
  uint32_t n_tok, k, dim, ff;
  const uint8_t* down;
  uint64_t down_bytes;
  const float* add;
  float* out;           // n_tok rows of dim
};

// a workgroup's copy of segments into LDS, in two halves so that other loads can be issued between them: load()
// issues every thread's 16-byte loads of the current round (up to kPer a thread: the weights of a tile fit one round),
// store() writes them to LDS. segment j (per_seg 16-byte words) comes from src(j) and lands at lds + j * per_seg * 16:
// the destination is the word's linear index, the source found by a reciprocal (exact: checked and corrected)
constexpr int kPer = 16;
struct Staged {
  uint4 v[kPer];
};
template <typename Src>
__device__ inline void stage_load(Staged& st, Src src, uint32_t n, uint32_t per_seg, float inv, uint32_t base) {
#pragma unroll
  for (int u = 0; u < kPer; u++) {
    const uint32_t l0 = base + u * kThreads + threadIdx.x, l = l0 < n ? l0 : 0;  // (past the end: word 0 again)
    uint32_t j = (uint32_t) ((float) l * inv);
    j -= j * per_seg > l;
    j += (j + 1) * per_seg <= l;
    st.v[u] = ((const uint4*) src(j))[l - j * per_seg];
  }
}
__device__ inline void stage_store(const Staged& st, uint8_t* lds, uint32_t n, uint32_t base) {
#pragma unroll
  for (int u = 0; u < kPer; u++) {
    const uint32_t l = base + u * kThreads + threadIdx.x;
    if (l < n) ((uint4*) lds)[l] = st.v[u];
  }
}

// rows of 32-value blocks rounded to int8 as q8_round rounds them (reference kernels/q8.h:263-277): 8 threads a
// block, 4 values (a float4) each; the block's max |x| by a 3-step xor exchange among the 8 (max is exact in any
// order), each value's code, the 4 codes one word. round_load() issues a round of up to kRPer float4 loads a thread
// (block base + threadIdx.x / 8 + 32 u), round_store() reduces and writes them; value(blk, c) is the address of block
// blk's value c
constexpr int kRPer = 8;
constexpr uint32_t kRoundBlocks = (kThreads / 8) * kRPer;  // blocks a round
struct Rounded {
  float4 v[kRPer];
};
template <typename Val>
__device__ inline void round_load(Rounded& r, Val value, uint32_t blocks, uint32_t base) {
  const uint32_t g = threadIdx.x / 8, c = 4 * (threadIdx.x % 8);
#pragma unroll
  for (int u = 0; u < kRPer; u++) {
    const uint32_t blk = base + g + (kThreads / 8) * u;
    r.v[u] = *(const float4*) value(blk < blocks ? blk : 0, c);
  }
}
__device__ inline uint32_t q8_byte(float v, float inv) { return (uint32_t) ((int) rintf(__fmul_rn(v, inv)) & 0xFF); }
__device__ inline void round_store(const Rounded& r, uint32_t blocks, uint32_t base, uint32_t nb_row, uint32_t cols,
                                   int8_t* q, float* d) {
  const uint32_t g = threadIdx.x / 8, c = 4 * (threadIdx.x % 8);
#pragma unroll
  for (int u = 0; u < kRPer; u++) {
    const uint32_t blk = base + g + (kThreads / 8) * u;
    const float4 v = r.v[u];
    float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    am = fmaxf(am, xor_lane(am, 1));
    am = fmaxf(am, xor_lane(am, 2));
    am = fmaxf(am, xor_lane(am, 4));
    if (blk < blocks) {
      const float inv = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
      const uint32_t row = blk / nb_row, s = blk % nb_row;
      *(uint32_t*) (q + row * cols + s * 32 + c) =
          q8_byte(v.x, inv) | q8_byte(v.y, inv) << 8 | q8_byte(v.z, inv) << 16 | q8_byte(v.w, inv) << 24;
      if (c == 0) d[blk] = __fdiv_rn(am, 127.0f);
    }
  }
}


// the codebook, copied by the first threads of a workgroup (1 - 16 KB of constant memory, 16-aligned)
template <uint32_t T>
__device__ inline void grid_copy(uint8_t* lds) {
  if constexpr (grid_bytes<T>() > 0) {
    constexpr uint32_t n = grid_bytes<T>() / 16;
    const uint4* src = (const uint4*) const_grid<T>();
    uint4 v[(n + kThreads - 1) / kThreads];
#pragma unroll
    for (uint32_t u = 0; u < (n + kThreads - 1) / kThreads; u++) {
      const uint32_t l = u * kThreads + threadIdx.x;
      v[u] = src[l < n ? l : 0];
    }
#pragma unroll
    for (uint32_t u = 0; u < (n + kThreads - 1) / kThreads; u++) {
      const uint32_t l = u * kThreads + threadIdx.x;
      if (l < n) ((uint4*) lds)[l] = v[u];
    }
  }
}

template <uint32_t T, int NT, int L>
__global__ __launch_bounds__(kThreads) void gu_kernel(GuArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr uint32_t per = Block<T>::values / 32, bb = Block<T>::bytes;
  const uint32_t m = blockIdx.y, r0 = blockIdx.x * kGuRows, n = a.n_tok * a.k;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.dim), nblk = a.dim / 32;
  const GuLds L_ = gu_lds(rb, a.dim, NT, grid_bytes<T>(), n);
  int32_t* ids = (int32_t*) (smem + L_.ids);
  int32_t* toks = (int32_t*) (smem + L_.toks);  // [0, kMaxTok): the expert's picks in token order; [kMaxTok + t]:
                                                 // token t's pick of it or -1; [2 kMaxTok]: their count
  for (uint32_t i = threadIdx.x; i < n; i += kThreads) ids[i] = a.ids[i];
  __syncthreads();
  const int32_t e = ids[m];
  // the expert's first pick owns the workgroup; the others leave (the same decision in every thread)
  int dup = 0;
  for (uint32_t j = threadIdx.x; j < m; j += kThreads) dup |= ids[j] == e;
  if (__syncthreads_or(dup)) return;
  if (threadIdx.x < kWave) {  // wave 0, a lane a token: its pick of this expert if any (a token's picks are distinct
                              // experts), placed by the count of earlier tokens that picked it (token order)
    int32_t p = -1;
    if (threadIdx.x < a.n_tok)
      for (uint32_t j = 0; j < a.k; j++)
        if (ids[threadIdx.x * a.k + j] == e) p = (int32_t) (threadIdx.x * a.k + j);
    const uint64_t has = __ballot(p >= 0);
    if (p >= 0) toks[__builtin_popcountll(has & ((1ull << threadIdx.x) - 1))] = p;
    if (threadIdx.x == 0) toks[2 * kMaxTok] = __builtin_popcountll(has);
  }
  __syncthreads();
  const int cnt = toks[2 * kMaxTok];
  int8_t* q = (int8_t*) (smem + L_.q);
  float* d = (float*) (smem + L_.d);
  // one round of loads: the tile's gate and up rows (contiguous in each tensor), the codebook, the first chunk's x
  const uint8_t* gsrc = a.gate + (uint64_t) e * a.gate_bytes + (uint64_t) r0 * rb;
  const uint8_t* usrc = a.up + (uint64_t) e * a.up_bytes + (uint64_t) r0 * rb;
  const uint32_t per_seg = kGuRows * rb / 16, nw = 2 * per_seg;
  const float inv_seg = 1.0f / (float) per_seg;
  auto wsrc = [=](uint32_t j) { return j ? usrc : gsrc; };
  const int live0 = cnt < NT ? cnt : NT;
  auto xval = [&](int live, int c0) {
    return [=](uint32_t blk, uint32_t i) {
      const uint32_t r = blk / nblk, tk = (uint32_t) toks[c0 + ((int) r < live ? (int) r : live - 1)] / a.k;
      return a.x + (uint64_t) tk * a.dim + (blk % nblk) * 32 + i;
    };
  };
  const uint32_t xblocks = NT * nblk;
  {
    Staged st;
    Rounded rx;
    stage_load(st, wsrc, nw, per_seg, inv_seg, 0);
    round_load(rx, xval(live0, 0), xblocks, 0);
    grid_copy<T>(smem + L_.grid);
    stage_store(st, smem + L_.wg, nw, 0);
    round_store(rx, xblocks, 0, nblk, a.dim, q, d);
    for (uint32_t base = kPer * kThreads; base < nw; base += kPer * kThreads) {  // (tiles past one round)
      stage_load(st, wsrc, nw, per_seg, inv_seg, base);
      stage_store(st, smem + L_.wg, nw, base);
    }
    for (uint32_t base = kRoundBlocks; base < xblocks; base += kRoundBlocks) {
      round_load(rx, xval(live0, 0), xblocks, base);
      round_store(rx, xblocks, base, nblk, a.dim, q, d);
    }
  }
  __syncthreads();
  const auto* grid = (const typename GridOf<T>::E*) (smem + L_.grid);
  const int lane = threadIdx.x % kWave, ll = lane % L, wave = threadIdx.x / kWave;
  constexpr int G = kWave / L, passes = (int) kGuRows / (kWaves * G);
  for (int c0 = 0; c0 < cnt; c0 += NT) {
    const int live = cnt - c0 < NT ? cnt - c0 : NT;
    if (c0) {  // the next chunk's x (the previous chunk's read first)
      __syncthreads();
      Rounded rx;
      for (uint32_t base = 0; base < xblocks; base += kRoundBlocks) {
        round_load(rx, xval(live, c0), xblocks, base);
        round_store(rx, xblocks, base, nblk, a.dim, q, d);
      }
      __syncthreads();
    }
#pragma unroll
    for (int p = 0; p < passes; p++) {
      const uint32_t row = (uint32_t) (p * kWaves * G + wave * G + lane / L);
      const uint8_t *rg = smem + L_.wg + row * rb, *ru = smem + L_.wu + row * rb;
      float ag[NT], au[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) ag[t] = au[t] = 0.0f;
#pragma unroll 4
      for (uint32_t s = ll; s < nblk; s += L) {
        Codes cg, cu;
        const uint32_t at = (s / per) * bb;
        codes<T>(rg + at, (int) (s % per), cg, grid);
        codes<T>(ru + at, (int) (s % per), cu, grid);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          int x[8];
          const int4* xp = (const int4*) (q + t * a.dim + s * 32);
          const int4 x0 = xp[0], x1 = xp[1];
          x[0] = x0.x, x[1] = x0.y, x[2] = x0.z, x[3] = x0.w, x[4] = x1.x, x[5] = x1.y, x[6] = x1.z, x[7] = x1.w;
          const float xd = d[t * nblk + s];
          ag[t] = __builtin_fmaf(xd, block_sum<T>(cg, x), ag[t]);
          au[t] = __builtin_fmaf(xd, block_sum<T>(cu, x), au[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const float vg = tree<L>(ag[t]), vu = tree<L>(au[t]);
        if (ll == 0 && t < live) {
          const int pk = toks[c0 + t];
          a.h[(uint64_t) pk * a.ff + r0 + row] = lane_swiglu(vg, vu, a.lim, a.w[pk]);
        }
      }
    }
  }
}

template <uint32_t T, int L>
__global__ __launch_bounds__(kThreads) void dn_kernel(DnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr uint32_t per = Block<T>::values / 32, bb = Block<T>::bytes;
  const uint32_t t = blockIdx.y, r0 = blockIdx.x * kDnRows, K = a.k;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.ff), nblk = a.ff / 32;
  const DnLds L_ = dn_lds(rb, a.ff, K, grid_bytes<T>());
  int32_t* picks = (int32_t*) (smem + L_.picks);  // [j]: the token's pick at sorted place j; [kMaxK + j]: its expert
  if (threadIdx.x < kWave) {  // wave 0, a lane a pick: its place in ascending expert id (then pick) by its rank
    const uint32_t j = threadIdx.x;
    const int32_t ex = j < K ? a.ids[t * K + j] : INT32_MAX;
    uint32_t rank = 0;
    for (uint32_t i = 0; i < K; i++) {
      const int32_t o = __shfl(ex, (int) i, kWave);
      rank += o < ex || (o == ex && i < j);
    }
    if (j < K) picks[rank] = (int32_t) (t * K + j), picks[kMaxK + rank] = ex;
  }
  __syncthreads();
  int8_t* q = (int8_t*) (smem + L_.q);
  float* d = (float*) (smem + L_.d);
  // one round of loads: the k experts' tile rows, the codebook, the k picks' activations
  const uint8_t* down = a.down + (uint64_t) r0 * rb;
  const uint64_t db = a.down_bytes;
  const uint32_t per_seg = kDnRows * rb / 16, nw = K * per_seg;
  const float inv_seg = 1.0f / (float) per_seg;
  auto wsrc = [=](uint32_t j) { return down + (uint64_t) picks[kMaxK + j] * db; };
  auto hval = [=](uint32_t blk, uint32_t i) { return a.h + (uint64_t) picks[blk / nblk] * a.ff + (blk % nblk) * 32 + i; };
  const uint32_t hblocks = K * nblk;
  {
    Staged st;
    Rounded rh;
    stage_load(st, wsrc, nw, per_seg, inv_seg, 0);
    round_load(rh, hval, hblocks, 0);
    grid_copy<T>(smem + L_.grid);
    stage_store(st, smem + L_.w, nw, 0);
    round_store(rh, hblocks, 0, nblk, a.ff, q, d);
    for (uint32_t base = kPer * kThreads; base < nw; base += kPer * kThreads) {
      stage_load(st, wsrc, nw, per_seg, inv_seg, base);
      stage_store(st, smem + L_.w, nw, base);
    }
    for (uint32_t base = kRoundBlocks; base < hblocks; base += kRoundBlocks) {
      round_load(rh, hval, hblocks, base);
      round_store(rh, hblocks, base, nblk, a.ff, q, d);
    }
  }
  __syncthreads();
  const auto* grid = (const typename GridOf<T>::E*) (smem + L_.grid);
  float* ye = (float*) (smem + L_.ye);
  const int lane = threadIdx.x % kWave, ll = lane % L, wave = threadIdx.x / kWave;
  constexpr int G = kWave / L, groups = (int) kDnRows / G;  // row groups a tile: a wave's G rows each
  for (uint32_t u = wave; u < K * groups; u += kWaves) {
    const uint32_t j = u / groups, row = (u % groups) * G + lane / L;
    const uint8_t* wr = smem + L_.w + (j * kDnRows + row) * rb;
    float acc = 0.0f;
#pragma unroll 4
    for (uint32_t s = ll; s < nblk; s += L) {
      Codes c;
      codes<T>(wr + (s / per) * bb, (int) (s % per), c, grid);
      int x[8];
      const int4* xp = (const int4*) (q + j * a.ff + s * 32);
      const int4 x0 = xp[0], x1 = xp[1];
      x[0] = x0.x, x[1] = x0.y, x[2] = x0.z, x[3] = x0.w, x[4] = x1.x, x[5] = x1.y, x[6] = x1.z, x[7] = x1.w;
      acc = __builtin_fmaf(d[j * nblk + s], block_sum<T>(c, x), acc);
    }
    const float v = tree<L>(acc);
    if (ll == 0) ye[j * kDnRows + row] = v;
  }
  __syncthreads();
  if (threadIdx.x < kDnRows) {
    float s = 0.0f;
    for (uint32_t j = 0; j < K; j++) s = __fadd_rn(s, ye[j * kDnRows + threadIdx.x]);
    const uint64_t o = (uint64_t) t * a.dim + r0 + threadIdx.x;
    a.out[o] = __fadd_rn(s, a.add[o]);
  }
}

}  // namespace fused
}  // namespace osm
