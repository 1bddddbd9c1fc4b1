// libosmos MI355X - the MoE plumbing around the expert products: the Qwen-style routing, expert tables and weighted
// sum (include/osmos/gpu/q4x_ops.h), the lane's element-wise ops (include/osmos/gpu/ops.h) and the lane's step tables
// built on the device (include/osmos_mi355x.h: osmos_lane_tables).
//
// contracts: reference include/osmos/gpu/q4x_ops.h:356-384 and kernels/q4x_moe.hip:38-200 (route: softmax, the k
// greatest, the lowest id among equals, weights over max(sum, 6.103515625e-5); tiles: picks sorted by expert then pick,
// slots in whole tiles of 16, parts of at most 128 tokens in runs of 1/2/4/8 tiles; the sum: picks in order, then the
// sigmoid-gated shared expert), reference include/osmos/gpu/ops.h:311-355 and kernels/ops.hip:502-525 (swiglu_lane,
// gather_rows, gather_sum_add), reference src/run/hip_lane.c:115-200 (the lane's entries and token order).
#include <atomic>
#include <map>
#include <mutex>
#include <utility>

#include "common.h"

#include "x16.h"

extern "C" {
#include "../../include/osmos_mi355x.h"
}

namespace osm {
namespace moe {

constexpr uint32_t kMaxExperts = 1024, kMaxK = 32;
constexpr float kSumFloor = 6.103515625e-5f;
constexpr int kTile = 16, kPart = kTile << (Q4X_TILE_RUNS - 1);  // 128: an entry's most tokens

__device__ inline float sigmoid(float x) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-x))); }
__device__ inline float silu(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, expf(-x))); }  // (kernels/block.h:87)

// ---- q4x_route: a workgroup a token. the softmax by workgroup trees; the picks by a sort: each expert becomes one
// 64-bit key (its probability's order-preserving bits above, its id inverted below, so a greater probability and then
// a lower id sort first; NaN ranks as -inf, below every number), the token's keys are sorted descending by a bitonic
// network in LDS, and the first k are the picks in order ----
constexpr int kRouteThreads = 512;

__device__ inline float wg_reduce(float v, float* lds, bool is_max) {
  lds[threadIdx.x] = v;
  __syncthreads();
  for (int s = kRouteThreads / 2; s > 0; s >>= 1) {
    if ((int) threadIdx.x < s)
      lds[threadIdx.x] = is_max ? fmaxf(lds[threadIdx.x], lds[threadIdx.x + s]) : __fadd_rn(lds[threadIdx.x], lds[threadIdx.x + s]);
    __syncthreads();
  }
  const float r = lds[0];
  __syncthreads();
  return r;
}

// the sort key of expert e with probability p (a softmax output: +0 .. 1, or NaN); 0 for a slot past the experts
__device__ inline uint64_t route_key(float p, uint32_t e, uint32_t n_exp) {
  if (e >= n_exp) return 0;
  const uint32_t rank = p == p ? (__float_as_uint(p) & 0x7FFFFFFFu) + 1u : 0u;  // (NaN: -inf's rank, under +0's)
  return (uint64_t) rank << 32 | (0xFFFFFFFFu - e);
}
__device__ inline float key_value(uint64_t key) {  // the pick's probability as the weights take it (NaN: -inf)
  const uint32_t rank = (uint32_t) (key >> 32);
  return rank ? __uint_as_float(rank - 1u) : -__builtin_inff();
}

__global__ __launch_bounds__(kRouteThreads) void route_kernel(const float* __restrict__ logits, uint32_t n_exp,
                                                              uint32_t k, int32_t* __restrict__ ids,
                                                              float* __restrict__ w, int32_t* __restrict__ rows) {
  __shared__ float p[kMaxExperts], lds[kRouteThreads];
  __shared__ uint64_t key[kMaxExperts];
  const uint32_t t = blockIdx.x;
  const float* l = logits + (uint64_t) t * n_exp;
  float m = -__builtin_inff();
  for (uint32_t i = threadIdx.x; i < n_exp; i += kRouteThreads) m = fmaxf(m, l[i]);
  m = wg_reduce(m, lds, true);
  float sum = 0.0f;
  for (uint32_t i = threadIdx.x; i < n_exp; i += kRouteThreads) sum = __fadd_rn(sum, (p[i] = expf(__fsub_rn(l[i], m))));
  const float inv = __fdiv_rn(1.0f, wg_reduce(sum, lds, false));
  for (uint32_t i = threadIdx.x; i < kMaxExperts; i += kRouteThreads)
    key[i] = route_key(i < n_exp ? __fmul_rn(p[i], inv) : 0.0f, i, n_exp);
  __syncthreads();
  // bitonic sort, descending, over the smallest power of two holding the experts: stage (size, dist) compares i with
  // i ^ dist, the pair's order descending where bit `size` of i is clear
  uint32_t n2 = 1;
  while (n2 < n_exp) n2 <<= 1;
  for (uint32_t size = 2; size <= n2; size <<= 1)
    for (uint32_t dist = size >> 1; dist > 0; dist >>= 1) {
      for (uint32_t i = threadIdx.x; i < n2; i += kRouteThreads) {
        const uint32_t j = i ^ dist;
        if (j > i) {
          const uint64_t a = key[i], b = key[j];
          const bool down = (i & size) == 0;
          if (down ? a < b : a > b) key[i] = b, key[j] = a;
        }
      }
      __syncthreads();
    }
  if (threadIdx.x == 0) {  // the picks in order, their weights over max(their sum, the floor)
    float total = 0.0f;
    for (uint32_t j = 0; j < k; j++) total = __fadd_rn(total, key_value(key[j]));
    const float div = fmaxf(total, kSumFloor);
    for (uint32_t j = 0; j < k; j++) w[t * k + j] = __fdiv_rn(key_value(key[j]), div);
  }
  for (uint32_t j = threadIdx.x; j < k; j += kRouteThreads)
    ids[t * k + j] = (int32_t) (0xFFFFFFFFu - (uint32_t) key[j]), rows[t * k + j] = (int32_t) t;
}

// ---- q4x_expert_tiles ----
// One workgroup builds the tables in three passes, each over the outputs it writes:
//   1. per-expert figures: a count histogram, then one record per expert - its places (its picks), its slots (picks
//      rounded up to tiles of 16) and its entries in each of the Q4X_TILE_RUNS runs - prefix-summed by a two-level
//      wave scan (a wave's 64 experts by cross-lane shifts, then the 16 waves' totals by one wave);
//   2. entry-major: every entry index of every run, up to the run's bound, is one thread's; it finds its expert by a
//      binary search over that run's prefix, works out which part of the expert it is, and writes the part (or cnt 0
//      past the run's live entries);
//   3. slot-major: every slot index up to the slot bound is one thread's; padding slots (past an expert's picks or
//      past the last expert's tiles) get -1. The live slots are written by the pick placement: with n <= 1024 picks,
//      in this workgroup, each pick ranking itself among the earlier picks of its expert; beyond that, by
//      place_kernel (a workgroup an expert).
constexpr int kTileThreads = 1024, kTileWaves = kTileThreads / kWave, kRecs = 2 + Q4X_TILE_RUNS;
constexpr uint32_t kPlaceInline = 1024;

// which run a part of m tokens (1 .. kPart) belongs to: tiles of 1, 2, 4 or 8
__device__ inline int part_run(int m) { return m > 64 ? 3 : m > 32 ? 2 : m > 16 ? 1 : 0; }

// expert record field f for an expert of c picks
__device__ inline int rec_field(int c, int f) {
  if (f == 0) return c;
  if (f == 1) return (c + kTile - 1) & ~(kTile - 1);
  const int full = c / kPart, tail = c - full * kPart, r = f - 2;
  int n = tail && part_run(tail) == r;
  if (r == Q4X_TILE_RUNS - 1) n += full;
  return n;
}

// index of the first element of the ascending inclusive prefix `inc[0 .. n)` that exceeds v
__device__ inline int first_above(const int* inc, int n, int v) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (inc[mid] > v) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

__global__ __launch_bounds__(kTileThreads) void tiles_kernel(const int32_t* __restrict__ ids, uint32_t n, uint32_t k,
                                                             uint32_t n_exp, uint32_t dim, uint32_t ff,
                                                             Q4xExpertTiles t, Q4xExpertBounds bd) {
  __shared__ int hist[kMaxExperts];
  __shared__ int inc[kRecs][kMaxExperts];  // inclusive prefix of each record field over experts
  __shared__ int wsum[kRecs][kTileWaves];
  __shared__ int pick_id[kPlaceInline];
  const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
  hist[tid] = 0;
  __syncthreads();
  const bool inline_place = n <= kPlaceInline;
  for (uint32_t i = tid; i < n; i += kTileThreads) {
    const int e = ids[i];
    if (inline_place) pick_id[i] = e;
    atomicAdd(&hist[e], 1);
  }
  __syncthreads();

  // pass 1: thread tid is expert tid (experts past n_exp count 0)
  const int c = hist[tid];
  int v[kRecs];
#pragma unroll
  for (int f = 0; f < kRecs; f++) {
    v[f] = rec_field(c, f);
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_up(v[f], d, kWave);
      if (lane >= d) v[f] += o;
    }
    if (lane == kWave - 1) wsum[f][wave] = v[f];
  }
  __syncthreads();
  if (wave == 0) {  // the waves' totals, exclusive, in place
#pragma unroll
    for (int f = 0; f < kRecs; f++) {
      const int s = lane < kTileWaves ? wsum[f][lane] : 0;
      int x = s;
#pragma unroll
      for (int d = 1; d < kTileWaves; d <<= 1) {
        const int o = __shfl_up(x, d, kWave);
        if (lane >= d) x += o;
      }
      if (lane < kTileWaves) wsum[f][lane] = x - s;
    }
  }
  __syncthreads();
#pragma unroll
  for (int f = 0; f < kRecs; f++) inc[f][tid] = v[f] + wsum[f][wave];
  __syncthreads();

  const int place0 = inc[0][tid] - c, slot0 = inc[1][tid] - rec_field(c, 1);
  if ((uint32_t) tid < n_exp) t.off[tid] = place0, t.off[n_exp + tid] = slot0, t.off[2 * n_exp + tid] = c;

  // pass 2: entries
  for (int r = 0; r < Q4X_TILE_RUNS; r++) {
    const int live = inc[2 + r][kMaxExperts - 1];
    for (uint32_t i = tid; i < bd.count[r]; i += kTileThreads) {
      const uint32_t en = bd.first[r] + i;
      if ((int) i >= live) {
        t.cnt[en] = 0;
        continue;
      }
      const int e = first_above(inc[2 + r], kMaxExperts, (int) i);
      const int ce = hist[e], li = (int) i - (inc[2 + r][e] - rec_field(ce, 2 + r));
      const int part = r == Q4X_TILE_RUNS - 1 ? li : ce / kPart;  // runs 0-2 hold only an expert's short last part
      const int m = min(kPart, ce - part * kPart);
      const uint32_t slot = (uint32_t) (inc[1][e] - rec_field(ce, 1) + part * kPart);
      const uint32_t place = (uint32_t) (inc[0][e] - ce + part * kPart);
      t.cnt[en] = m;
      t.xg[en] = slot * dim, t.xd[en] = slot * ff, t.yg[en] = place * ff, t.yd[en] = place * dim;
      for (int j = 0; j < Q4X_GROUP_TENSORS; j++) {
        const void* mat = t.tab[j] ? (const void*) t.tab[j][e] : (const void*) ((const uint8_t*) t.base[j] + (uint64_t) e * t.bytes[j]);
        t.ptr[j][en] = mat;
      }
    }
  }

  // pass 3: padding slots
  const int live_slots = inc[1][kMaxExperts - 1];
  for (uint32_t s = tid; s < bd.slots; s += kTileThreads) {
    bool pad = (int) s >= live_slots;
    if (!pad) {
      const int e = first_above(inc[1], kMaxExperts, (int) s);
      pad = (int) s - (inc[1][e] - rec_field(hist[e], 1)) >= hist[e];
    }
    if (pad) t.gidx[s] = -1, t.hidx[s] = -1;
  }

  // the placement of small steps: pick i's place is its expert's first plus the earlier picks of that expert
  if (inline_place)
    for (uint32_t i = tid; i < n; i += kTileThreads) {
      const int e = pick_id[i];
      int before = 0;
      for (uint32_t j = 0; j < i; j++) before += pick_id[j] == e;
      const int q = inc[0][e] - hist[e] + before;
      const int s = inc[1][e] - rec_field(hist[e], 1) + before;
      t.where[i] = q, t.gidx[s] = (int32_t) (i / k), t.hidx[s] = q;
    }
}

// a workgroup an expert: its picks placed in pick order, a tile of 256 picks at a time (a wave's ballot prefix, then
// the waves' counts in order)
constexpr int kPlaceThreads = 256;
__global__ __launch_bounds__(kPlaceThreads) void place_kernel(const int32_t* __restrict__ ids, uint32_t n, uint32_t k,
                                                              uint32_t n_exp, Q4xExpertTiles t) {
  __shared__ int wave_cnt[kPlaceThreads / kWave];
  const uint32_t e = blockIdx.x;
  const int c = t.off[2 * n_exp + e];
  if (!c) return;
  const int p0 = t.off[e], s0 = t.off[n_exp + e];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int done = 0;
  for (uint32_t i0 = 0; i0 < n && done < c; i0 += kPlaceThreads) {
    const uint32_t i = i0 + threadIdx.x;
    const bool f = i < n && ids[i] == (int32_t) e;
    const uint64_t mask = __ballot(f);
    const int before = __builtin_popcountll(mask & ((1ull << lane) - 1));
    if (lane == 0) wave_cnt[wave] = __builtin_popcountll(mask);
    __syncthreads();
    int base = done;
    for (int v = 0; v < wave; v++) base += wave_cnt[v];
    if (f) {
      const int q = p0 + base + before;
      t.where[i] = q, t.gidx[s0 + q - p0] = (int32_t) (i / k), t.hidx[s0 + q - p0] = q;
    }
    for (int v = 0; v < kPlaceThreads / kWave; v++) done += wave_cnt[v];
    __syncthreads();
  }
}

// ---- q4x_moe_sum (kernels/q4x_moe.hip:172-180): each value its own products and sums, in pick order ----
__global__ __launch_bounds__(256) void moe_sum_kernel(const float* __restrict__ y, const int32_t* __restrict__ where,
                                                      const float* __restrict__ w, uint32_t n_tok, uint32_t k,
                                                      uint32_t dim, const float* __restrict__ shared,
                                                      const float* __restrict__ shared_logit, float* __restrict__ out) {
  const uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t) n_tok * dim) return;
  const uint64_t t = i / dim, d = i % dim;
  float sum = 0.0f;
  for (uint32_t j = 0; j < k; j++) sum = __fadd_rn(sum, __fmul_rn(y[(uint64_t) where[t * k + j] * dim + d], w[t * k + j]));
  out[i] = __fadd_rn(sum, __fmul_rn(shared[i], sigmoid(shared_logit[t])));
}

// ---- q4x_swiglu (kernels/q4x_moe.hip:167-170): a thread 4 values, each silu(g) u (swiglu_rows_kernel's expression),
// and, with a side output, its f16 at its (row, column) of the tiled x16 ----
struct Side {
  _Float16* x16;
  int32_t* overflow;
  uint32_t cols, row0;
};
__global__ __launch_bounds__(256) void swiglu_kernel(const float* g, const float* u, uint64_t n, float* y, Side side) {
  const uint64_t i0 = ((uint64_t) blockIdx.x * 256 + threadIdx.x) * 4;
  bool over = false;
#pragma unroll
  for (uint64_t i = i0; i < i0 + 4; i++) {
    if (i >= n) break;
    const float v = __fmul_rn(silu(g[i]), u[i]);
    y[i] = v;
    if (side.x16) side.x16[x16_at(side.row0 + (uint32_t) (i / side.cols), (uint32_t) (i % side.cols), side.cols)] = x16_round(v, over);
  }
  if (over) *side.overflow = 1;
}

// ---- q4x_spin: one thread sleeping until the constant-rate clock has moved on by `ticks` ----
__global__ __launch_bounds__(64) void spin_kernel(uint64_t ticks) {
  if (threadIdx.x) return;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
}

// ---- ops ----
__global__ __launch_bounds__(256) void swiglu_lane_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                          uint32_t n, float lim, const float* __restrict__ scale,
                                                          uint32_t n_tok, float* __restrict__ h) {
  const uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t) n * n_tok) return;
  h[i] = lane_swiglu(g[i], u[i], lim, scale[i / n]);
}

__global__ __launch_bounds__(256) void gather_rows_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                          const int32_t* __restrict__ idx, uint32_t n, uint32_t len) {
  const uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x;
  if (i < (uint64_t) n * len) dst[i] = src[(uint64_t) idx[i / len] * len + i % len];
}

// the stream held until *flag (host memory the GPU maps) holds value, with or without its top bit (the host's mark of
// a failed job) - one thread polling it with system-scope acquire loads (vector loads: never the scalar cache, which
// would not see the host's store), a short sleep (2 x 64 clocks) between polls. the wait is bounded by the wall clock
// (s_memrealtime's 100 MHz counter; the reference waits without bound, kernels/ops.hip:878-882): past `limit` ticks it
// gives up. Its outcome goes to the expiry word of its stream (expiry[slot], one word a (device, stream) pair, given
// out by the host on the stream's first wait), and the copies queued after it on that stream read that word: NaN rows
// after a wait that expired, the host's rows after one that saw its value. Other streams' waits and copies touch
// other words. Slot 0 is never waited on: copies on a stream that never waited always copy.
constexpr int kExpirySlots = 1024;
__device__ uint32_t expiry[kExpirySlots];
__global__ __launch_bounds__(64) void wait_kernel(const uint32_t* flag, uint32_t value, uint64_t limit, uint32_t slot) {
  if (threadIdx.x) return;
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint32_t out = 0;
  for (;;) {
    const uint32_t v = __hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
    if ((v & 0x7FFFFFFFu) == value) break;
    if (__builtin_amdgcn_s_memrealtime() - t0 > limit) {
      out = 1;
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  __hip_atomic_store(&expiry[slot], out, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// rows idx[0 .. n) of src copied to the same rows of dst, len floats a row (src may be mapped host memory); NaN rows
// instead after a wait on this stream that expired
__global__ __launch_bounds__(256) void copy_rows_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                        const int32_t* __restrict__ idx, uint32_t n, uint32_t len,
                                                        uint32_t slot) {
  const uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x;
  if (i < (uint64_t) n * len) {
    const uint64_t at = (uint64_t) idx[i / len] * len + i % len;
    dst[at] = __hip_atomic_load(&expiry[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ? __builtin_nanf("") : src[at];
  }
}

// y[t][d] = sum over j in order of src[idx[t m + j]][d] (from 0), then add's (kernels/ops.hip:515-525); 4 values a thread
__global__ __launch_bounds__(256) void gather_sum_kernel(float* __restrict__ y, const float* __restrict__ src,
                                                         const int32_t* __restrict__ idx, uint32_t m, uint32_t n,
                                                         uint32_t dim, const float* __restrict__ add) {
  const uint64_t i = (uint64_t) blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t) n * dim) return;
  const uint32_t t = (uint32_t) (i / dim), d = (uint32_t) (i % dim);
  float s = 0.0f;
  for (uint32_t j = 0; j < m; j++) s = __fadd_rn(s, src[(uint64_t) idx[t * m + j] * dim + d]);
  y[i] = add ? __fadd_rn(s, add[i]) : s;
}

// ---- osmos_lane_tables: the lane's step tables on the device (reference src/run/hip_lane.c:115-200's) ----
constexpr int kLaneThreads = 1024;
struct LaneBases {
  const uint8_t* base[3];
  uint64_t bytes[3];
};

__global__ __launch_bounds__(kLaneThreads) void lane_tables_kernel(const int32_t* __restrict__ ids, uint32_t n_tok,
                                                                   uint32_t k, uint32_t n_exp, LaneBases b,
                                                                   int32_t* __restrict__ tok, int32_t* __restrict__ pair,
                                                                   int32_t* __restrict__ cnt, int32_t* __restrict__ xrow,
                                                                   const void** __restrict__ wg,
                                                                   const void** __restrict__ wu,
                                                                   const void** __restrict__ wd,
                                                                   int32_t* __restrict__ order) {
  __shared__ int count[kMaxExperts], start[kMaxExperts], estart[kMaxExperts];
  __shared__ int row_of[OSMOS_LANE_MAX_PAIRS];
  __shared__ int n_entries;
  const uint32_t n = n_tok * k, e = threadIdx.x;
  count[e] = 0;
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < n; i += kLaneThreads) atomicAdd(&count[ids[i]], 1);
  __syncthreads();
  const int c = e < n_exp ? count[e] : 0, ne = (c + MV_MAX_TOKENS - 1) / MV_MAX_TOKENS;
  start[e] = c, estart[e] = ne;
  __syncthreads();
  for (uint32_t d = 1; d < kMaxExperts; d <<= 1) {  // inclusive scans, then each less its own
    const int a = e >= d ? start[e - d] : 0, bb = e >= d ? estart[e - d] : 0;
    __syncthreads();
    start[e] += a, estart[e] += bb;
    __syncthreads();
  }
  if (e == kMaxExperts - 1) n_entries = estart[e];
  start[e] -= c, estart[e] -= ne;
  __syncthreads();
  // each pick's row: its expert's first plus the expert's picks before it (sorted by expert, then pick)
  for (uint32_t i = threadIdx.x; i < n; i += kLaneThreads) {
    const int32_t ex = ids[i];
    int rank = 0;
    for (uint32_t j = 0; j < i; j++) rank += ids[j] == ex;
    const int r = start[ex] + rank;
    row_of[i] = r, tok[r] = (int32_t) (i / k), pair[r] = (int32_t) i;
  }
  // each expert's entries of at most MV_MAX_TOKENS rows, in order
  if (c)
    for (int p = 0; p < ne; p++) {
      const int en = estart[e] + p;
      cnt[en] = c - p * MV_MAX_TOKENS < MV_MAX_TOKENS ? c - p * MV_MAX_TOKENS : MV_MAX_TOKENS;
      xrow[en] = start[e] + p * MV_MAX_TOKENS;
      wg[en] = b.base[0] + (uint64_t) e * b.bytes[0];
      wu[en] = b.base[1] + (uint64_t) e * b.bytes[1];
      wd[en] = b.base[2] + (uint64_t) e * b.bytes[2];
    }
  __syncthreads();
  for (uint32_t en = (uint32_t) n_entries + threadIdx.x; en < n; en += kLaneThreads) cnt[en] = 0, xrow[en] = 0;
  // a token's rows in ascending order (its experts ascending: rows ascend by expert)
  for (uint32_t t = threadIdx.x; t < n_tok; t += kLaneThreads) {
    int r[kMaxK];
    for (uint32_t j = 0; j < k; j++) {
      int v = row_of[t * k + j], q = (int) j;
      while (q > 0 && r[q - 1] > v) r[q] = r[q - 1], q--;
      r[q] = v;
    }
    for (uint32_t j = 0; j < k; j++) order[t * k + j] = r[j];
  }
}

inline unsigned grid256(uint64_t n) { return (unsigned) ((n + 255) / 256); }

// ---- q4x_swiglu_rows (kernels/q4x_moe.hip:235-253): a thread 8 columns of a slot, silu(g) u (swiglu_kernel's
// expression) rounded to f16 as mm_x16_rows rounds ----
__global__ __launch_bounds__(256) void swiglu_rows_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                          uint32_t ff, const int32_t* __restrict__ idx, uint32_t slots,
                                                          _Float16* __restrict__ x16, int32_t* __restrict__ overflow) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x, groups = ff / 8;
  const uint32_t sl = i / groups, c = (i % groups) * 8;
  if (sl >= slots) return;
  const int32_t r = idx[sl];
  typedef _Float16 half8 __attribute__((ext_vector_type(8)));
  half8 h;
  bool over = false;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint64_t at = (uint64_t) (r >= 0 ? r : 0) * ff + c + j;
    h[j] = x16_round(r >= 0 ? __fmul_rn(silu(g[at]), u[at]) : 0.0f, over);
  }
  *(half8*) (x16 + x16_at(sl, c, ff)) = h;
  if (over) *overflow = 1;
}

}  // namespace moe
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool q4x_route(const float* logits, uint32_t n_tok, uint32_t n_exp, uint32_t k, int32_t* ids,
                                  float* w, int32_t* rows, void* stream) {
  if (!logits || !ids || !w || !rows || !n_tok || !n_exp || n_exp > moe::kMaxExperts || !k || k > moe::kMaxK ||
      k > n_exp)
    return false;
  moe::route_kernel<<<n_tok, moe::kRouteThreads, 0, (hipStream_t) stream>>>(logits, n_exp, k, ids, w, rows);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API void q4x_expert_bounds(uint32_t n, uint32_t n_exp, Q4xExpertBounds* b) {
  const uint32_t most = n < n_exp ? n : n_exp;
  const uint32_t cap[Q4X_TILE_RUNS] = {most, n / 17 < most ? n / 17 : most, n / 33 < most ? n / 33 : most, n / 65};
  b->entries = 0;
  for (int r = 0; r < Q4X_TILE_RUNS; r++) b->first[r] = b->entries, b->count[r] = cap[r], b->entries += cap[r];
  b->slots = n + (moe::kTile - 1) * most;
}

extern "C" OSM_API bool q4x_expert_tiles(const int32_t* ids, uint32_t n, uint32_t k, uint32_t n_exp, uint32_t dim,
                                         uint32_t ff, const Q4xExpertTiles* t, void* stream) {
  if (!ids || !n || !k || n % k || !n_exp || n_exp > moe::kMaxExperts || !dim || !ff || !t || !t->cnt || !t->gidx ||
      !t->hidx || !t->xg || !t->yg || !t->xd || !t->yd || !t->where || !t->off)
    return false;
  for (int j = 0; j < Q4X_GROUP_TENSORS; j++)
    if ((!t->tab[j] && (!t->base[j] || !t->bytes[j])) || !t->ptr[j]) return false;
  Q4xExpertBounds bd;
  q4x_expert_bounds(n, n_exp, &bd);
  const hipStream_t s = (hipStream_t) stream;
  moe::tiles_kernel<<<1, moe::kTileThreads, 0, s>>>(ids, n, k, n_exp, dim, ff, *t, bd);
  if (hipGetLastError() != hipSuccess) return false;
  if (n > moe::kPlaceInline) moe::place_kernel<<<n_exp, moe::kPlaceThreads, 0, s>>>(ids, n, k, n_exp, *t);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool q4x_swiglu(const float* g, const float* u, uint64_t n, float* y, const Q4xX16* side,
                                   void* stream) {
  if (!g || !u || !y || !n) return false;
  moe::Side sd{nullptr, nullptr, 1, 0};
  if (side && side->x16) {
    if (!side->overflow || !side->cols) return false;
    sd = moe::Side{(_Float16*) side->x16, side->overflow, side->cols, side->row0};
  }
  const uint64_t threads = (n + 3) / 4;
  if ((threads + 255) / 256 > 0x7FFFFFFFull) return false;
  moe::swiglu_kernel<<<(uint32_t) ((threads + 255) / 256), 256, 0, (hipStream_t) stream>>>(g, u, n, y, sd);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool q4x_spin(uint32_t us, void* stream) {
  moe::spin_kernel<<<1, 64, 0, (hipStream_t) stream>>>((uint64_t) us * 100ull);  // (s_memrealtime: 100 MHz)
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool q4x_swiglu_rows(const float* g, const float* u, uint32_t ff, const int32_t* idx,
                                        uint32_t slots, void* x16, int32_t* overflow, void* stream) {
  if (!g || !u || !idx || !x16 || (uintptr_t) x16 % 16 || !overflow || !slots || !ff || ff % kX16Tile) return false;
  const uint64_t threads = (uint64_t) slots * (ff / 8);
  moe::swiglu_rows_kernel<<<(uint32_t) ((threads + 255) / 256), 256, 0, (hipStream_t) stream>>>(
      g, u, ff, idx, slots, (_Float16*) x16, overflow);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool q4x_moe_sum(const float* y, const int32_t* where, const float* w, uint32_t n_tok, uint32_t k,
                                    uint32_t dim, const float* shared, const float* shared_logit, float* out,
                                    void* stream) {
  if (!y || !where || !w || !shared || !shared_logit || !out || !n_tok || !k || !dim) return false;
  moe::moe_sum_kernel<<<moe::grid256((uint64_t) n_tok * dim), 256, 0, (hipStream_t) stream>>>(y, where, w, n_tok, k, dim,
                                                                                             shared, shared_logit, out);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool ops_swiglu_lane(const float* g, const float* u, uint32_t n, float lim, const float* scale,
                                        uint32_t n_tok, float* h, void* stream) {
  if (!g || !u || !h || !n || !n_tok || !scale) return false;
  moe::swiglu_lane_kernel<<<moe::grid256((uint64_t) n * n_tok), 256, 0, (hipStream_t) stream>>>(g, u, n, lim, scale,
                                                                                               n_tok, h);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool ops_gather_rows(float* dst, const float* src, const int32_t* idx, uint32_t n, uint32_t len,
                                        void* stream) {
  if (!dst || !src || !idx || !n || !len) return false;
  moe::gather_rows_kernel<<<moe::grid256((uint64_t) n * len), 256, 0, (hipStream_t) stream>>>(dst, src, idx, n, len);
  return hipGetLastError() == hipSuccess;
}

namespace {
std::atomic<uint64_t> wait_limit_ticks{600ull * 100000000ull};  // (ten minutes of the 100 MHz counter)

// the expiry word of each (device, stream) pair that has waited: slot 1 .. kExpirySlots - 1, given out in order
std::mutex slot_mu;
std::map<std::pair<int, uintptr_t>, uint32_t> slot_of;
uint32_t slots_used[64];  // by device

// the stream's slot; with `give`, one is given out on its first call (0: none left, or no device)
uint32_t stream_slot(void* stream, bool give) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lk(slot_mu);
  const auto key = std::make_pair(dev, (uintptr_t) stream);
  const auto it = slot_of.find(key);
  if (it != slot_of.end()) return it->second;
  if (!give || slots_used[dev] + 1 >= (uint32_t) moe::kExpirySlots) return 0;
  return slot_of[key] = ++slots_used[dev];
}
}  // namespace

extern "C" OSM_API void osmos_wait_limit(uint64_t us) {
  wait_limit_ticks.store(us ? us * 100ull : 600ull * 100000000ull, std::memory_order_relaxed);
}

extern "C" OSM_API bool ops_wait(const uint32_t* flag, uint32_t value, void* stream) {
  if (!flag || (value & 0x80000000u)) return false;  // (a value with the failed mark's bit: no post could match it)
  const uint32_t slot = stream_slot(stream, true);
  if (!slot) return false;  // (more streams have waited on this device than there are expiry words)
  moe::wait_kernel<<<1, 64, 0, (hipStream_t) stream>>>(flag, value, wait_limit_ticks.load(std::memory_order_relaxed),
                                                      slot);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool ops_copy_rows(float* dst, const float* src, const int32_t* idx, uint32_t n, uint32_t len,
                                      void* stream) {
  if (!dst || !src || !idx || !n || !len) return false;
  moe::copy_rows_kernel<<<moe::grid256((uint64_t) n * len), 256, 0, (hipStream_t) stream>>>(
      dst, src, idx, n, len, stream_slot(stream, false));
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool ops_gather_sum_add(float* y, const float* src, const int32_t* idx, uint32_t m, uint32_t n,
                                           uint32_t dim, const float* add, void* stream) {
  if (!y || !src || !idx || !m || !n || !dim || !add) return false;
  moe::gather_sum_kernel<<<moe::grid256((uint64_t) n * dim), 256, 0, (hipStream_t) stream>>>(y, src, idx, m, n, dim, add);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool osmos_lane_tables(const int32_t* ids, uint32_t n_tok, uint32_t k, uint32_t n_exp,
                                          const void* const* base, const uint64_t* bytes, int32_t* tok, int32_t* pair,
                                          int32_t* cnt, int32_t* xrow, const void** wg, const void** wu,
                                          const void** wd, int32_t* order, void* stream) {
  if (!ids || !n_tok || !k || k > moe::kMaxK || !n_exp || n_exp > moe::kMaxExperts ||
      (uint64_t) n_tok * k > OSMOS_LANE_MAX_PAIRS || !base || !bytes || !tok || !pair || !cnt || !xrow || !wg || !wu ||
      !wd || !order)
    return false;
  moe::LaneBases b;
  for (int i = 0; i < 3; i++) b.base[i] = (const uint8_t*) base[i], b.bytes[i] = bytes[i];
  moe::lane_tables_kernel<<<1, moe::kLaneThreads, 0, (hipStream_t) stream>>>(ids, n_tok, k, n_exp, b, tok, pair, cnt,
                                                                            xrow, wg, wu, wd, order);
  return hipGetLastError() == hipSuccess;
}
