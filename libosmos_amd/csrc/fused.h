// libosmos MI355X - the routed layer's fused kernels (osmos_lane_layer, layer.hip), bit for bit the lane contract's
// sums in the reference's layer order (src/cpu/lane.c:98-118, src/run/hip_lane.c:164-220):
//
// gu1_kernel (gate/up, one token: decode): a workgroup is (a pick, a tile of 4 of its ff rows). the pick's expert id
//   is a scalar load; the codebook and the token's x are issued before it is waited for, the tile's gate and up rows
//   right after (one scalar base a matrix). x is rounded in LDS (q8_round's bits), then each row's lane sums, the
//   tree and lane_swiglu(gate, up, lim, w[pick]) into h[pick][row].
// gu_kernel (gate/up, a batch): a workgroup is (an expert, a tile of 8 of its ff rows). its expert's first pick owns
//   it: the picks that chose the same expert (at most one a token) are its tokens, read once for all of them.
// dn_kernel (down): a workgroup is (a token, a tile of 8 of the dim rows). it rounds h of the token's k picks into LDS
//   (q8_round's bits), stages the k experts' tile rows, sums each (expert, row) in the lane order, then each row's k
//   sums in ascending expert id (the reference's ops_gather_sum_add order) and add[t][row] after.
#pragma once
#include <type_traits>

#include "lanedec.h"

namespace osm {
namespace fused {

using namespace lane;

// a gate/up tile's workgroup and rows: small tiles for one token (latency: every CU busy, no tail), larger for a
// batch (each decoded block serves several tokens); a down tile's
template <int NT>
struct GuShape {
  static constexpr int threads = NT == 1 ? 256 : 512;
  static constexpr uint32_t rows = NT == 1 ? 4 : 8;
};
constexpr int kDnThreads = 1024;
constexpr uint32_t kGuRowsMax = 8, kDnRows = 8, kMaxTok = 64, kMaxK = 32;

__host__ __device__ constexpr uint32_t align16(uint32_t v) { return (v + 15u) & ~15u; }

// gu_kernel's LDS: the gate and up tiles, NT tokens' int8 x and scales, the codebook, the expert's tokens
struct GuLds {
  uint32_t wg, wu, q, d, grid, toks, ids, subs, gv, total;
};
__host__ __device__ inline GuLds gu_lds(uint32_t row_bytes, uint32_t dim, int nt, uint32_t grid_bytes, uint32_t n) {
  const uint32_t kGuRows = nt == 1 ? GuShape<1>::rows : GuShape<2>::rows;
  GuLds l;
  uint32_t at = 0;
  l.wg = at, at += align16(kGuRows * row_bytes);
  l.wu = at, at += align16(kGuRows * row_bytes);
  l.q = at, at += align16((uint32_t) nt * dim);
  l.d = at, at += align16((uint32_t) nt * (dim / 32) * 4);
  l.grid = at, at += align16(grid_bytes);
  l.toks = at, at += align16((2 * kMaxTok + 1) * 4);
  l.ids = at, at += align16(n * 4);
  l.subs = at, at += align16(2 * (uint32_t) nt * kGuRows * (dim / 32 + 1) * 4);
  l.gv = at, at += align16(2 * (uint32_t) nt * kGuRows * 4);
  l.total = at;
  return l;
}

// dn_kernel's LDS: the k experts' tiles, the k rounded h rows and scales, the codebook, the row sums, the sorted picks
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
  const int8_t* xq;     // x already rounded (q8_round's codes and scales), for the kernels that take it: or null
  const float* xd;
};

struct DnArgs {
  const float* h;
  const int32_t* ids;
  uint32_t n_tok, k, dim, ff;
  const uint8_t* down;
  uint64_t down_bytes;
  const float* add;
  float* out;           // n_tok rows of dim
  const int8_t* hq;     // h already rounded (q8_round's codes and scales, rows by pick), for dn_kernel<.., P>
  const float* hd;
};

// a workgroup's copy of segments into LDS, in two halves so that other loads can be issued between them: load()
// issues every thread's 16-byte loads of the current round (up to kPer a thread: the weights of a tile fit one round),
// store() writes them to LDS. segment j (per_seg 16-byte words) comes from src(j) and lands at lds + j * per_seg * 16:
// the destination is the word's linear index, the source found by a reciprocal (exact: checked and corrected)
constexpr int kPer = 4;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // (native vectors: kept in registers across waits)
typedef float f32x4 __attribute__((ext_vector_type(4)));
// a weight word: read once a launch, so a streaming load (no allocation in the caches it would only pass through)
__device__ __forceinline__ u32x4 wload(const u32x4* p) {
#ifdef OSM_NO_NT
  return *p;
#else
  return __builtin_nontemporal_load(p);
#endif
}
struct Staged {
  u32x4 v0, v1, v2, v3;
  template <int U>
  __device__ __forceinline__ u32x4& at() {
    static_assert(U >= 0 && U < kPer);
    if constexpr (U == 0) return v0;
    else if constexpr (U == 1) return v1;
    else if constexpr (U == 2) return v2;
    else return v3;
  }
  template <int U>
  __device__ __forceinline__ const u32x4& at() const {
    return const_cast<Staged*>(this)->at<U>();
  }
};
// f(integral_constant<int, u>) for u = 0 .. N - 1, unrolled at compile time (constant indices keep the staged words
// in registers)
template <int N, int U = 0, typename F>
__device__ __forceinline__ void unroll(F&& f) {
  if constexpr (U < N) {
    f(std::integral_constant<int, U>());
    unroll<N, U + 1>(f);
  }
}
template <int NTH, int S = kPer, typename Src>
__device__ __forceinline__ void stage_load(Staged& st, Src src, uint32_t n, uint32_t per_seg, float inv, uint32_t base) {
  unroll<S>([&](auto u) __attribute__((always_inline)) {
    const uint32_t l0 = base + u.value * NTH + threadIdx.x, l = l0 < n ? l0 : 0;  // (past the end: word 0 again)
    uint32_t j = (uint32_t) ((float) l * inv);
    j -= j * per_seg > l;
    j += (j + 1) * per_seg <= l;
    st.template at<u.value>() = wload((const u32x4*) src(j) + (l - j * per_seg));
  });
}
template <int NTH, int S = kPer>
__device__ __forceinline__ void stage_store(const Staged& st, uint8_t* lds, uint32_t n, uint32_t base) {
  unroll<S>([&](auto u) __attribute__((always_inline)) {
    const uint32_t l = base + u.value * NTH + threadIdx.x;
    if (l < n) ((u32x4*) lds)[l] = st.template at<u.value>();
  });
}

// rows of 32-value blocks rounded to int8 as q8_round rounds them (reference kernels/q8.h:263-277): 8 threads a
// block, 4 values (a float4) each; the block's max |x| by a 3-step xor exchange among the 8 (max is exact in any
// order), each value's code, the 4 codes one word. round_load() issues a round of up to kRPer float4 loads a thread
// (block base + threadIdx.x / 8 + 32 u), round_store() reduces and writes them; value(blk, c) is the address of block
// blk's value c
constexpr int kRPer = 2;
template <int NTH>
constexpr uint32_t kRoundBlocks = (NTH / 8) * kRPer;  // blocks a round
struct Rounded {
  f32x4 v0, v1;
  template <int U>
  __device__ __forceinline__ f32x4& at() {
    static_assert(U >= 0 && U < kRPer);
    if constexpr (U == 0) return v0;
    else return v1;
  }
  template <int U>
  __device__ __forceinline__ const f32x4& at() const {
    return const_cast<Rounded*>(this)->at<U>();
  }
};
template <int NTH, typename Val>
__device__ __forceinline__ void round_load(Rounded& r, Val value, uint32_t blocks, uint32_t base) {
  const uint32_t g = threadIdx.x / 8, c = 4 * (threadIdx.x % 8);
  unroll<kRPer>([&](auto u) __attribute__((always_inline)) {
    const uint32_t blk = base + g + (NTH / 8) * u.value;
    r.template at<u.value>() = *(const f32x4*) value(blk < blocks ? blk : 0, c);
  });
}
__device__ inline uint32_t q8_byte(float v, float inv) { return (uint32_t) ((int) rintf(__fmul_rn(v, inv)) & 0xFF); }
template <int NTH>
__device__ __forceinline__ void round_store(const Rounded& r, uint32_t blocks, uint32_t base, uint32_t nb_row, uint32_t cols,
                                   int8_t* q, float* d) {
  const uint32_t g = threadIdx.x / 8, c = 4 * (threadIdx.x % 8);
  unroll<kRPer>([&](auto u) __attribute__((always_inline)) {
    const uint32_t blk = base + g + (NTH / 8) * u.value;
    const f32x4 v = r.template at<u.value>();
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
  });
}


// rows of 32-value blocks rounded as q8_round rounds them (reference kernels/q8.h:263-277), 4 lanes a block (8 values
// each: two float4): round8_load() issues the loads of blocks base .. base + NTH / 4 - 1, value(blk, c) the address of
// block blk's value c; round8_store() takes the block's max |x| by a 2-step xor exchange among its 4 lanes (max is
// exact in any order), writes its 32 codes at q + 32 blk and its scale d[blk]
struct Rounded8 {
  f32x4 a, b;
};
template <int NTH, typename Val>
__device__ __forceinline__ void round8_load(Rounded8& r, Val value, uint32_t blocks, uint32_t base) {
  const uint32_t blk = base + threadIdx.x / 4, c = 8 * (threadIdx.x % 4), b = blk < blocks ? blk : 0;
  r.a = *(const f32x4*) value(b, c), r.b = *(const f32x4*) value(b, c + 4);
}
template <int NTH>
__device__ __forceinline__ void round8_store(const Rounded8& r, uint32_t blocks, uint32_t base, int8_t* q, float* d) {
  const uint32_t blk = base + threadIdx.x / 4, c = 8 * (threadIdx.x % 4);
  float am = fmaxf(fmaxf(fmaxf(fabsf(r.a.x), fabsf(r.a.y)), fmaxf(fabsf(r.a.z), fabsf(r.a.w))),
                   fmaxf(fmaxf(fabsf(r.b.x), fabsf(r.b.y)), fmaxf(fabsf(r.b.z), fabsf(r.b.w))));
  am = fmaxf(am, xor_lane(am, 1));
  am = fmaxf(am, xor_lane(am, 2));
  if (blk < blocks) {
    const float inv = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
    uint32_t* dst = (uint32_t*) (q + blk * 32 + c);
    dst[0] = q8_byte(r.a.x, inv) | q8_byte(r.a.y, inv) << 8 | q8_byte(r.a.z, inv) << 16 | q8_byte(r.a.w, inv) << 24;
    dst[1] = q8_byte(r.b.x, inv) | q8_byte(r.b.y, inv) << 8 | q8_byte(r.b.z, inv) << 16 | q8_byte(r.b.w, inv) << 24;
    if (c == 0) d[blk] = __fdiv_rn(am, 127.0f);
  }
}

// the codebook (1 - 16 KB of constant memory, 16-aligned): grid_load() issues its loads into registers, grid_store()
// writes them to the workgroup's LDS copy - apart, so the loads can be issued first and waited for last. IQ3_XXS's
// signed table (16 KB) is not loaded: its 256 grid words (1 KB) are, and each is expanded in LDS to its 16 sign
// variants - variant s of word g takes byte i from -g where bit i of s is set, from g otherwise (one byte permute
// each), 16 g + s as the lookups index it. (the table's address is passed through an empty asm: its loads are then
// ordinary global loads, issued where they are written rather than moved next to their use)
template <uint32_t T, int NTH, bool Expand = true>
struct GridStage {
  static constexpr bool expand = Expand && T == kIQ3_XXS;
  static constexpr uint32_t n = expand ? 256 : grid_bytes<T>() / 16, words = expand ? 1 : 4;
  static constexpr uint32_t per = (n + NTH - 1) / NTH;
  // expanding: the table's 1024 16-byte words (4 a grid word: its variants 4 q .. 4 q + 3) written in `passes` rounds,
  // word p NTH + threadIdx.x in round p - consecutive lanes, consecutive words (no LDS bank conflicts)
  static constexpr uint32_t passes = 1024 / NTH;
  static_assert(!expand || (NTH >= 256 && NTH <= 1024 && NTH % 256 == 0), "the expansion's thread split");
  uint32_t v[expand ? passes : (per > 0 ? per * words : 1)];
};
typedef const __attribute__((address_space(1))) uint32_t* gptr32;
typedef const __attribute__((address_space(1))) u32x4* gptr128;
template <typename P, typename Q>
__device__ __forceinline__ P opaque_global(const Q* p) {
  uint64_t v = (uint64_t) p;
  asm volatile("" : "+s"(v));
  return (P) v;
}
template <uint32_t T, int NTH, bool E>
__device__ __forceinline__ void grid_load(GridStage<T, NTH, E>& g) {
  using G = GridStage<T, NTH, E>;
  if constexpr (G::expand) {
    const gptr32 src = opaque_global<gptr32>(kGrids.iq3xxs);
#pragma unroll
    for (uint32_t p = 0; p < G::passes; p++) g.v[p] = src[(p * NTH + threadIdx.x) / 4];
  } else if constexpr (G::n > 0) {
    const gptr128 src = opaque_global<gptr128>(const_grid<T>());
#pragma unroll
    for (uint32_t u = 0; u < G::per; u++) {
      const uint32_t l = u * NTH + threadIdx.x;
      const u32x4 w = src[l < G::n ? l : 0];
      g.v[4 * u] = w.x, g.v[4 * u + 1] = w.y, g.v[4 * u + 2] = w.z, g.v[4 * u + 3] = w.w;
    }
  }
}
template <uint32_t T, int NTH, bool E>
__device__ __forceinline__ void grid_store(const GridStage<T, NTH, E>& g, uint8_t* lds) {
  using G = GridStage<T, NTH, E>;
  if constexpr (G::expand) {
    const uint32_t qd = threadIdx.x % 4;  // (the lane's variants 4 qd .. 4 qd + 3: bits 2 and 3 of the variant)
    const uint32_t sh = (qd & 1) * 0x040000u + (qd >> 1) * 0x04000000u;
#pragma unroll
    for (uint32_t p = 0; p < G::passes; p++) {
      const uint32_t pos = g.v[p], neg = ~pos + 0x01010101u;  // (bytes 4 .. 62: no borrow between bytes)
      uint32_t w[4];
#pragma unroll
      for (uint32_t i = 0; i < 4; i++)
        w[i] = __builtin_amdgcn_perm(neg, pos, 0x03020100u + (i & 1) * 0x04u + (i >> 1) * 0x0400u + sh);
      ((u32x4*) lds)[p * NTH + threadIdx.x] = u32x4{w[0], w[1], w[2], w[3]};
    }
  } else if constexpr (G::n > 0) {
#pragma unroll
    for (uint32_t u = 0; u < G::per; u++) {
      const uint32_t l = u * NTH + threadIdx.x;
      if (l < G::n) ((u32x4*) lds)[l] = u32x4{g.v[4 * u], g.v[4 * u + 1], g.v[4 * u + 2], g.v[4 * u + 3]};
    }
  }
}

// the kernels' compute is in two phases. A: every (matrix, row, block) of the tile gets its block's `sub` (the codes,
// the exact integer half-dots, the contract's float parts: block_sum) from any thread, into LDS - the bulk of the work,
// spread over all the waves; items are ordered so that a wave's lanes share a block index (its x words read once for
// all of them). B: each row's logical lanes run the contract's chain, acc = fmaf(xd[s], sub[s], acc) over their blocks
// s = ll, ll + L, ... in order, and the lanes' xor tree - the same values in the same order as the reference's
// per-lane loop, so the same bits.

// the lanes' tree over a run-time lane count (16 or 32; uniform across the wave)
__device__ inline float tree_rt(float v, int L) { return L == 32 ? tree<32>(v) : tree<16>(v); }

// one gate/up tile: expert of pick m (its first pick's tile: others return at once), rows tile * kGuRows .. + kGuRows
// (GuShape<NT>::rows)
template <uint32_t T, int NT>
__device__ __forceinline__ void gu_item(const GuArgs& a, uint32_t m, uint32_t tile, uint8_t* smem, int L) {
  constexpr int kThreads = GuShape<NT>::threads;
  constexpr uint32_t kGuRows = GuShape<NT>::rows;
  constexpr uint32_t per = Block<T>::values / 32, bb = Block<T>::bytes;
  const uint32_t r0 = tile * kGuRows, n = a.n_tok * a.k;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.dim), nblk = a.dim / 32;
  const GuLds L_ = gu_lds(rb, a.dim, NT, grid_bytes<T>(), n);
  int32_t* toks = (int32_t*) (smem + L_.toks);  // [0, kMaxTok): the expert's picks in token order; [2 kMaxTok]: count
  // loads that need no routing first: the codebook and, for one token, its x row (the pick's own token)
  GridStage<T, kThreads, false> gs;  // (the full table: the batch tiles' loads are not what bounds them)
  grid_load(gs);
  Rounded rx;
  if constexpr (NT == 1) {
    const float* xrow = a.x + (uint64_t) (m / a.k) * a.dim;
    round_load<kThreads>(rx, [=](uint32_t blk, uint32_t i) __attribute__((always_inline)) { return xrow + blk * 32 + i; },
                         NT * (a.dim / 32), 0);
  }
  int32_t e;
  if constexpr (NT == 1) {  // one token (NT 1 is launched for a single token alone): its pick owns the tile
    e = a.ids[m];
    if (threadIdx.x == 0) toks[0] = (int32_t) m, toks[2 * kMaxTok] = 1;
  } else {
    int32_t* ids = (int32_t*) (smem + L_.ids);
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) ids[i] = a.ids[i];
    __syncthreads();
    e = __builtin_amdgcn_readfirstlane(ids[m]);  // (uniform: scalar addressing)
    // the expert's first pick owns the tile; the others leave (the same decision in every thread)
    int dup = 0;
    for (uint32_t j = threadIdx.x; j < m; j += kThreads) dup |= ids[j] == e;
    if (__syncthreads_or(dup)) return;
    if (threadIdx.x < kWave) {  // wave 0, a lane a token: its pick of this expert if any (a token's picks are
                                // distinct experts), placed by the count of earlier tokens that picked it
      int32_t p = -1;
      if (threadIdx.x < a.n_tok)
        for (uint32_t j = 0; j < a.k; j++)
          if (ids[threadIdx.x * a.k + j] == e) p = (int32_t) (threadIdx.x * a.k + j);
      const uint64_t has = __ballot(p >= 0);
      if (p >= 0) toks[__builtin_popcountll(has & ((1ull << threadIdx.x) - 1))] = p;
      if (threadIdx.x == 0) toks[2 * kMaxTok] = __builtin_popcountll(has);
    }
  }
  __syncthreads();
  const int cnt = __builtin_amdgcn_readfirstlane(toks[2 * kMaxTok]);
  // the first chunk's router weights, loaded now so that their latency is not the tile's last step
  float w0 = 0.0f;
  if (threadIdx.x < NT * kGuRows && (int) threadIdx.x / (int) kGuRows < cnt) w0 = a.w[toks[threadIdx.x / kGuRows]];
  int8_t* q = (int8_t*) (smem + L_.q);
  float* d = (float*) (smem + L_.d);
  // one round of loads: the tile's gate and up rows (contiguous in each tensor), the codebook, the first chunk's x
  const uint8_t* gsrc = a.gate + (uint64_t) e * a.gate_bytes + (uint64_t) r0 * rb;
  const uint8_t* usrc = a.up + (uint64_t) e * a.up_bytes + (uint64_t) r0 * rb;
  const uint32_t per_seg = kGuRows * rb / 16, nw = 2 * per_seg;
  const float inv_seg = 1.0f / (float) per_seg;
  auto wsrc = [=](uint32_t j) __attribute__((always_inline)) { return j ? usrc : gsrc; };
  const int live0 = cnt < NT ? cnt : NT;
  auto xval = [&](int live, int c0) __attribute__((always_inline)) {
    return [=](uint32_t blk, uint32_t i) __attribute__((always_inline)) {
      const uint32_t r = blk / nblk, tk = (uint32_t) toks[c0 + ((int) r < live ? (int) r : live - 1)] / a.k;
      return a.x + (uint64_t) tk * a.dim + (blk % nblk) * 32 + i;
    };
  };
  const uint32_t xblocks = NT * nblk;
  {
    Staged st;
    stage_load<kThreads>(st, wsrc, nw, per_seg, inv_seg, 0);
    if constexpr (NT > 1) round_load<kThreads>(rx, xval(live0, 0), xblocks, 0);
    grid_store(gs, smem + L_.grid);
    round_store<kThreads>(rx, xblocks, 0, nblk, a.dim, q, d);
    stage_store<kThreads>(st, smem + L_.wg, nw, 0);
    for (uint32_t base = kPer * kThreads; base < nw; base += kPer * kThreads) {  // (tiles past one round)
      stage_load<kThreads>(st, wsrc, nw, per_seg, inv_seg, base);
      stage_store<kThreads>(st, smem + L_.wg, nw, base);
    }
    for (uint32_t base = kRoundBlocks<kThreads>; base < xblocks; base += kRoundBlocks<kThreads>) {
      round_load<kThreads>(rx, xval(live0, 0), xblocks, base);
      round_store<kThreads>(rx, xblocks, base, nblk, a.dim, q, d);
    }
  }
  __syncthreads();
  const auto* grid = (const typename GridOf<T>::E*) (smem + L_.grid);
  float* subs = (float*) (smem + L_.subs);  // [(m NT + t) 16 + row][s]
  float* gv = (float*) (smem + L_.gv);      // [(m NT + t) 16 + row]
  for (int c0 = 0; c0 < cnt; c0 += NT) {
    const int live = cnt - c0 < NT ? cnt - c0 : NT;
    if (c0) {  // the next chunk's x (the previous chunk's read first)
      __syncthreads();
      Rounded rx;
      for (uint32_t base = 0; base < xblocks; base += kRoundBlocks<kThreads>) {
        round_load<kThreads>(rx, xval(live, c0), xblocks, base);
        round_store<kThreads>(rx, xblocks, base, nblk, a.dim, q, d);
      }
      __syncthreads();
    }
    // phase A: (block, matrix, row) items, the row fastest: the 2 kGuRows lanes of a block share its x
    const uint32_t items = 2 * kGuRows * nblk;
    for (uint32_t it = threadIdx.x; it < items; it += kThreads) {
      const uint32_t row = it % kGuRows, mm = (it / kGuRows) & 1, s = it / (2 * kGuRows);
      Codes c;
      codes<T>((lbytes) (smem + (mm ? L_.wu : L_.wg) + row * rb + (s / per) * bb), (int) (s % per), c, grid);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        int x[8];
        const int4* xp = (const int4*) (q + t * a.dim + s * 32);
        const int4 x0 = xp[0], x1 = xp[1];
        x[0] = x0.x, x[1] = x0.y, x[2] = x0.z, x[3] = x0.w, x[4] = x1.x, x[5] = x1.y, x[6] = x1.z, x[7] = x1.w;
        subs[((mm * NT + t) * kGuRows + row) * (nblk + 1) + s] = block_sum<T>(c, x);
      }
    }
    __syncthreads();
    // phase B: a chain a (matrix, token, row, logical lane), whole waves so a tree's lanes are all present
    const uint32_t chains = 2 * NT * kGuRows * L, lgL = L == 32 ? 5 : 4;
    for (uint32_t ch = threadIdx.x; ch < (chains + kWave - 1) / kWave * kWave; ch += kThreads) {
      const uint32_t ll = ch & (L - 1), unit = (ch >> lgL) < 2 * NT * kGuRows ? ch >> lgL : 0, t = (unit / kGuRows) % NT;
      const float* sb = subs + unit * (nblk + 1);
      float acc = 0.0f;
      for (uint32_t s = ll; s < nblk; s += L) acc = __builtin_fmaf(d[t * nblk + s], sb[s], acc);
      const float v = tree_rt(acc, L);
      if (ll == 0 && ch < chains) gv[unit] = v;
    }
    __syncthreads();
    if (threadIdx.x < NT * kGuRows) {
      const int t = (int) threadIdx.x / (int) kGuRows, row = (int) threadIdx.x % (int) kGuRows;
      if (t < live) {
        const int pk = toks[c0 + t];
        a.h[(uint64_t) pk * a.ff + r0 + row] =
            lane_swiglu(gv[t * kGuRows + row], gv[(NT + t) * kGuRows + row], a.lim, c0 ? a.w[pk] : w0);
      }
    }
  }
}

// one down tile: token t, rows tile * kDnRows .. + kDnRows
template <uint32_t T, int S, bool P>
__device__ __forceinline__ void dn_item(const DnArgs& a, uint32_t t, uint32_t tile, uint8_t* smem, int L) {
  constexpr int kThreads = kDnThreads;
  constexpr uint32_t per = Block<T>::values / 32, bb = Block<T>::bytes;
  const uint32_t r0 = tile * kDnRows, K = a.k;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.ff), nblk = a.ff / 32;
  const DnLds L_ = dn_lds(rb, a.ff, K, grid_bytes<T>());
  // one round of loads: the activations first (h is by pick, so it needs no routing), the k experts' tile rows (in
  // pick order), the codebook
  auto hval = [=](uint32_t blk, uint32_t i) __attribute__((always_inline)) {
    return a.h + (uint64_t) (t * K + blk / nblk) * a.ff + (blk % nblk) * 32 + i;
  };
  const uint32_t hblocks = K * nblk;
  // the picks' expert ids first: the weights wait on them, and loads are waited for in issue order
  const int32_t pid = threadIdx.x < K ? a.ids[t * K + threadIdx.x] : 0;
  __builtin_amdgcn_sched_barrier(0);
  // the token's k activation rows: rounded here, or (P) their codes and scales already rounded (the first two
  // 16-byte words and the first scale a thread loaded now, the rest after the weights)
  Rounded8 rh;
  u32x4 hw[2];
  float hs = 0.0f;
  const u32x4* hqs = (const u32x4*) (a.hq + (uint64_t) t * K * a.ff);
  const float* hds = a.hd + (uint64_t) t * hblocks;
  const uint32_t hwords = K * a.ff / 16;
  if constexpr (P) {
    hw[0] = hqs[min((uint32_t) threadIdx.x, hwords - 1)];
    hw[1] = hqs[min((uint32_t) threadIdx.x + kThreads, hwords - 1)];
    hs = hds[min((uint32_t) threadIdx.x, hblocks - 1)];
  } else {
    round8_load<kThreads>(rh, hval, hblocks, 0);
  }
  const uint64_t o = (uint64_t) t * a.dim + r0 + threadIdx.x;
  const float addv = threadIdx.x < kDnRows ? a.add[o] : 0.0f;  // (loaded now: its latency off the tile's end)
  GridStage<T, kThreads, false> gs;  // (the full table: expanding it in 4 of the 16 waves is slower here)
  grid_load(gs);
  int32_t* picks = (int32_t*) (smem + L_.picks);  // [j]: pick j's expert; [kMaxK + r]: the pick j of rank r
  if (threadIdx.x < K) picks[threadIdx.x] = pid;
  __syncthreads();
  int8_t* q = (int8_t*) (smem + L_.q);
  float* d = (float*) (smem + L_.d);
  const uint8_t* down = a.down + (uint64_t) r0 * rb;
  const uint64_t db = a.down_bytes;
  const uint32_t per_seg = kDnRows * rb / 16, nw = K * per_seg;
  const float inv_seg = 1.0f / (float) per_seg;
  auto wsrc = [=](uint32_t j) __attribute__((always_inline)) { return down + (uint64_t) picks[j] * db; };
  {
    Staged st;
    stage_load<kThreads, S>(st, wsrc, nw, per_seg, inv_seg, 0);
    if (threadIdx.x < kWave) {  // wave 0, a lane a pick: its rank in ascending expert id (then pick); and its h
      const uint32_t j = threadIdx.x;
      const int32_t ex = j < K ? picks[j] : INT32_MAX;
      uint32_t rank = 0;
      for (uint32_t i = 0; i < K; i++) {
        const int32_t o = __shfl(ex, (int) i, kWave);
        rank += o < ex || (o == ex && i < j);
      }
      if (j < K) picks[kMaxK + rank] = (int32_t) j;
    }
    grid_store(gs, smem + L_.grid);
    if constexpr (P) {
      if (threadIdx.x < hwords) ((u32x4*) q)[threadIdx.x] = hw[0];
      if (threadIdx.x + kThreads < hwords) ((u32x4*) q)[threadIdx.x + kThreads] = hw[1];
      if (threadIdx.x < hblocks) d[threadIdx.x] = hs;
    } else {
      round8_store<kThreads>(rh, hblocks, 0, q, d);
    }
    stage_store<kThreads, S>(st, smem + L_.w, nw, 0);
    for (uint32_t base = S * kThreads; base < nw; base += S * kThreads) {
      stage_load<kThreads, S>(st, wsrc, nw, per_seg, inv_seg, base);
      stage_store<kThreads, S>(st, smem + L_.w, nw, base);
    }
    if constexpr (P) {
      for (uint32_t i = threadIdx.x + 2 * kThreads; i < hwords; i += kThreads) ((u32x4*) q)[i] = hqs[i];
      for (uint32_t i = threadIdx.x + kThreads; i < hblocks; i += kThreads) d[i] = hds[i];
    } else {
      for (uint32_t base = kThreads / 4; base < hblocks; base += kThreads / 4) {
        round8_load<kThreads>(rh, hval, hblocks, base);
        round8_store<kThreads>(rh, hblocks, base, q, d);
      }
    }
  }
  __syncthreads();
  const auto* grid = (const typename GridOf<T>::E*) (smem + L_.grid);
  float* ye = (float*) (smem + L_.ye);  // [j 8 + row]
  // phases A and B as one: a thread a chain (pick j, row, logical lane ll), the lane fastest, then the row (a wave's
  // rows share their blocks of x): the lane's blocks s = ll, ll + L, ... each summed (block_sum) and chained in order,
  // acc = fmaf(d[s], sub, acc), then the tree across the row's L lanes
  const uint32_t chains = K * kDnRows * L, lgL = L == 32 ? 5 : 4;
  for (uint32_t ch = threadIdx.x; ch < (chains + kWave - 1) / kWave * kWave; ch += kThreads) {
    const uint32_t ll = ch & (L - 1), unit = (ch >> lgL) < K * kDnRows ? ch >> lgL : 0, j = unit / kDnRows;
    const uint8_t* wr = smem + L_.w + unit * rb;
    float acc = 0.0f;
    for (uint32_t s = ll; s < nblk; s += L) {
      Codes c;
      codes<T>((lbytes) (wr + (s / per) * bb), (int) (s % per), c, grid);
      int x[8];
      load_x(q, j * a.ff + s * 32, x);
      acc = __builtin_fmaf(d[j * nblk + s], block_sum<T>(c, x), acc);
    }
    const float v = tree_rt(acc, L);
    if (ll == 0 && ch < chains) ye[unit] = v;
  }
  __syncthreads();
  if (threadIdx.x < kDnRows) {  // each row's k sums in ascending expert id, then add's
    float s = 0.0f;
    for (uint32_t r = 0; r < K; r++) s = __fadd_rn(s, ye[picks[kMaxK + r] * kDnRows + threadIdx.x]);
    a.out[o] = __fadd_rn(s, addv);
  }
}

template <uint32_t T, int NT, int L>
__global__ __launch_bounds__(GuShape<NT>::threads) void gu_kernel(GuArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  gu_item<T, NT>(a, blockIdx.y, blockIdx.x, smem, L);
}

// gu1_kernel: the one-token gate/up (decode). workgroup (tile, pick m): rows kG1Rows tile .. of the gate and up
// matrices of expert ids[m]; lane_swiglu(gate, up, lim, w[m]) into h[m][row]. its loads are issued with no work between
// the expert id's arrival and the weights' issue: each 16-byte word's offset in its matrix's rows is set before the id
// is waited for, the rows' bases are scalar (the id is a scalar load), and every staging slot holds one matrix's words
// (a slot's loads: one scalar base plus the lane's offset). its LDS is a static array laid out for the largest dim of
// its lane count (G1Max), so every LDS address folds into the instruction. one wave a row (wave w: row w), the gate's
// lane chains in lanes 0 .. 31, the up's in 32 .. 63.
constexpr int kG1Threads = GuShape<1>::threads;
constexpr uint32_t kG1Rows = GuShape<1>::rows;
constexpr uint32_t kG1Slots = kPer;  // staging slots a matrix at most: its rows at most kG1Slots kG1Threads words
static_assert(kG1Threads == (int) kG1Rows * kWave, "gu1_kernel: a wave a row");
// the dims each lane count takes: 16 lanes up to 2048 (whole 16-block chains: a multiple of 512), 32 lanes 4096 ..
// 8192 (whole 32-block chains: a multiple of 1024)
template <int L> struct G1Max { static constexpr uint32_t dim = L == 16 ? 2048 : 8192; };

// gu1_kernel's LDS: the codebook first, x's codes and scales, the gate and up rows
template <uint32_t T, int L>
struct G1Lds {
  static constexpr uint32_t D = G1Max<L>::dim;
  static constexpr uint32_t grid = 0, q = align16(grid_bytes<T>()), d = q + D, w = d + D / 32 * 4;
  static constexpr uint32_t total = w + align16(2 * kG1Rows * (uint32_t) row_bytes<T>(D));
};

// q8_gate_up's operands for gu1_item (TAB): matrix m's gate and up rows from the pointer tables, its token's input row
// xin[xrow[m]] (or xrow[m]) of the rounded q / d, its scale scale[win[xrow[m]]] (or scale[xrow[m]]), its h row
// xrow[m] (hs floats apart); a matrix with no token is skipped
struct G1Tab {
  const uint8_t* const* wg;
  const uint8_t* const* wu;
  const int32_t *cnt, *xrow, *xin, *win;
  const int8_t* q;
  const float *d, *scale;
  float* h;
  uint32_t hs;
};

// one gate/up tile of one token: the layer's (pick m's expert ids[m], its rows at gate + id gate_bytes, router weight
// w[m], h row m) or, TAB, q8_gate_up's matrix m (tb). S: staging slots a matrix (the fewest that hold its tile rows);
// L: the contract's lanes a row (16 or 32)
template <uint32_t T, int S, int L, bool P = false, bool TAB = false>
__device__ __forceinline__ void gu1_item(const GuArgs& a, const G1Tab& tb, uint32_t m, uint32_t tile, uint8_t* smem) {
  using LD = G1Lds<T, L>;
  constexpr int kThreads = kG1Threads;
  constexpr uint32_t per = Block<T>::values / 32, bb = Block<T>::bytes;
  constexpr int R = (int) (G1Max<L>::dim / 32 / (kThreads / 4));  // x's rounding rounds (4 lanes a block)
  static_assert(!TAB || P, "q8_gate_up's x is rounded already");
  const uint32_t r0 = tile * kG1Rows;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.dim), nblk = a.dim / 32;
  const uint32_t per_seg = kG1Rows * rb / 16;  // a matrix's words
  // the lane's word of each slot (past the matrix's end: its last word again, loaded and not stored)
  uint32_t idx[S];
#pragma unroll
  for (uint32_t u = 0; u < (uint32_t) S; u++) idx[u] = min(u * kThreads + threadIdx.x, per_seg - 1);
  uint32_t e = 0, rout = 0;
  float wm;
  const int8_t* xq = a.xq;
  const float* xdp = a.xd;
  if constexpr (TAB) {
    if (!tb.cnt[m]) return;  // (the whole workgroup)
    rout = (uint32_t) tb.xrow[m];
    const uint32_t rin = tb.xin ? (uint32_t) tb.xin[rout] : rout;
    wm = tb.scale[tb.win ? (uint32_t) tb.win[rout] : rout];
    xq = tb.q + (uint64_t) rin * a.dim, xdp = tb.d + (uint64_t) rin * nblk;
  } else {
    e = (uint32_t) a.ids[m];  // (an expert id: not negative; unsigned, so no sign extension to wait for)
    wm = a.w[m];
  }
  GridStage<T, kThreads> gs;
  grid_load(gs);
  // the one token's row: rounded here, or (P) its codes and scales already rounded, copied
  constexpr int RQ = (int) (G1Max<L>::dim / 16 / kThreads) > 0 ? (int) (G1Max<L>::dim / 16 / kThreads) : 1;
  Rounded8 rx[P ? 1 : R];
  u32x4 xw[RQ];
  float xs = 0.0f;
  if constexpr (P) {
    const uint32_t nw = a.dim / 16;
#pragma unroll
    for (int r = 0; r < RQ; r++) xw[r] = ((const u32x4*) xq)[min(r * kThreads + threadIdx.x, nw - 1)];
    xs = xdp[min((uint32_t) threadIdx.x, nblk - 1)];  // (nblk <= 256 = kThreads)
  } else {
    auto xval = [=](uint32_t blk, uint32_t c) __attribute__((always_inline)) { return a.x + blk * 32 + c; };
#pragma unroll
    for (int r = 0; r < R; r++)
      if (r == 0 || (uint32_t) r * (kThreads / 4) < nblk) round8_load<kThreads>(rx[r], xval, nblk, r * (kThreads / 4));
  }
  // (a scheduling barrier: the codebook and x loads issue before the id is waited for)
  __builtin_amdgcn_sched_barrier(0);
  u32x4 wv[2 * S];
  if constexpr (TAB) {
    const uint8_t* gb = table_at(tb.wg, m) + (uint64_t) r0 * rb;
    const uint8_t* ub = table_at(tb.wu, m) + (uint64_t) r0 * rb;
    if ((((uintptr_t) gb | (uintptr_t) ub) & 15) == 0) {
#pragma unroll
      for (uint32_t u = 0; u < (uint32_t) S; u++) wv[u] = wload((const u32x4*) gb + idx[u]), wv[S + u] = wload((const u32x4*) ub + idx[u]);
    } else {  // (a matrix that is not 16-aligned: the same words from two-byte loads)
      auto w16 = [](const uint8_t* p) __attribute__((always_inline)) {
        u32x4 v;
        v.x = osm::ld16(p) | osm::ld16(p + 2) << 16, v.y = osm::ld16(p + 4) | osm::ld16(p + 6) << 16;
        v.z = osm::ld16(p + 8) | osm::ld16(p + 10) << 16, v.w = osm::ld16(p + 12) | osm::ld16(p + 14) << 16;
        return v;
      };
#pragma unroll
      for (uint32_t u = 0; u < (uint32_t) S; u++) wv[u] = w16(gb + 16 * idx[u]), wv[S + u] = w16(ub + 16 * idx[u]);
    }
  } else {
    const u32x4* gsrc = (const u32x4*) (a.gate + (uint64_t) e * a.gate_bytes + (uint64_t) r0 * rb);
    const u32x4* usrc = (const u32x4*) (a.up + (uint64_t) e * a.up_bytes + (uint64_t) r0 * rb);
#pragma unroll
    for (uint32_t u = 0; u < (uint32_t) S; u++) wv[u] = wload(gsrc + idx[u]), wv[S + u] = wload(usrc + idx[u]);
  }
  int8_t* q = (int8_t*) (smem + LD::q);
  float* d = (float*) (smem + LD::d);
  grid_store(gs, smem + LD::grid);
  if constexpr (P) {
#pragma unroll
    for (int r = 0; r < RQ; r++)
      if (r * kThreads + threadIdx.x < a.dim / 16) ((u32x4*) q)[r * kThreads + threadIdx.x] = xw[r];
    if (threadIdx.x < nblk) d[threadIdx.x] = xs;
  } else {
#pragma unroll
    for (int r = 0; r < R; r++)
      if (r == 0 || (uint32_t) r * (kThreads / 4) < nblk) round8_store<kThreads>(rx[r], nblk, r * (kThreads / 4), q, d);
  }
#pragma unroll
  for (uint32_t u = 0; u < (uint32_t) S; u++) {
    const uint32_t l = u * kThreads + threadIdx.x;
    if (l < per_seg) {
      ((u32x4*) (smem + LD::w))[l] = wv[u];
      ((u32x4*) (smem + LD::w))[per_seg + l] = wv[S + u];
    }
  }
  __syncthreads();
  const auto* grid = (const typename GridOf<T>::E*) (smem + LD::grid);
  const uint32_t lane = threadIdx.x % kWave, row = threadIdx.x / kWave;
  const uint8_t* wr = smem + LD::w + ((lane / 32) * kG1Rows + row) * rb;
  float v;
  if constexpr (L == 16) {
    // logical lane ll = l % 16's chain, blocks s = ll + 16 i for i < C = nblk / 16, is split in two: lanes 0 .. 15
    // (of each half-wave) take i < CA = (C + 1) / 2, lanes 16 .. 31 the rest. every lane sums its blocks
    // (block_sum); the first lanes run the chain's first links, acc = fmaf(d[s], sub, acc) from 0, and hand acc to
    // lane l + 16 (xor 16), which runs the rest; then the tree over lanes 16 .. 31 - the contract's links in its
    // order, with no barrier and no sums in LDS
    const uint32_t half = lane / 16 % 2, ll = lane % 16;
    const uint32_t C = nblk / 16, CA = (C + 1) / 2, i0 = half ? CA : 0, n_i = half ? C - CA : CA;
    float sub[2] = {0.0f, 0.0f}, xd[2] = {0.0f, 0.0f};
#pragma unroll
    for (uint32_t k = 0; k < 2; k++)
      if (k < n_i) {
        const uint32_t sb = ll + 16 * (i0 + k);
        Codes c;
        codes<T>((lbytes) (wr + (sb / per) * bb), (int) (sb % per), c, grid);
        int x[8];
        load_x(q, sb * 32, x);
        sub[k] = block_sum<T>(c, x), xd[k] = d[sb];
      }
    float acc = 0.0f;  // the first lanes' links
#pragma unroll
    for (uint32_t k = 0; k < 2; k++)
      if (k < CA) acc = __builtin_fmaf(xd[k], sub[k], acc);
    acc = xor_lane(acc, 16);  // (the second lanes now hold their first lanes' acc)
#pragma unroll
    for (uint32_t k = 0; k < 2; k++)
      if (k < C - CA) acc = __builtin_fmaf(xd[k], sub[k], acc);
    v = tree<16>(acc);
  } else {
    // logical lane ll = l % 32's whole chain, blocks s = ll + 32 i in order, then the tree over the half-wave
    const uint32_t ll = lane % 32;
    float acc = 0.0f;
    for (uint32_t sb = ll; sb < nblk; sb += 32) {
      Codes c;
      codes<T>((lbytes) (wr + (sb / per) * bb), (int) (sb % per), c, grid);
      int x[8];
      load_x(q, sb * 32, x);
      acc = __builtin_fmaf(d[sb], block_sum<T>(c, x), acc);
    }
    v = tree<32>(acc);
  }
  const float g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  if constexpr (TAB) {
    if (lane == 0) tb.h[(uint64_t) rout * tb.hs + r0 + row] = lane_swiglu(g, u, a.lim, wm);
  } else {
    if (lane == 0) a.h[(uint64_t) m * a.ff + r0 + row] = lane_swiglu(g, u, a.lim, wm);
  }
}

template <uint32_t T, int S, int L, bool P = false>
__global__ __launch_bounds__(kG1Threads) void gu1_kernel(GuArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[G1Lds<T, L>::total];
  gu1_item<T, S, L, P>(a, G1Tab{}, blockIdx.y, blockIdx.x, smem);
}

// q8_gate_up at one token a matrix on gu1_kernel's tile: workgroup (tile of 4 rows, matrix m)
template <uint32_t T, int S, int L>
__global__ __launch_bounds__(kG1Threads) void gu1_tab_kernel(GuArgs a, G1Tab tb) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[G1Lds<T, L>::total];
  gu1_item<T, S, L, true, true>(a, tb, blockIdx.y, blockIdx.x, smem);
}

// gub_kernel: gate/up for a batch (n_tok >= 2), gu1_kernel's tile and lane layout with several tokens a pass.
// workgroup (tile, pick m): owned by the first pick of its expert e (a later pick of e leaves at once); its tokens
// are the picks of e (at most one a token), NB a pass: their x rows rounded into LDS, then each lane decodes its blocks
// once and runs its chain links for every token of the pass (a chain accumulator a token), the trees, and
// lane_swiglu(gate, up, lim, w[pick]) into h[pick][row] for each.
template <uint32_t T, int L, int NB, int W = 4>  // W: the workgroup's waves, a row each
struct GbLds {
  static constexpr uint32_t D = G1Max<L>::dim;
  static constexpr uint32_t grid = 0, q = align16(grid_bytes<T>()), d = q + NB * D, w = d + NB * (D / 32) * 4;
  static constexpr uint32_t toks = w + align16(2 * (uint32_t) W * (uint32_t) row_bytes<T>(D));
  static constexpr uint32_t ids = toks + align16((kMaxTok + 1) * 4);  // the routing ids of the first 2 (kWave * W) picks
  static constexpr uint32_t total = ids + 2 * (kWave * W) * 4;
};

// one pass of gub_kernel: tokens toks[c0 .. c0 + live) (live <= NB), x rows from..NB-1 rounded into q/d (the rows
// before from are there already), chains, trees and h
template <uint32_t T, int L, int NB, bool P, int W>
__device__ __forceinline__ void gub_pass(const GuArgs& a, const int32_t* toks, int c0, int live, int from, int8_t* q,
                                         float* d, const typename GridOf<T>::E* grid, const uint8_t* wr, uint32_t r0) {
  constexpr int kThreads = (kWave * W);
  constexpr uint32_t per = Block<T>::values / 32, bb = Block<T>::bytes;
  const uint32_t nblk = a.dim / 32, lane = threadIdx.x % kWave, row = threadIdx.x / kWave;
  // the pass's x rows rounded (q8_round's bits): block b nblk + s is token b's block s (the rows past the live ones
  // repeat the last: summed, never stored)
  auto xval = [&](uint32_t blk, uint32_t c) __attribute__((always_inline)) {
    const uint32_t b = blk / nblk, tb = (int) b < live ? b : (uint32_t) live - 1;
    return a.x + (uint64_t) ((uint32_t) toks[c0 + (int) tb] / a.k) * a.dim + (blk % nblk) * 32 + c;
  };
  if constexpr (P) {  // (x already rounded: the rows' codes and scales copied)
    const uint32_t wpr = a.dim / 16;
    for (uint32_t i = from * wpr + threadIdx.x; i < NB * wpr; i += kThreads) {
      const uint32_t b = i / wpr, tb = (int) b < live ? b : (uint32_t) live - 1;
      ((u32x4*) q)[i] = ((const u32x4*) (a.xq + (uint64_t) ((uint32_t) toks[c0 + (int) tb] / a.k) * a.dim))[i % wpr];
    }
    for (uint32_t i = from * nblk + threadIdx.x; i < NB * nblk; i += kThreads) {
      const uint32_t b = i / nblk, tb = (int) b < live ? b : (uint32_t) live - 1;
      d[i] = a.xd[(uint64_t) ((uint32_t) toks[c0 + (int) tb] / a.k) * nblk + i % nblk];
    }
  } else {
    for (uint32_t base = from * nblk; base < NB * nblk; base += kThreads / 4) {
      Rounded8 rx;
      round8_load<kThreads>(rx, xval, NB * nblk, base);
      round8_store<kThreads>(rx, NB * nblk, base, q, d);
    }
  }
  __syncthreads();
  float v[NB];
  if constexpr (L == 16) {  // gu1_kernel's split chains, an accumulator a token
    const uint32_t half = lane / 16 % 2, ll = lane % 16;
    const uint32_t C = nblk / 16, CA = (C + 1) / 2, i0 = half ? CA : 0, n_i = half ? C - CA : CA;
    float sub[2][NB], xd[2][NB];
#pragma unroll
    for (uint32_t k = 0; k < 2; k++)
#pragma unroll
      for (int b = 0; b < NB; b++) sub[k][b] = 0.0f, xd[k][b] = 0.0f;
#pragma unroll
    for (uint32_t k = 0; k < 2; k++)
      if (k < n_i) {
        const uint32_t sb = ll + 16 * (i0 + k);
        Codes c;
        codes<T>((lbytes) (wr + (sb / per) * bb), (int) (sb % per), c, grid);
#pragma unroll
        for (int b = 0; b < NB; b++) {
          int x[8];
          load_x(q, (b * nblk + sb) * 32, x);
          sub[k][b] = block_sum<T>(c, x), xd[k][b] = d[b * nblk + sb];
        }
      }
#pragma unroll
    for (int b = 0; b < NB; b++) {
      float acc = 0.0f;
#pragma unroll
      for (uint32_t k = 0; k < 2; k++)
        if (k < CA) acc = __builtin_fmaf(xd[k][b], sub[k][b], acc);
      acc = xor_lane(acc, 16);
#pragma unroll
      for (uint32_t k = 0; k < 2; k++)
        if (k < C - CA) acc = __builtin_fmaf(xd[k][b], sub[k][b], acc);
      v[b] = tree<16>(acc);
    }
  } else {  // a lane's whole chain, an accumulator a token
    const uint32_t ll = lane % 32;
    float acc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = 0.0f;
    for (uint32_t sb = ll; sb < nblk; sb += 32) {
      Codes c;
      codes<T>((lbytes) (wr + (sb / per) * bb), (int) (sb % per), c, grid);
#pragma unroll
      for (int b = 0; b < NB; b++) {
        int x[8];
        load_x(q, (b * nblk + sb) * 32, x);
        acc[b] = __builtin_fmaf(d[b * nblk + sb], block_sum<T>(c, x), acc[b]);
      }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) v[b] = tree<32>(acc[b]);
  }
#pragma unroll
  for (int b = 0; b < NB; b++) {
    const float g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[b]), 16));
    const float u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[b]), 48));
    if (lane == 0 && b < live) {
      const int32_t pk = toks[c0 + b];
      a.h[(uint64_t) pk * a.ff + r0 + row] = lane_swiglu(g, u, a.lim, a.w[pk]);
    }
  }
}

template <uint32_t T, int S, int L, int NB, bool P = false, int W = 4>
__global__ __launch_bounds__(kWave * W) void gub_kernel(GuArgs a) {
  using LD = GbLds<T, L, NB, W>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[LD::total];
  constexpr int kThreads = (kWave * W);
  constexpr uint32_t R = LD::D / 32 / (kThreads / 4) > 0 ? LD::D / 32 / (kThreads / 4) : 1;  // rounds for a row
  const uint32_t m = blockIdx.y, r0 = blockIdx.x * (uint32_t) W, n = a.n_tok * a.k;
  const uint32_t rb = (uint32_t) row_bytes<T>(a.dim), nblk = a.dim / 32;
  const uint32_t per_seg = (uint32_t) W * rb / 16;
  uint32_t idx[S];
#pragma unroll
  for (uint32_t u = 0; u < (uint32_t) S; u++) idx[u] = min(u * kThreads + threadIdx.x, per_seg - 1);
  const uint32_t e = (uint32_t) a.ids[m];
  // loads in the order they are waited on: the routing ids (the first 2 kThreads picks), the codebook, pick m's
  // own x row (the owner pick is the expert's first: its token's row is the first pass's first), then the weights
  const uint32_t* ids = (const uint32_t*) a.ids;
  const uint32_t i0 = threadIdx.x, i1 = threadIdx.x + kThreads;
  const uint32_t id0 = ids[min(i0, n - 1)], id1 = ids[min(i1, n - 1)];
  __builtin_amdgcn_sched_barrier(0);
  GridStage<T, kThreads> gs;
  grid_load(gs);
  const float* xrow = a.x + (uint64_t) (m / a.k) * a.dim;
  auto xval = [=](uint32_t blk, uint32_t c) __attribute__((always_inline)) { return xrow + blk * 32 + c; };
  Rounded8 rx[P ? 1 : R];
  constexpr int RQ = (int) (LD::D / 16 / kThreads) > 0 ? (int) (LD::D / 16 / kThreads) : 1;
  u32x4 xw[RQ];
  float xs = 0.0f;
  if constexpr (P) {  // (x already rounded: the owner's row's codes and scales, copied)
    const u32x4* src = (const u32x4*) (a.xq + (uint64_t) (m / a.k) * a.dim);
#pragma unroll
    for (int r = 0; r < RQ; r++) xw[r] = src[min(r * kThreads + threadIdx.x, a.dim / 16 - 1)];
    xs = a.xd[(uint64_t) (m / a.k) * nblk + min((uint32_t) threadIdx.x, nblk - 1)];
  } else {
#pragma unroll
    for (uint32_t r = 0; r < R; r++) round8_load<kThreads>(rx[r], xval, nblk, r * (kThreads / 4));
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t* sid = (uint32_t*) (smem + LD::ids);
  if (i0 < n) sid[i0] = id0;
  if (i1 < n) sid[i1] = id1;
  // the expert's first pick owns the tile (the same decision in every thread)
  int dup = (i0 < m && id0 == e) || (i1 < m && id1 == e);
  for (uint32_t j = threadIdx.x + 2 * kThreads; j < m; j += kThreads) dup |= ids[j] == e;
  if (__syncthreads_or(dup)) return;
  const u32x4* gsrc = (const u32x4*) (a.gate + (uint64_t) e * a.gate_bytes + (uint64_t) r0 * rb);
  const u32x4* usrc = (const u32x4*) (a.up + (uint64_t) e * a.up_bytes + (uint64_t) r0 * rb);
  u32x4 wv[2 * S];
#pragma unroll
  for (uint32_t u = 0; u < (uint32_t) S; u++) wv[u] = gsrc[idx[u]], wv[S + u] = usrc[idx[u]];
  int32_t* toks = (int32_t*) (smem + LD::toks);  // [0, kMaxTok): the expert's picks in token order; [kMaxTok]: count
  if (threadIdx.x < kWave) {  // wave 0, a lane a token: its pick of e if any, placed by the earlier tokens' count
    int32_t pk = -1;
    if (threadIdx.x < a.n_tok) {  // (a uniform choice of table: LDS reads or global ones, never a flat load of either)
      if (n <= 2 * kThreads) {
        for (uint32_t j = 0; j < a.k; j++)
          if (sid[threadIdx.x * a.k + j] == e) pk = (int32_t) (threadIdx.x * a.k + j);
      } else {
        for (uint32_t j = 0; j < a.k; j++)
          if (ids[threadIdx.x * a.k + j] == e) pk = (int32_t) (threadIdx.x * a.k + j);
      }
    }
    const uint64_t has = __ballot(pk >= 0);
    if (pk >= 0) toks[__builtin_popcountll(has & ((1ull << threadIdx.x) - 1))] = pk;
    if (threadIdx.x == 0) toks[kMaxTok] = __builtin_popcountll(has);
  }
  int8_t* q = (int8_t*) (smem + LD::q);
  float* d = (float*) (smem + LD::d);
  grid_store(gs, smem + LD::grid);
  if constexpr (P) {
#pragma unroll
    for (int r = 0; r < RQ; r++)
      if (r * kThreads + threadIdx.x < a.dim / 16) ((u32x4*) q)[r * kThreads + threadIdx.x] = xw[r];
    if (threadIdx.x < nblk) d[threadIdx.x] = xs;
  } else {
#pragma unroll
    for (uint32_t r = 0; r < R; r++) round8_store<kThreads>(rx[r], nblk, r * (kThreads / 4), q, d);
  }
#pragma unroll
  for (uint32_t u = 0; u < (uint32_t) S; u++) {
    const uint32_t l = u * kThreads + threadIdx.x;
    if (l < per_seg) {
      ((u32x4*) (smem + LD::w))[l] = wv[u];
      ((u32x4*) (smem + LD::w))[per_seg + l] = wv[S + u];
    }
  }
  __syncthreads();
  const int cnt = __builtin_amdgcn_readfirstlane(toks[kMaxTok]);
  const auto* grid = (const typename GridOf<T>::E*) (smem + LD::grid);
  const uint32_t lane = threadIdx.x % kWave, row = threadIdx.x / kWave;
  const uint8_t* wr = smem + LD::w + ((lane / 32) * (uint32_t) W + row) * rb;
  // the first pass holds the owner's row already; full passes while NB tokens are left, then a token a pass
  int c0 = 0;
  if (cnt >= NB) {
    gub_pass<T, L, NB, P, W>(a, toks, 0, NB, 1, q, d, grid, wr, r0);
    c0 = NB;
  } else {
    gub_pass<T, L, 1, P, W>(a, toks, 0, 1, 1, q, d, grid, wr, r0);
    c0 = 1;
  }
  for (; c0 + NB <= cnt; c0 += NB) {
    __syncthreads();  // (the previous pass's codes read)
    gub_pass<T, L, NB, P, W>(a, toks, c0, NB, 0, q, d, grid, wr, r0);
  }
  for (; c0 < cnt; c0++) {
    __syncthreads();
    gub_pass<T, L, 1, P, W>(a, toks, c0, 1, 0, q, d, grid, wr, r0);
  }
}

// S: staging slots a round (1, 2 or kPer: the fewest that hold the tile in one round)
template <uint32_t T, int L, int S, bool P = false>
__global__ __launch_bounds__(kDnThreads) void dn_kernel(DnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  dn_item<T, S, P>(a, blockIdx.y, blockIdx.x, smem, L);
}

}  // namespace fused
}  // namespace osm
