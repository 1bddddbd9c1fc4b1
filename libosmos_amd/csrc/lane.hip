// libosmos MI355X - the lane's int8 expert products (include/osmos/gpu/q8.h): q8_round, q8_group_tok, q8_gate_up.
//
// contract (reference kernels/lane.h:43-75, kernels/q8.h:133-212, include/osmos/gpu/q8.h:17-44): a row's 32-value
// blocks s go to logical lane s % L (L = 32 for cols >= 4096, else 16) in ascending order; per block each 16-value
// half's exact integer dot with the int8 activations (v_dot4_i32_i8), then ((d * s21) / 8) * isum per half, the halves
// added, fmaf'd with the block's activation scale onto the lane's sum; then the lanes' xor tree. the float steps and
// their order are the reference's, so each output's bits are the reference CPU path's.
//
// CDNA4 mapping: a wave64 holds 64 / L rows (4 at 16 lanes, 2 at 32), logical lane ll = lane % L of row lane / L -
// the tree's partners (ll ^ o, o < L) stay inside the row's aligned group of lanes. a workgroup is 4 waves.
#include <type_traits>

#include "fused.h"

extern "C" {
#include "../../include/osmos/gpu/mv.h"
#include "../../include/osmos/gpu/q8.h"
}

namespace osm {
namespace lane {

constexpr int kWaves = 4;              // a workgroup's waves
constexpr int kThreads = kWave * kWaves;

// matrix blockIdx.y: 64 / L rows a wave; logical lane ll its blocks ll, ll + L, ... for each of NT tokens
// the G row groups of a wave (L logical lanes each) hold the same blocks of different rows, so at a token tile that G
// divides each group loads the x codes and scales of NT / G of the tile's tokens and lane swaps (v_permlane16_swap,
// v_permlane32_swap) hand every group all of them: a G-th of the vector-memory work for x (2048 -> 6144 Q3_K at 8
// tokens 12.4 -> 10.4 us; Q4_K even at 12.1)
template <int NT, int G> constexpr bool xs_shares() { return NT > 1 && NT % G == 0 && (G == 2 || G == 4); }
// the x rows of group g's tokens g K + j (selects over the unrolled tokens: no run-time index into xr)
template <int NT, int G>
__device__ __forceinline__ void xs_rows(const uint64_t* xr, int g, uint64_t* mr) {
  constexpr int K = NT / G;
#pragma unroll
  for (int j = 0; j < K; j++) {
    mr[j] = xr[j];
#pragma unroll
    for (int t = 1; t < NT; t++)
      if (t % K == j) mr[j] = g * K + j == t ? xr[t] : mr[j];
  }
}
// block s's x for every token of the tile: xv[t] its 8 code words, then its scale's bits
template <int NT, int G>
__device__ __forceinline__ void xs_block(const int8_t* __restrict__ q, const float* __restrict__ d, const uint64_t* mr,
                                         uint32_t cols, uint32_t nblk, uint32_t s, int (*xv)[9]) {
  constexpr int K = NT / G;
#pragma unroll
  for (int j = 0; j < K; j++) {
    int w[9];
    load_x(q, mr[j] * cols + (uint64_t) s * 32, w);
    w[8] = __float_as_int(d[mr[j] * nblk + s]);
#pragma unroll
    for (int e = 0; e < 9; e++) {
      if constexpr (G == 2) {
        const auto r = __builtin_amdgcn_permlane32_swap((uint32_t) w[e], (uint32_t) w[e], false, false);
        xv[j][e] = (int) r[0], xv[K + j][e] = (int) r[1];
      } else {  // rows of 16 lanes 0 1 2 3: (0 0 2 2 | 1 1 3 3), then each across the halves
        const auto r = __builtin_amdgcn_permlane16_swap((uint32_t) w[e], (uint32_t) w[e], false, false);
        const auto u = __builtin_amdgcn_permlane32_swap(r[0], r[0], false, false);
        const auto v = __builtin_amdgcn_permlane32_swap(r[1], r[1], false, false);
        xv[j][e] = (int) u[0], xv[K + j][e] = (int) v[0], xv[2 * K + j][e] = (int) u[1], xv[3 * K + j][e] = (int) v[1];
      }
    }
  }
}
// a row group's products for the tile's tokens from its row's bytes rb (global memory, or with STG its LDS copy)
template <uint32_t T, int NT, int L, bool STG>
__device__ __forceinline__ void tok_rows(const uint8_t* rb, uint32_t row, uint32_t rows, uint32_t cols, uint32_t n,
                                         uint32_t r0, const int32_t* __restrict__ xin, const int8_t* __restrict__ q,
                                         const float* __restrict__ d, float* __restrict__ y, uint32_t ys) {
  constexpr int G = kWave / L, per = (int) (Block<T>::values / 32);
  const int lane = threadIdx.x % kWave, ll = lane % L;
  const uint32_t nblk = cols / 32;
  uint64_t xr[NT];
  in_rows<NT>(xin, r0, n, xr);
  float acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = 0.0f;
  constexpr bool XS = xs_shares<NT, G>();
  constexpr int K = XS ? NT / G : 1;
  uint64_t mr[K];
  if constexpr (XS) xs_rows<NT, G>(xr, lane / L, mr);
#pragma unroll(NT == 1 ? 4 : XS ? 1 : 2)  // (one token: 4 blocks' loads in flight; the swaps are convergent, so a
                                            // loop holding them stays rolled)
  for (uint32_t s = ll; s < nblk; s += L) {
    Codes c;
    codes<T>(rb + (s / per) * Block<T>::bytes, (int) (s % per), c, const_grid<T>());
    if constexpr (XS) {
      int xv[NT][9];
      xs_block<NT, G>(q, d, mr, cols, nblk, s, xv);
#pragma unroll
      for (int t = 0; t < NT; t++) acc[t] = __builtin_fmaf(__int_as_float(xv[t][8]), block_sum<T>(c, xv[t]), acc[t]);
    } else {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        int x[8];
        load_x(q, xr[t] * cols + (uint64_t) s * 32, x);
        acc[t] = __builtin_fmaf(d[xr[t] * nblk + s], block_sum<T>(c, x), acc[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const float v = tree<L>(acc[t]);
    if (ll == 0 && row < rows && (uint32_t) t < n) y[(uint64_t) (r0 + t) * ys + row] = v;
  }
}
// the types group_tok_kernel stages (its row copied into LDS first): Q4_K, whose decode reads the 6-bit scale fields in
// small pieces (2048 -> 6144 at 8 tokens 12.3 -> 10.4 us; Q3_K was slower staged, 10.4 -> 11.8)
template <uint32_t T> constexpr bool tok_stages() { return T == kQ4_K; }
template <uint32_t T, int NT, int L, bool STG = false>
__global__ __launch_bounds__(kThreads) void group_tok_kernel(const uint8_t* const* __restrict__ w,
                                                             const int32_t* __restrict__ cnt,
                                                             const int32_t* __restrict__ xrow,
                                                             const int32_t* __restrict__ xin, uint32_t rows,
                                                             uint32_t cols, const int8_t* __restrict__ q,
                                                             const float* __restrict__ d, float* __restrict__ y,
                                                             uint32_t ys) {
  constexpr int G = kWave / L;
  const int lane = threadIdx.x % kWave, ll = lane % L;
  const uint32_t m = blockIdx.y, row = (blockIdx.x * kWaves + threadIdx.x / kWave) * G + lane / L;
  // (blockIdx.z: the matrix's token tile, tokens z NT .. z NT + NT - 1 of its cnt[m])
  const uint32_t n_all = (uint32_t) cnt[m], z0 = blockIdx.z * NT;
  if (n_all <= z0) return;  // an entry past a device-built table's live ones (osmos_lane_tables), or a tile past its
                            // tokens: nothing read or written
  const uint32_t n = n_all - z0 < (uint32_t) NT ? n_all - z0 : NT;
  const uint32_t r0 = (uint32_t) xrow[m] + z0;
  const uint64_t rbytes = row_bytes<T>(cols);
  const uint8_t* rb = table_at(w, m) + (uint64_t) (row < rows ? row : 0) * rbytes;
  // STG (the matrix 16-aligned, a row a whole number of 16-byte words within a slot: known here, uniform a matrix):
  // the row group first copies its row into its own LDS slot with 16-byte loads, then decodes from there
  if constexpr (STG) {
    constexpr uint32_t kSlot = L == 16 ? 2304 : 4608;  // (Q4_K at 4096 / 8192 columns; 36 KB a workgroup)
    __shared__ __attribute__((aligned(16))) uint8_t stg[kWaves * G][kSlot];
    if ((uintptr_t) w[m] % 16 == 0 && rbytes % 16 == 0 && rbytes <= kSlot) {
      typedef uint32_t w4 __attribute__((ext_vector_type(4)));
      uint8_t* slot = stg[threadIdx.x / L];
      const uint32_t words = (uint32_t) (rbytes / 16);
      constexpr int kMax = (int) (kSlot / 16 + L - 1) / L;
      w4 r[kMax];
#pragma unroll
      for (int i = 0; i < kMax; i++) r[i] = ((const w4*) rb)[min((uint32_t) (ll + i * L), words - 1)];
#pragma unroll
      for (int i = 0; i < kMax; i++) ((w4*) slot)[min((uint32_t) (ll + i * L), words - 1)] = r[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // (the slot is the group's own: no workgroup barrier)
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      tok_rows<T, NT, L, true>(slot, row, rows, cols, n, r0, xin, q, d, y, ys);
      return;
    }
  }
  tok_rows<T, NT, L, false>(rb, row, rows, cols, n, r0, xin, q, d, y, ys);
}

// one token (q8_group_tok at max_cnt 1, the decode GEMV): a row a group of 2L lanes (a half-wave at 16 logical lanes,
// a wave at 32) - twice the lanes a row of group_tok_kernel, so twice the waves in flight. logical lane ll's chain
// (blocks ll, ll + L, ... in order) is split: lane ll of the group's first half sums its first links' blocks and runs
// them, lane ll of the second half sums the rest, takes the first's acc and finishes the chain; then the tree over
// the second half - the contract's links in its order. STG: the group first copies its row into its own LDS slot with
// 16-byte loads (a row whose bytes are a whole number of 16-byte words, at most kOneStg, the matrix 16-aligned) and
// decodes from there: a row's bytes in a few wide loads instead of a block's header and codes in small pieces
constexpr uint32_t kOneStg = 4608;  // a slot's bytes (Q4_K at 8192 columns)
template <int L> struct OneShape {
  static constexpr int group = 2 * L, rows = kThreads / group;  // a row's lanes, a workgroup's rows
};
// the types it serves and those it stages: measured on config 2's 2048 -> 6144 and config 1's 2048 -> 8192 at one
// token (us, group_tok_kernel / one_kernel direct / one_kernel staged): Q4_K 8.49 / - / 7.87, Q3_K 7.49 / 6.68 / 8.25,
// Q4_0 5.97 / 6.36 / 8.97 (Q4_0 stays with group_tok_kernel)
template <uint32_t T> constexpr bool one_serves() { return T == kQ4_K || T == kQ3_K; }  // (widths wide_kernel does not take)
template <uint32_t T> constexpr bool one_stages() { return T == kQ4_K; }

// a lane's run of block bytes held in registers (wide_kernel's 36 words), read by the decoders (codes<T> takes it as its block
// pointer) at byte offsets that are compile-time constants: each read folds to a register and a shift
struct RegBytes {
  const uint32_t* w;
  int off;
  __device__ RegBytes operator+(int o) const { return {w, off + o}; }
  __device__ uint32_t operator[](int i) const { return (w[(off + i) >> 2] >> (8 * ((off + i) & 3))) & 0xFFu; }
};
__device__ inline uint32_t ld16(RegBytes p) {
  if ((p.off & 3) == 3) return p[0] | p[1] << 8;
  return (p.w[p.off >> 2] >> (8 * (p.off & 3))) & 0xFFFFu;
}
__device__ inline uint32_t ld16s(RegBytes p) { return ld16(p); }

// one token of a type whose 8 contract blocks are 144 bytes - nine 16-byte words (Q4_0: 8 blocks of 18 bytes; Q4_K:
// one super-block): lane p of a row's R lanes loads blocks 8 p .. 8 p + 7 with 9 wide loads and sums each
// (block_sum, x from LDS) into the row's LDS line; then each lane runs the contract's chains ll = p + R c (C = L / R of
// them: blocks ll, ll + L, ... in order, acc = fmaf(x's scale, sum, acc)), the tree's levels L/2 .. R in its own
// registers and R/2 .. 1 across the row's lanes - the contract's steps in its order, group_tok_kernel's bits.
// (a matrix that is not 16-aligned: the same words from two-byte loads)
template <int B, typename F>
__device__ __forceinline__ void each8(F&& f) {
  if constexpr (B < 8) {
    f(std::integral_constant<int, B>());
    each8<B + 1>(f);
  }
}

// Q3_K's 8 contract blocks are one 110-byte super-block, 2-aligned: a lane loads the 8 16-byte words that cover it (a
// buffer descriptor from the matrix's 16-byte-aligned start: words past the end read as zeros) and shifts them in
// registers to the chunk's first byte (a two-step dword select, then a byte align by 0 or 2)
// (the same for IQ1_S and IQ1_M, whose 8 blocks are one 50- or 56-byte super-block. measured at one token, us,
// group_tok_kernel / wide_kernel: IQ1_S 2048 -> 7168 5.74 / 5.19, IQ1_M 6.45 / 5.19; IQ2_XXS 5.47 / 5.90, IQ3_XXS
// 4096 -> 2048 5.43 / 6.13 and 512 -> 2048 (10 matrices) 6.06 / 6.58 stay with group_tok_kernel - their codebook
// lookups spread over more lanes there - and so do the types not measured)
template <uint32_t T>
constexpr bool wide_serves() {
  return T == kQ4_0 || T == kQ4_K || T == kQ3_K || T == kIQ1_S || T == kIQ1_M;
}
template <uint32_t T>
constexpr uint32_t wide_chunk() {
  return T == kQ4_0 ? 144 : Block<T>::bytes;
}
template <uint32_t T, int L, int R, int NTH>
__global__ __launch_bounds__(NTH) void wide_kernel(const uint8_t* const* __restrict__ w, const int32_t* __restrict__ cnt,
                                                   const int32_t* __restrict__ xrow, const int32_t* __restrict__ xin,
                                                   uint32_t rows, const int8_t* __restrict__ q,
                                                   const float* __restrict__ d, float* __restrict__ y, uint32_t ys) {
  constexpr int RW = NTH / R, nblk = 8 * R, C = L / R, cols = 32 * nblk;
  constexpr uint32_t CB = wide_chunk<T>(), rb = CB * R;
  static_assert(C >= 1 && R <= 32, "a row's lanes within a 32-lane group, chains whole");
  static_assert(CB % 16 == 0 ? CB == 144 : CB <= 114, "a lane's chunk: nine aligned words, or within 8 words shifted");
  __shared__ __attribute__((aligned(16))) int8_t xq[cols];
  __shared__ float xd[nblk];
  __shared__ __attribute__((aligned(16))) float subs[RW][nblk + 4];  // (+4: the rows' lines on different banks)
  const uint32_t m = blockIdx.y;
  if (!cnt[m]) return;  // (an entry past a device-built table's live ones: nothing read or written)
  const int t = threadIdx.x, rl = t / R, p = t % R;
  const uint32_t row = blockIdx.x * RW + rl;
  const uint8_t* src = table_at(w, m) + (uint64_t) (row < rows ? row : 0) * rb + CB * p;
  // the token's codes and scales first, into registers (from L2: the copy into LDS then waits for these loads alone,
  // not for the weights issued after them - the wait counter is in order). Q4_0 issues them after its weights: at one
  // token, 2048 -> 8192 Q4_0 5.46 us (5.75 with x first), 2048 -> 6144 Q4_K 4.98 and Q3_K 4.81 with x first (the
  // copy as a loop of loads and stores behind the weights: 5.61, 5.13, 5.11)
  constexpr bool kXFirst = T != kQ4_0;
  uint64_t xr;
  in_rows<1>(xin, (uint32_t) xrow[m], 1, &xr);
  constexpr int XW = (cols / 16 + NTH - 1) / NTH, XD = (nblk + NTH - 1) / NTH;
  int4 xv[XW];
  float dv[XD];
  if constexpr (kXFirst) {
#pragma unroll
    for (int u = 0; u < XW; u++) xv[u] = ((const int4*) (q + xr * cols))[min(t + u * NTH, cols / 16 - 1)];
#pragma unroll
    for (int u = 0; u < XD; u++) dv[u] = d[xr * nblk + min(t + u * NTH, nblk - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t W[36];
  if constexpr (CB % 16) {
    const uintptr_t a0 = (uintptr_t) w[m] & ~(uintptr_t) 15, at = (uintptr_t) src;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*) a0, (short) 0, (int) ((uintptr_t) w[m] - a0 + (uint64_t) rows * rb), 0x00020000);
    const uint32_t o = (uint32_t) ((at & ~(uintptr_t) 15) - a0), sh = (uint32_t) (at & 15);
    uint32_t V[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      typedef uint32_t u4 __attribute__((ext_vector_type(4)));
      const u4 v = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, o + 16 * i, 0, 0));
      V[4 * i] = v.x, V[4 * i + 1] = v.y, V[4 * i + 2] = v.z, V[4 * i + 3] = v.w;
    }
    // (the selects as byte permutes of a dword pair: a conditional the compiler would turn into a load at a run-time
    // index, which puts the array in scratch memory)
    const uint32_t p1 = sh & 4 ? 0x07060504u : 0x03020100u, p2 = sh & 8 ? 0x07060504u : 0x03020100u;
#pragma unroll
    for (int i = 0; i < 31; i++) V[i] = __builtin_amdgcn_perm(V[i + 1], V[i], p1);
#pragma unroll
    for (int i = 0; i < 29; i++) V[i] = __builtin_amdgcn_perm(V[i + 2], V[i], p2);
#pragma unroll
    for (int i = 0; i < 28; i++) W[i] = __builtin_amdgcn_alignbyte(V[i + 1], V[i], sh & 3);
  } else if (((uintptr_t) w[m] & 15) == 0) {
#pragma unroll
    for (int i = 0; i < 9; i++) {
      const uint4 v = ((const uint4*) src)[i];
      W[4 * i] = v.x, W[4 * i + 1] = v.y, W[4 * i + 2] = v.z, W[4 * i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 36; i++) W[i] = osm::ld16(src + 4 * i) | osm::ld16(src + 4 * i + 2) << 16;
  }
  if constexpr (!kXFirst) {
#pragma unroll
    for (int u = 0; u < XW; u++) xv[u] = ((const int4*) (q + xr * cols))[min(t + u * NTH, cols / 16 - 1)];
#pragma unroll
    for (int u = 0; u < XD; u++) dv[u] = d[xr * nblk + min(t + u * NTH, nblk - 1)];
  }
#pragma unroll
  for (int u = 0; u < XW; u++)  // (unconditional where the words divide evenly: no branch to sink the loads into)
    if ((cols / 16) % NTH == 0 || t + u * NTH < cols / 16) ((int4*) xq)[t + u * NTH] = xv[u];
#pragma unroll
  for (int u = 0; u < XD; u++)
    if (nblk % NTH == 0 || t + u * NTH < nblk) xd[t + u * NTH] = dv[u];
  __syncthreads();
  float sub[8];
  each8<0>([&](auto bc) __attribute__((always_inline)) {  // (unrolled by construction: every offset a constant)
    constexpr int b = decltype(bc)::value;
    Codes c;
    if constexpr (T == kQ4_0) codes<T>(RegBytes{W, 18 * b}, 0, c, nullptr);
    else codes<T>(RegBytes{W, 0}, b, c, const_grid<T>());  // (block b of the super-block)
    int x[8];
    load_x(xq, (uint64_t) (8 * p + b) * 32, x);
    sub[b] = block_sum<T>(c, x);
  });
  ((float4*) &subs[rl][8 * p])[0] = make_float4(sub[0], sub[1], sub[2], sub[3]);
  ((float4*) &subs[rl][8 * p])[1] = make_float4(sub[4], sub[5], sub[6], sub[7]);
  __syncthreads();
  float acc[C];
#pragma unroll
  for (int c = 0; c < C; c++) {
    acc[c] = 0.0f;
#pragma unroll
    for (int s = p + R * c; s < nblk; s += L) acc[c] = __builtin_fmaf(xd[s], subs[rl][s], acc[c]);
  }
#pragma unroll
  for (int o = C / 2; o > 0; o >>= 1)
#pragma unroll
    for (int c = 0; c < o; c++) acc[c] = __fadd_rn(acc[c], acc[c + o]);
  float v = acc[0];
#pragma unroll
  for (int o = R / 2; o > 0; o >>= 1) v = __fadd_rn(v, xor_lane(v, o));
  if (p == 0 && row < rows) y[(uint64_t) (uint32_t) xrow[m] * ys + row] = v;
}

template <uint32_t T, int L, bool STG>
__device__ __forceinline__ void one_row(const uint8_t* wm, uint32_t row, uint32_t r0, const int32_t* __restrict__ xin,
                                        uint32_t cols, const int8_t* __restrict__ q, const float* __restrict__ d,
                                        float* __restrict__ y, uint32_t ys) {
  constexpr int GL = OneShape<L>::group, per = (int) (Block<T>::values / 32);
  const int gl = threadIdx.x % GL, half = gl / L, ll = gl % L;
  const uint32_t nblk = cols / 32;
  const uint64_t rb = row_bytes<T>(cols);
  const uint8_t* base = wm + (uint64_t) row * rb;
  if constexpr (STG) {
    __shared__ __attribute__((aligned(16))) uint8_t stg[OneShape<L>::rows][kOneStg];
    uint8_t* slot = stg[threadIdx.x / GL];
    const uint32_t words = (uint32_t) (rb / 16);
    typedef uint32_t w4 __attribute__((ext_vector_type(4)));  // (native: an array of HIP's uint4 stays in scratch)
    const w4* src = (const w4*) base;
    constexpr int kMax = (int) (kOneStg / 16 + GL - 1) / GL;
    w4 r[kMax];
#pragma unroll
    for (int i = 0; i < kMax; i++)
      r[i] = src[min((uint32_t) (gl + i * GL), words - 1)];  // (every load made: a conditional one puts r in scratch)
#pragma unroll
    for (int i = 0; i < kMax; i++)  // (past the row's end: its last word again, to the same place - no branches)
      ((w4*) slot)[min((uint32_t) (gl + i * GL), words - 1)] = r[i];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // (the slot is the group's own: no workgroup barrier)
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    base = slot;
  }
  uint64_t xr;
  in_rows<1>(xin, r0, 1, &xr);
  const int8_t* xq = q + xr * cols;
  const float* xd = d + xr * nblk;
  // links i of chain ll: blocks ll + L i < nblk; the first half takes i < ca, the second the rest
  const uint32_t links = (nblk + L - 1) / L, ca = (links + 1) / 2, i0 = half ? ca : 0, i1 = half ? links : ca;
  constexpr int kU = L == 16 ? 4 : 8;  // the most links a half takes unrolled (16 lanes: 4096 columns / 512)
  float sub[kU], xs[kU];
#pragma unroll
  for (int k = 0; k < kU; k++) {
    const uint32_t s = ll + L * (i0 + (uint32_t) k);
    sub[k] = 0.0f, xs[k] = 0.0f;
    if (i0 + (uint32_t) k < i1 && s < nblk) {
      Codes c;
      codes<T>(base + (s / per) * Block<T>::bytes, (int) (s % per), c, const_grid<T>());
      int x[8];
      load_x(xq, (uint64_t) s * 32, x);
      sub[k] = block_sum<T>(c, x), xs[k] = xd[s];
    }
  }
  // the chain: the first half's links from 0, handed to the second half (lane ll + L), which runs its own
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < kU; k++)
    if (!half && (uint32_t) k < ca && ll + L * (uint32_t) k < nblk) acc = __builtin_fmaf(xs[k], sub[k], acc);
  acc = L == 16 ? xor_lane(acc, 16) : __shfl_xor(acc, 32, kWave);
#pragma unroll
  for (int k = 0; k < kU; k++)
    if (half && ca + (uint32_t) k < links && ll + L * (ca + (uint32_t) k) < nblk) acc = __builtin_fmaf(xs[k], sub[k], acc);
  const float v = tree<L>(acc);
  if (half && ll == 0) y[(uint64_t) r0 * ys + row] = v;
}
template <uint32_t T, int L, bool STG>
__global__ __launch_bounds__(kThreads) void one_kernel(const uint8_t* const* __restrict__ w,
                                                       const int32_t* __restrict__ cnt, const int32_t* __restrict__ xrow,
                                                       const int32_t* __restrict__ xin, uint32_t rows, uint32_t cols,
                                                       const int8_t* __restrict__ q, const float* __restrict__ d,
                                                       float* __restrict__ y, uint32_t ys) {
  const uint32_t m = blockIdx.y, row = blockIdx.x * OneShape<L>::rows + threadIdx.x / OneShape<L>::group;
  if (!cnt[m] || row >= rows) return;  // (no token; or a group past the rows: its tree's partners are its own)
  const uint8_t* wm = table_at(w, m);
  // (the staged form needs the matrix 16-aligned: known only here, a uniform choice a matrix)
  if (STG && (uintptr_t) wm % 16 == 0)
    one_row<T, L, STG>(wm, row, (uint32_t) xrow[m], xin, cols, q, d, y, ys);
  else
    one_row<T, L, false>(wm, row, (uint32_t) xrow[m], xin, cols, q, d, y, ys);
}

// gate and up at once, then the activation (reference kernels/q8.h:214-261)
template <uint32_t T, int NT, int L>
__global__ __launch_bounds__(kThreads) void gate_up_kernel(const uint8_t* const* __restrict__ wg,
                                                           const uint8_t* const* __restrict__ wu,
                                                           const int32_t* __restrict__ cnt,
                                                           const int32_t* __restrict__ xrow,
                                                           const int32_t* __restrict__ xin,
                                                           const int32_t* __restrict__ win, uint32_t rows,
                                                           uint32_t cols, const int8_t* __restrict__ q,
                                                           const float* __restrict__ d,
                                                           const float* __restrict__ scale, float lim,
                                                           float* __restrict__ h, uint32_t hs) {
  constexpr int G = kWave / L, per = (int) (Block<T>::values / 32);
  const int lane = threadIdx.x % kWave, ll = lane % L;
  const uint32_t m = blockIdx.y, row = (blockIdx.x * kWaves + threadIdx.x / kWave) * G + lane / L;
  const uint32_t n_all = (uint32_t) cnt[m], z0 = blockIdx.z * NT;
  if (n_all <= z0) return;  // as group_tok_kernel
  const uint32_t n = n_all - z0 < (uint32_t) NT ? n_all - z0 : NT;
  const uint32_t nblk = cols / 32, r0 = (uint32_t) xrow[m] + z0;
  const uint64_t off = (uint64_t) (row < rows ? row : 0) * row_bytes<T>(cols);
  const uint8_t *rg = table_at(wg, m) + off, *ru = table_at(wu, m) + off;
  uint64_t xr[NT];
  in_rows<NT>(xin, r0, n, xr);
  float ag[NT], au[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) ag[t] = au[t] = 0.0f;
  constexpr bool XS = xs_shares<NT, G>();
  uint64_t mr[XS ? NT / G : 1];
  if constexpr (XS) xs_rows<NT, G>(xr, lane / L, mr);
#pragma unroll(NT == 1 ? 4 : XS ? 1 : 2)  // (one token: 4 blocks' loads in flight; the swaps are convergent, so a
                                            // loop holding them stays rolled)
  for (uint32_t s = ll; s < nblk; s += L) {
    Codes cg, cu;
    const uint64_t at = (s / per) * Block<T>::bytes;
    codes<T>(rg + at, (int) (s % per), cg, const_grid<T>());
    codes<T>(ru + at, (int) (s % per), cu, const_grid<T>());
    if constexpr (XS) {
      int xv[NT][9];
      xs_block<NT, G>(q, d, mr, cols, nblk, s, xv);
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const float xd = __int_as_float(xv[t][8]);
        ag[t] = __builtin_fmaf(xd, block_sum<T>(cg, xv[t]), ag[t]);
        au[t] = __builtin_fmaf(xd, block_sum<T>(cu, xv[t]), au[t]);
      }
    } else {
#pragma unroll
      for (int t = 0; t < NT; t++) {
        int x[8];
        load_x(q, xr[t] * cols + (uint64_t) s * 32, x);
        const float xd = d[xr[t] * nblk + s];
        ag[t] = __builtin_fmaf(xd, block_sum<T>(cg, x), ag[t]);
        au[t] = __builtin_fmaf(xd, block_sum<T>(cu, x), au[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const float vg = tree<L>(ag[t]), vu = tree<L>(au[t]);
    if (ll == 0 && row < rows && (uint32_t) t < n)
      h[(uint64_t) (r0 + t) * hs + row] = lane_swiglu(vg, vu, lim, scale[win ? win[r0 + t] : r0 + t]);
  }
}

// rows of x to int8 a block at a time (reference kernels/q8.h:263-277): half a wave a block, lane i its value i; the
// block's largest magnitude by the half-wave's tree (max is exact in any order)
__global__ __launch_bounds__(kThreads) void round_kernel(const float* __restrict__ x, uint32_t rows, uint32_t cols,
                                                         uint32_t xs, int8_t* __restrict__ q, float* __restrict__ d) {
  const uint32_t nblk = cols / 32;
  const uint64_t blk = (uint64_t) blockIdx.x * (kThreads / 32) + threadIdx.x / 32;
  const int i = threadIdx.x % 32;
  if (blk >= (uint64_t) rows * nblk) return;  // a whole half-wave
  const uint32_t r = (uint32_t) (blk / nblk), s = (uint32_t) (blk % nblk);
  const float v = x[(uint64_t) r * xs + (uint64_t) s * 32 + i];
  float a = fabsf(v);
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
  const float inv = a > 0.0f ? __fdiv_rn(127.0f, a) : 0.0f;
  q[(uint64_t) r * cols + (uint64_t) s * 32 + i] = (int8_t) (int) rintf(__fmul_rn(v, inv));
  if (i == 0) d[(uint64_t) r * nblk + s] = __fdiv_rn(a, 127.0f);
}

// the same rounding with 4 lanes a block, 8 values a lane (two 16-byte loads, one 8-byte store): for x rows 16-aligned
// and q 8-aligned. each value's code is rintf(v * inv) as above; the block's max by a 2-step exchange of the 4 lanes'
__global__ __launch_bounds__(kThreads) void round8_kernel(const float* __restrict__ x, uint32_t rows, uint32_t cols,
                                                          uint32_t xs, int8_t* __restrict__ q, float* __restrict__ d) {
  const uint32_t nblk = cols / 32;
  const uint64_t blk = ((uint64_t) blockIdx.x * kThreads + threadIdx.x) / 4;
  const uint32_t c = threadIdx.x % 4;
  const uint64_t nb = (uint64_t) rows * nblk, b = blk < nb ? blk : nb - 1;  // (past the end: the last block, no stores)
  const uint32_t r = (uint32_t) (b / nblk), s = (uint32_t) (b % nblk);
  const float4* src = (const float4*) (x + (uint64_t) r * xs + (uint64_t) s * 32 + 8 * c);
  const float4 lo = src[0], hi = src[1];
  const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) a = fmaxf(a, fabsf(v[i]));
  a = fmaxf(a, __shfl_xor(a, 1, 4));
  a = fmaxf(a, __shfl_xor(a, 2, 4));
  const float inv = a > 0.0f ? __fdiv_rn(127.0f, a) : 0.0f;
  uint64_t w = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) w |= (uint64_t) (uint8_t) (int8_t) (int) rintf(__fmul_rn(v[i], inv)) << (8 * i);
  if (blk < nb) {
    *(uint64_t*) (q + (uint64_t) r * cols + (uint64_t) s * 32 + 8 * c) = w;
    if (c == 0) d[(uint64_t) r * nblk + s] = __fdiv_rn(a, 127.0f);
  }
}

// ---- dispatch ----
struct Args {
  const void* const *wg, *const *wu;
  const int32_t *cnt, *xrow, *xin, *win;
  uint32_t n, rows, cols;
  const int8_t* q;
  const float *d, *scale;
  float lim;
  float* y;
  uint32_t ys;
};

template <uint32_t T, int NT, int L>
bool launch(const Args& a, bool fused, hipStream_t s, uint32_t tiles = 1) {
  constexpr uint32_t per_block = kWaves * (kWave / L);
  const dim3 grid((a.rows + per_block - 1) / per_block, a.n, tiles);
  if (fused)
    gate_up_kernel<T, NT, L><<<grid, kThreads, 0, s>>>((const uint8_t* const*) a.wg, (const uint8_t* const*) a.wu,
                                                         a.cnt, a.xrow, a.xin, a.win, a.rows, a.cols, a.q, a.d,
                                                         a.scale, a.lim, a.y, a.ys);
  else
    group_tok_kernel<T, NT, L, tok_stages<T>()><<<grid, kThreads, 0, s>>>((const uint8_t* const*) a.wg, a.cnt, a.xrow, a.xin, a.rows,
                                                           a.cols, a.q, a.d, a.y, a.ys);
  return hipGetLastError() == hipSuccess;
}

// one token of q8_group_tok: one_kernel, staged where the type gains by it and the rows allow
template <uint32_t T, int L>
bool one_launch(const Args& a, hipStream_t s) {
  const dim3 grid((a.rows + OneShape<L>::rows - 1) / OneShape<L>::rows, a.n);
  const uint64_t rb = row_bytes<T>(a.cols);
  if (one_stages<T>() && rb % 16 == 0 && rb <= kOneStg)
    one_kernel<T, L, true><<<grid, kThreads, 0, s>>>((const uint8_t* const*) a.wg, a.cnt, a.xrow, a.xin, a.rows,
                                                      a.cols, a.q, a.d, a.y, a.ys);
  else
    one_kernel<T, L, false><<<grid, kThreads, 0, s>>>((const uint8_t* const*) a.wg, a.cnt, a.xrow, a.xin, a.rows,
                                                       a.cols, a.q, a.d, a.y, a.ys);
  return hipGetLastError() == hipSuccess;
}

// one token on wide_kernel (R: a row's lanes, cols / 256); false: not taken
template <uint32_t T, int L, int R>
bool wide_launch_r(const Args& a, hipStream_t s) {
  // (a wave a workgroup: measured at one token on config 1's Q4_0 2048 -> 8192 / config 2's Q4_K 2048 -> 6144, us:
  // 64 threads 5.63 / 5.08, 128 6.12 / 6.05, 256 5.55 / 6.04; two lanes a chunk, 4 blocks each, no faster)
  constexpr int kN = 64, RW = kN / R;
  const dim3 grid((a.rows + RW - 1) / RW, a.n);
  wide_kernel<T, L, R, kN><<<grid, kN, 0, s>>>((const uint8_t* const*) a.wg, a.cnt, a.xrow, a.xin, a.rows, a.q, a.d,
                                               a.y, a.ys);
  return hipGetLastError() == hipSuccess;
}
template <uint32_t T>
bool wide_launch(const Args& a, hipStream_t s, bool* taken) {
  *taken = true;
  switch (a.cols) {
    case 1024: return wide_launch_r<T, 16, 4>(a, s);
    case 2048: return wide_launch_r<T, 16, 8>(a, s);
    case 4096: return wide_launch_r<T, 32, 16>(a, s);
    case 8192: return wide_launch_r<T, 32, 32>(a, s);
    default: *taken = false; return false;
  }
}

// q8_gate_up at one token a matrix on the fused layer's gate/up tile (fused::gu1_tab_kernel): where its widths, tile
// rows and staging fit (false in *taken: not taken)
template <uint32_t T, int L>
bool tab_launch_l(const Args& a, hipStream_t s, uint32_t words) {
  fused::GuArgs ga{};
  ga.dim = a.cols, ga.ff = a.rows, ga.lim = a.lim;
  const fused::G1Tab tb = {(const uint8_t* const*) a.wg, (const uint8_t* const*) a.wu, a.cnt, a.xrow, a.xin, a.win,
                           a.q, a.d, a.scale, a.y, a.ys};
  const dim3 grid(a.rows / fused::kG1Rows, a.n);
  constexpr int kT = fused::kG1Threads;
  if (words <= (uint32_t) kT) fused::gu1_tab_kernel<T, 1, L><<<grid, kT, 0, s>>>(ga, tb);
  else if (words <= 2u * kT) fused::gu1_tab_kernel<T, 2, L><<<grid, kT, 0, s>>>(ga, tb);
  else fused::gu1_tab_kernel<T, fused::kG1Slots, L><<<grid, kT, 0, s>>>(ga, tb);
  return hipGetLastError() == hipSuccess;
}
template <uint32_t T>
bool tab_launch(const Args& a, hipStream_t s, bool* taken) {
  const uint32_t rb = (uint32_t) row_bytes<T>(a.cols), words = fused::kG1Rows * rb / 16;
  *taken = a.rows % fused::kG1Rows == 0 && (fused::kG1Rows * rb) % 16 == 0 && words <= fused::kG1Slots * fused::kG1Threads;
  if (*taken && a.cols % 512 == 0 && a.cols <= fused::G1Max<16>::dim) return tab_launch_l<T, 16>(a, s, words);
  if (*taken && a.cols % 1024 == 0 && a.cols >= 4096 && a.cols <= fused::G1Max<32>::dim)
    return tab_launch_l<T, 32>(a, s, words);
  *taken = false;
  return false;
}

template <uint32_t T, int NT>
bool by_lanes(const Args& a, bool fused, hipStream_t s, uint32_t tiles = 1) {
  if constexpr (NT == 1) {
    if (fused) {
      bool taken = false;
      const bool ok = tab_launch<T>(a, s, &taken);
      if (taken) return ok;
    }
  }
  if constexpr (wide_serves<T>() && NT == 1) {
    bool taken = false;
    if (!fused) {
      const bool ok = wide_launch<T>(a, s, &taken);
      if (taken) return ok;
    }
  }
  if constexpr (one_serves<T>() && NT == 1)
    if (!fused && a.cols <= 8192) return a.cols >= 4096 ? one_launch<T, 32>(a, s) : one_launch<T, 16>(a, s);
  return a.cols >= 4096 ? launch<T, NT, 32>(a, fused, s, tiles) : launch<T, NT, 16>(a, fused, s, tiles);
}

template <uint32_t T>
bool by_tokens(const Args& a, uint32_t max_cnt, bool fused, hipStream_t s) {
  if (a.cols % Block<T>::values) return false;
  switch (max_cnt) {
    case 1: return by_lanes<T, 1>(a, fused, s);
    case 2: return by_lanes<T, 2>(a, fused, s);
    case 3: return by_lanes<T, 3>(a, fused, s);
    case 4: return by_lanes<T, 4>(a, fused, s);
    // (5 to 8 tokens: two tiles of 4 - twice the waves for the matrix, each with half the tokens' sums a block; every
    // token's chain the same)
    case 5: case 6: case 7: case 8: return by_lanes<T, 4>(a, fused, s, 2);
    default: return false;
  }
}

bool dispatch(uint32_t type, const Args& a, uint32_t max_cnt, bool fused, hipStream_t s) {
  switch (type) {
    case kIQ2_XXS: return by_tokens<kIQ2_XXS>(a, max_cnt, fused, s);
    case kIQ2_XS: return by_tokens<kIQ2_XS>(a, max_cnt, fused, s);
    case kIQ1_M: return by_tokens<kIQ1_M>(a, max_cnt, fused, s);
    case kIQ1_S: return by_tokens<kIQ1_S>(a, max_cnt, fused, s);
    case kIQ2_S: return by_tokens<kIQ2_S>(a, max_cnt, fused, s);
    case kIQ3_XXS: return by_tokens<kIQ3_XXS>(a, max_cnt, fused, s);
    case kQ2_K: return by_tokens<kQ2_K>(a, max_cnt, fused, s);
    case kQ4_0: return by_tokens<kQ4_0>(a, max_cnt, fused, s);
    case kQ4_K: return by_tokens<kQ4_K>(a, max_cnt, fused, s);
    case kQ3_K: return by_tokens<kQ3_K>(a, max_cnt, fused, s);
    default: return false;
  }
}

}  // namespace lane
}  // namespace osm

using namespace osm;

extern "C" OSM_API bool q8_round(const float* x, uint32_t rows, uint32_t cols, uint32_t xs, int8_t* q, float* d,
                         void* stream) {
  if (!x || !q || !d || !rows || !cols || cols % 32 || xs < cols) return false;
  const uint64_t blocks = (uint64_t) rows * (cols / 32);
  if ((uintptr_t) x % 16 == 0 && xs % 4 == 0 && (uintptr_t) q % 8 == 0) {  // (the vector form where it is aligned)
    const uint64_t per8 = lane::kThreads / 4;
    lane::round8_kernel<<<(unsigned) ((blocks + per8 - 1) / per8), lane::kThreads, 0, (hipStream_t) stream>>>(
        x, rows, cols, xs, q, d);
    return hipGetLastError() == hipSuccess;
  }
  const uint64_t per = lane::kThreads / 32;
  lane::round_kernel<<<(unsigned) ((blocks + per - 1) / per), lane::kThreads, 0, (hipStream_t) stream>>>(x, rows, cols,
                                                                                                        xs, q, d);
  return hipGetLastError() == hipSuccess;
}

extern "C" OSM_API bool q8_group_tok(uint32_t type, const void* const* w, const int32_t* cnt, const int32_t* xrow,
                             const int32_t* xin, uint32_t n, uint32_t max_cnt, uint32_t rows, uint32_t cols,
                             const int8_t* q, const float* d, float* y, uint32_t ys, void* stream) {
  if (!w || !cnt || !xrow || !q || !d || !y || !n || n > MV_MAX_GROUP || !rows || !max_cnt ||
      max_cnt > MV_MAX_TOKENS || !cols || cols % 32)
    return false;
  const lane::Args a = {w, nullptr, cnt, xrow, xin, nullptr, n, rows, cols, q, d, nullptr, 0.0f, y, ys};
  return lane::dispatch(type, a, max_cnt, false, (hipStream_t) stream);
}

extern "C" OSM_API bool q8_gate_up(uint32_t type, const void* const* wg, const void* const* wu, const int32_t* cnt,
                           const int32_t* xrow, const int32_t* xin, const int32_t* win, uint32_t n, uint32_t max_cnt,
                           uint32_t rows, uint32_t cols, const int8_t* q, const float* d, const float* scale,
                           float lim, float* h, uint32_t hs, void* stream) {
  if (!wg || !wu || !cnt || !xrow || !q || !d || !h || !n || n > MV_MAX_GROUP || !rows || !max_cnt ||
      max_cnt > MV_MAX_TOKENS || !cols || cols % 32 || !scale || hs < rows)
    return false;
  const lane::Args a = {wg, wu, cnt, xrow, xin, win, n, rows, cols, q, d, scale, lim, h, hs};
  return lane::dispatch(type, a, max_cnt, true, (hipStream_t) stream);
}
