// libosmos MI355X - the lane contract at prefill scale on the int8 matrix cores (include/osmos_mi355x.h:
// osmos_lane_group): q8_group_tok's sums for any token count, the same bits.
//
// contract (reference kernels/lane.h:43-75, kernels/q8.h:133-212, src/cpu/q8.c:383-407): a row's 32-value blocks s go to
// logical lane ll = s % L (L = 32 for cols >= 4096, else 16) in ascending order; per block each 16-value half's exact
// integer dot with the int8 activations, then ((d s21) / 8) isum per half, the halves added, fmaf'd with the block's
// activation scale onto the lane's sum; then the lanes' xor tree (pairs ll, ll ^ L/2 first, then ll ^ L/4, ...).
//
// CDNA4 mapping: a workgroup owns 16 rows (their whole slab and the codebook staged in LDS once) x G groups of 8
// tokens a pass. the integer half-dots are MFMAs: each 32-value block's codes (lane l: row l % 16, values 8 (l / 16) ..
// + 7, decoded from LDS straight into its B operand - the IQ1 types' 8 grid + delta folded into one int8 per value)
// against an A operand of 8 tokens' halves (row i: token i / 2's half i % 2, the other half's k zeroed), one
// v_mfma_i32_16x16x32_i8 a group: lane l gets both half-dots of tokens 2 (l / 16), 2 (l / 16) + 1 for its row l % 16,
// so it applies that row's half factors itself, the dots coming out of the MFMA as floats' bits (a bias in its
// accumulator) so each product is one fma. the float steps then run per output in the contract's order. the W waves
// split the logical lanes (wave w the chains ll = w mod W, blocks s = w mod W), so a wave keeps L / W chains an output
// in registers; the xor tree is finished across the waves through LDS with the same additions (fadd commutes exactly).
// groups of 8 tokens waste at most 7 token slots a matrix (prefill's many small experts). kernel16 (most types) takes
// 16 tokens a pass instead, one token a lane in the A operand and the halves split on the weights' side (below).
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
  signs8(grid[q[k]], sm[(ld32b(q + 4) >> (7 * k)) & 0x7F], w0, w1);
}
template <>
__device__ inline void scales<kIQ2_XXS>(lbytes b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (int) (ld32b(b + 2 + 8 * j + 4) >> 28) + 1;
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
  const uint32_t sg = (ld32b(b + 66 + 4 * j) >> (7 * k)) & 0x7F, par = __builtin_popcount(sg) & 1u;
  w0 = grid[16 * q[2 * k] + (sg & 15)];
  w1 = grid[16 * q[2 * k + 1] + ((sg >> 4) | par << 3)];
}
template <>
__device__ inline void scales<kIQ3_XXS>(lbytes b, int j, float& d, int& s0, int& s1) {
  s0 = s1 = 2 * (2 * (int) (ld32b(b + 66 + 4 * j) >> 28) + 1);
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

// a block's two half factors, the contract's ((d s21) / 8) per half (lane_part's first two products)
template <uint32_t T>
__device__ inline void factors(lbytes b, int j, float& f0, float& f1) {
  float d;
  int s0, s1;
  scales<T>(b, j, d, s0, s1);
  f0 = __fmul_rn(__fmul_rn(d, (float) s0), 0.125f), f1 = __fmul_rn(__fmul_rn(d, (float) s1), 0.125f);
}

// the integer half-dots come out of the MFMA biased by kBias (its accumulator input): kBias + I as a float's bits is
// 1.5 2^23 + I exactly for |I| < 2^22 (a half's dot is under 2^18: 16 codes of at most 127 x 62), so
// fmaf(f, bits, -(f 1.5 2^23)) is f I rounded once - RN(f I), the contract's product, with no int-to-float convert.
// (-(f 1.5 2^23) is exact: f has at most 17 significant bits. for a finite f; a block whose scale d is not finite
// gives NaN there, where the contract's product is +-inf or NaN)
constexpr int kBias = 0x4B400000;

// acc + v(lane n of the lane's 16-lane row) x x, one rounding: the contract's chain step with its token scale taken
// by DPP row_newbcast in the same instruction (v_fmac_f32 with a DPP source: no separate broadcast move; config 5's
// IQ2_XXS gate 921-936 -> 898 us, every type 0-3 % faster; n a compile-time constant once unrolled). a DPP read of a
// VGPR that a VALU instruction wrote in the two before needs two wait states, and the compiler's hazard pass does not
// look inside the asm, so the asm brings its own (s_nop 1: 0.5-0.8 % of the kernel)
__device__ inline float fmac_bcast(float acc, float v, float x, int n) {
  switch (n) {
#define B(i) \
  case i: asm("s_nop 1\n\tv_fmac_f32_dpp %0, %1, %2 row_newbcast:" #i " row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(v), "v"(x)); break;
    B(0) B(1) B(2) B(3) B(4) B(5) B(6) B(7) B(8) B(9) B(10) B(11) B(12) B(13) B(14) B(15)
#undef B
  }
  return acc;
}
constexpr float kBiasF = 12582912.0f;

// tokens an MFMA: the A operand's 16 rows are 8 tokens' two halves, row i token i / 2's half i % 2 (a first half's
// values 0 .. 15 in the lanes of k 0 .. 15, zeros in those of k 16 .. 31; a second half's the other way round), the B
// operand the block's full 32 codes of 16 weight rows: one MFMA gives both half-dots of 8 tokens x 16 rows, and lane l
// holds D rows 4 (l / 16) .. + 3 of column l % 16 - both halves of tokens 2 (l / 16) and 2 (l / 16) + 1 of its row
constexpr int kGroup = 8;
// token groups a pass (G) and waves a workgroup (W) by type and lane count. G = 1: kernel16, 16 tokens a pass (the
// halves split on the weights' side); G = 2: kernel, two groups of 8 a pass (each decoded block serving both). the
// kernels are bound by their loads, not their decode (a build of kernel without the decode ran 1227 us against 1241,
// one without its A loads 890): kernel16 halves the A loads a full group issues. measured on config 5's routing (512
// tokens, 250 experts, the busiest 441), us, 2048 x 7168 / 7168 x 2048: kernel16 (W 8 / 4) IQ2_XXS 1098 / 1201,
// IQ1_S 1133 / 1283, IQ2_XS 1136 / 1260, IQ2_S 1399 / 1434, IQ3_XXS 1260 (W 16; 1326 at 8) / 1421, and with the
// last pass of at most 8 tokens in the 8-token layout 1055 / 1189, 1064 / 1232, 1082 / 1217, 1340 / -, 1218 / 1376,
// and as built now (A rows staged where stage_a says, the scales' broadcast inside the fmac) 898 / 985, 1058 / 1145,
// 1076 / 1024, 1329 / 1422, 1215 / 1308;
// kernel with one group
// of 8 a pass 1161 / 1223, 1188 / 1325, 1214 / 1254, 1583 / 1497, 1612 / 1508 (it was 1308 / 1362 for IQ2_XXS before
// its loads were reworked); with two groups 1344 / 1360, 1347 / 1509, 1368 / 1386, 1709 / 1501, 1411 (W 16) / 1747;
// IQ1_M two groups 1426 / 2107 against kernel16's 1450 / 2113 and one group's 2015 / 3169 (its scale decode holds 88
// VGPRs: occupancy 5)
struct Shape {
  int g, w;
};
template <uint32_t T, int L>
constexpr Shape shape() {
#ifdef OSM_LG  // (a build-time override, for tuning sweeps)
  return L == 16 ? Shape{OSM_LG16, OSM_LW16} : Shape{OSM_LG32, OSM_LW32};
#endif
  if constexpr (T == kIQ1_M) return {2, L == 16 ? 4 : 8};
  else if constexpr (L == 16) return {1, 4};
  else if constexpr (T == kIQ3_XXS) return {1, 16};
  else return {1, 8};
}

template <uint32_t T>
constexpr uint32_t grid_bytes_of() {
  return GridOf<T>::n * sizeof(typename GridOf<T>::E);
}

// dynamic LDS: the workgroup's 16 weight rows (the whole slab), the codebook, the sign masks, the waves' partial trees
template <int G, int W, int L = 0>
struct Lds {
  uint32_t slab, grid, sm, part, total;
  __host__ __device__ Lds(uint32_t rb, uint32_t grid_bytes) {
    slab = 0;
    grid = (16 * rb + 15) / 16 * 16;
    sm = grid + grid_bytes;
    part = sm + 128 * 8;
    // (L: kernel16 staging a round's A rows, 16 tokens x L blocks, kAS = 32 L + 16 bytes apart, where the partial
    // trees go at the pass's end)
    const uint32_t tree = W * G * 2 * kWave * 4, arow = L ? 16 * (32 * L + 16) : 0;
    total = part + (tree > arow ? tree : arow);
  }
};
// kernel16 with each round's A rows staged in LDS (16-byte loads of the 16 tokens' bytes, the next round's in registers
// meanwhile) rather than loaded a lane's 8 bytes at a time: measured on config 5's routing, us, 2048 x 7168 (32
// lanes) / 7168 x 2048 (16 lanes), staged against not: IQ2_XXS 953 (held to 6 waves a SIMD: 80 VGPRs, 7 spilled;
// 1078 without) / 1010 against 1053 / 1192, IQ1_S 1149 / 1163 against 1065 / 1232, IQ2_XS 1140 / 1046 against
// 1084 / 1219, IQ2_S 1410 / 1574 against 1339 / 1434, IQ3_XXS 1690 / 1320 against 1218 / 1375
template <uint32_t T, int L>
constexpr bool stage_a() {
  return T != kIQ2_S && (L == 16 || T == kIQ2_XXS);
}

// blockIdx.x: 16 rows; blockIdx.y: the matrix, its cnt[m] tokens from row xrow[m] of q / d, G groups of 8 a pass.
// wave w takes the blocks s = w (mod W): its chains are the logical lanes ll = w (mod W), L / W accumulators an
// output; the xor tree's levels L/2 .. W pair chains of one wave (in registers), its levels W/2 .. 1 pair the waves
// (through LDS) - the same additions as the tree
template <uint32_t T, int L, int G, int W, bool FULL>
__global__ __launch_bounds__(W * kWave) void kernel(const uint8_t* const* __restrict__ w, const int32_t* __restrict__ cnt,
                                                   const int32_t* __restrict__ xrow, uint32_t cols,
                                                   const int8_t* __restrict__ q, const float* __restrict__ d,
                                                   float* __restrict__ y, uint32_t ys) {
  constexpr int kThreads = W * kWave, per = (int) (Block<T>::values / 32), C = L / W, TOK = kGroup * G;
  static_assert(G >= 2, "one group a pass: kernel16");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t m = blockIdx.y, n = (uint32_t) cnt[m];
  if (!n) return;  // (the whole workgroup)
  // (the wave index through readfirstlane: uniform, so the block loop and its offsets are scalar)
  const int wave = __builtin_amdgcn_readfirstlane((int) (threadIdx.x / kWave)), lane = threadIdx.x % kWave;
  const int col = lane % 16, quad = lane / 16;
  const uint32_t row0 = blockIdx.x * kTile, nblk = cols / 32, r0 = (uint32_t) xrow[m];
  const uint32_t rb = (uint32_t) row_bytes<T>(cols);
  const Lds<G, W> L_(rb, grid_bytes_of<T>());
  {  // the slab (16 rows x rb: contiguous, 16-aligned) and the codebook into LDS
    const u32x4* src = (const u32x4*) (table_at(w, m) + (uint64_t) row0 * rb);
    const uint32_t nw = 16 * rb / 16;
    for (uint32_t i = threadIdx.x; i < nw; i += kThreads) ((u32x4*) (smem + L_.slab))[i] = src[i];
    constexpr uint32_t ng = grid_bytes_of<T>() / 16;
    const u32x4* gs = (const u32x4*) const_grid<T>();
    for (uint32_t i = threadIdx.x; i < ng; i += kThreads) ((u32x4*) (smem + L_.grid))[i] = gs[i];
    if (threadIdx.x < 128) ((uint64_t*) (smem + L_.sm))[threadIdx.x] = sign_mask(threadIdx.x);
  }
  const auto* grid = (const typename GridOf<T>::E*) (smem + L_.grid);
  const uint64_t* sm = (const uint64_t*) (smem + L_.sm);
  float* part = (float*) (smem + L_.part);  // [wave][g][pair][lane]
  const uint8_t* brow = smem + L_.slab + col * rb;  // this lane's B row (a weight row)
  // the A operand's rows from a buffer descriptor over the matrix's token rows: a lane whose (row, k) is a zero of
  // the layout, or whose token is past the count, reads at an offset past the descriptor's end - zeros, no access
  const __amdgpu_buffer_rsrc_t qr =
      __builtin_amdgcn_make_buffer_rsrc((void*) (q + (uint64_t) r0 * cols), (short) 0, (int) (n * cols), 0x00020000);
  // and the block scales of this lane's output tokens (a token past the count: zero, no access)
  const __amdgpu_buffer_rsrc_t dr =
      __builtin_amdgcn_make_buffer_rsrc((void*) (d + (uint64_t) r0 * nblk), (short) 0, 0x7FFFFFFF, 0x00020000);
  const bool lives = (col % 2 == 0) == (quad < 2);
  // this lane's two outputs of a group: tokens ot, ot + 1 of the group, row col
  const int ot = 2 * quad;
  v4i bias = {kBias, kBias, kBias, kBias};
  asm volatile("" : "+v"(bias));  // (held in registers, not rebuilt before every MFMA)
  for (uint32_t c0 = 0; c0 < n; c0 += TOK) {
    __syncthreads();  // (the slab's first pass; then the last pass's partial trees read before they are rewritten)
    const int groups = (int) ((n - c0 + kGroup - 1) / kGroup) < G ? (int) ((n - c0 + kGroup - 1) / kGroup) : G;
    uint32_t voff[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      const uint32_t t = c0 + g * kGroup + col / 2;
      voff[g] = lives && t < n ? t * cols + 8 * quad : 0x80000000u;
    }
    float acc[C][G][2];
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
      for (int g = 0; g < G; g++) acc[c][g][0] = acc[c][g][1] = 0.0f;
    // two or more groups a pass (the types whose decode is dearest: each decoded block serves both): the A words and
    // token scales one block ahead, each lane loading its two outputs' scales (a ring here costs these kernels
    // their occupancy)
    uint32_t xo[G][2];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int p = 0; p < 2; p++) {
        const uint32_t to = c0 + g * kGroup + ot + p;
        xo[g][p] = to < n ? to * nblk * 4 : 0x80000000u;
      }
    long an[G];
    float xn[G][2];
    auto aload = [&](uint32_t s) __attribute__((always_inline)) {
#pragma unroll
      for (int g = 0; g < G; g++)
        if (g < groups) {
          an[g] = __builtin_bit_cast(long, __builtin_amdgcn_raw_buffer_load_b64(qr, voff[g], s * 32, 0));
#pragma unroll
          for (int p = 0; p < 2; p++)
            xn[g][p] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(dr, xo[g][p], s * 4, 0));
        }
    };
    aload((uint32_t) wave);
    for (uint32_t s0 = (uint32_t) wave; s0 < nblk; s0 += L) {
#pragma unroll
      for (int c = 0; c < C; c++) {
        const uint32_t s = s0 + W * c;  // logical lane wave + W c
        if (!FULL && s >= nblk) break;  // (uniform)
        long a[G];
        float x[G][2];
#pragma unroll
        for (int g = 0; g < G; g++) a[g] = an[g], x[g][0] = xn[g][0], x[g][1] = xn[g][1];
        aload(s + W < nblk ? s + W : s);  // (the last block: loaded again, unused - no branch)
        const uint8_t* blk = brow + (s / per) * Block<T>::bytes;
        const int j = (int) (s % per);
        uint32_t w0, w1;
        chunk<T>((lbytes) blk, j, quad, grid, sm, w0, w1);
        const long b = (long) (((uint64_t) w1 << 32) | w0);
        float f0, f1;
        factors<T>((lbytes) blk, j, f0, f1);
        const float n0 = -__fmul_rn(f0, kBiasF), n1 = -__fmul_rn(f1, kBiasF);
#pragma unroll
        for (int g = 0; g < G; g++) {
          if (g < groups) {
            const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[g], b, bias, 0, 0, 0);
            const float s0_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(D[0]), n0),
                                        __builtin_fmaf(f1, __int_as_float(D[1]), n1));
            const float s1_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(D[2]), n0),
                                        __builtin_fmaf(f1, __int_as_float(D[3]), n1));
            acc[c][g][0] = __builtin_fmaf(x[g][0], s0_, acc[c][g][0]);
            acc[c][g][1] = __builtin_fmaf(x[g][1], s1_, acc[c][g][1]);
          }
        }
      }
    }
    // the tree's levels L/2 .. W within the wave: chains c and c + o (logical lanes ll and ll ^ W o)
#pragma unroll
    for (int o = C / 2; o > 0; o >>= 1)
#pragma unroll
      for (int c = 0; c < o; c++)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
          for (int p = 0; p < 2; p++) acc[c][g][p] = __fadd_rn(acc[c][g][p], acc[c + o][g][p]);
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int p = 0; p < 2; p++) part[((wave * G + g) * 2 + p) * kWave + lane] = acc[0][g][p];
    __syncthreads();
    // levels W/2 .. 1 across the waves (T_w: wave w's subtree, logical lanes w mod W): each pass pairs w with
    // w + o for w < o, as the tree pairs logical lanes ll and ll ^ o. a lane's 2 G outputs are shared out over the
    // waves: wave v finishes outputs v, v + W, ...
    {
      const uint32_t wv = G * 2 * kWave;  // a wave's stride
      for (int oi = (int) wave; oi < G * 2; oi += W) {
        const int g = oi / 2, p = oi % 2;
        const float* pp = part + (g * 2 + p) * kWave + lane;
        float t[W];
#pragma unroll
        for (int v = 0; v < W; v++) t[v] = pp[v * wv];
#pragma unroll
        for (int o = W / 2; o > 0; o >>= 1)
#pragma unroll
          for (int v = 0; v < o; v++) t[v] = __fadd_rn(t[v], t[v + o]);
        const uint32_t tk = c0 + g * kGroup + ot + p;
        if (tk < n) y[(uint64_t) (r0 + tk) * ys + row0 + col] = t[0];
      }
    }
  }
}

// one group of 16 tokens a pass, the halves split on the weights' side: the A operand's 16 rows are 16 tokens (lane l:
// token l % 16's values 8 (l / 16) .. + 7 of the block - every lane a token's bytes, none a zero of the layout), and two
// MFMAs take the block's B words with the second half's k zeroed and with the first half's: lane l holds the two
// half-dots of tokens 4 (l / 16) + i, i < 4, for its weight row l % 16. the same products, sums and chains as kernel's
// (one A load a block serves 16 tokens, not 8: the kernel is bound by its loads). the token scales: lane col of a
// 16-lane row loads token 4 (row) + col % 4's scale of the round's block col / 4, each block's four broadcast from it.
// a matrix's last pass with at most 8 tokens takes the 8-token layout instead (pass8: one MFMA a block, 2 outputs a
// lane, all live; config 5's IQ2_XXS gate 1095-1119 -> 1049-1072 us, the same bits)
template <uint32_t T, int L, int W, bool FULL>
// (IQ2_XXS at 32 lanes with whole rounds held to 80 VGPRs, 6 waves a SIMD: 1078 -> 953 us, 7 registers spilled; a
// 16-wave workgroup held to 64, two workgroups a CU - IQ3_XXS at 32 lanes ran 1613 against 1215 us at 65)
__global__ __launch_bounds__(W * kWave)
__attribute__((amdgpu_waves_per_eu(T == kIQ2_XXS && L == 32 && FULL ? 6 : W == 16 ? 8 : 1)))
void kernel16(const uint8_t* const* __restrict__ w,
                                                     const int32_t* __restrict__ cnt, const int32_t* __restrict__ xrow,
                                                     uint32_t cols, const int8_t* __restrict__ q,
                                                     const float* __restrict__ d, float* __restrict__ y, uint32_t ys) {
  constexpr int kThreads = W * kWave, per = (int) (Block<T>::values / 32), C = L / W, TOK = 16;
  // the A ring's depth (a divisor of C: its slots static). measured on config 5's IQ2_XXS gate with 8 tokens a group
  // (us): 1 block ahead 1239, 2 1146, 4 1195
  constexpr int PD = C >= 2 ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t m = blockIdx.y, n = (uint32_t) cnt[m];
  if (!n) return;  // (the whole workgroup)
  const int wave = __builtin_amdgcn_readfirstlane((int) (threadIdx.x / kWave)), lane = threadIdx.x % kWave;
  const int col = lane % 16, quad = lane / 16;
  const uint32_t row0 = blockIdx.x * kTile, nblk = cols / 32, r0 = (uint32_t) xrow[m];
  const uint32_t rb = (uint32_t) row_bytes<T>(cols);
  constexpr bool kStageA = stage_a<T, L>();
  const Lds<1, W, kStageA ? L : 0> L_(rb, grid_bytes_of<T>());
  {  // the slab (16 rows x rb: contiguous, 16-aligned) and the codebook into LDS
    const u32x4* src = (const u32x4*) (table_at(w, m) + (uint64_t) row0 * rb);
    const uint32_t nw = 16 * rb / 16;
    for (uint32_t i = threadIdx.x; i < nw; i += kThreads) ((u32x4*) (smem + L_.slab))[i] = src[i];
    constexpr uint32_t ng = grid_bytes_of<T>() / 16;
    const u32x4* gs = (const u32x4*) const_grid<T>();
    for (uint32_t i = threadIdx.x; i < ng; i += kThreads) ((u32x4*) (smem + L_.grid))[i] = gs[i];
    if (threadIdx.x < 128) ((uint64_t*) (smem + L_.sm))[threadIdx.x] = sign_mask(threadIdx.x);
  }
  const auto* grid = (const typename GridOf<T>::E*) (smem + L_.grid);
  const uint64_t* sm = (const uint64_t*) (smem + L_.sm);
  float* part = (float*) (smem + L_.part);  // [wave][pair][lane]: two outputs a lane at a time
  const uint8_t* brow = smem + L_.slab + col * rb;  // this lane's B row (a weight row)
  // (the A rows' range the matrix's own n rows: a staged round's 16-byte words past a row's end - cols not a whole
  // number of rounds - read the next token's bytes, unused, or zeros past the last row; their offset is all in the
  // vector offset, which the range check covers)
  const __amdgpu_buffer_rsrc_t qr =
      __builtin_amdgcn_make_buffer_rsrc((void*) (q + (uint64_t) r0 * cols), (short) 0, (int) (n * cols), 0x00020000);
  const __amdgpu_buffer_rsrc_t dr =
      __builtin_amdgcn_make_buffer_rsrc((void*) (d + (uint64_t) r0 * nblk), (short) 0, 0x7FFFFFFF, 0x00020000);
  const uint32_t kc = (uint32_t) (col / 4) < (uint32_t) C ? (uint32_t) (col / 4) : (uint32_t) (C - 1);
  v4i bias = {kBias, kBias, kBias, kBias};
  asm volatile("" : "+v"(bias));  // (held in registers, not rebuilt before every MFMA)
  // a pass of at most 8 tokens: the A operand's 16 rows are its 8 tokens' halves (row i: token i / 2's half i % 2,
  // the other half's k zeros of the layout), so one MFMA gives both half-dots of the 8 tokens and lane l holds both
  // halves of tokens 2 (l / 16), 2 (l / 16) + 1 for its row: half the epilogue of a 16-token pass, every output live
  // (not IQ2_S at 16 lanes: its registers would cross 96, one wave a SIMD fewer - 1434 -> 1472 us at 7168 x 2048)
  constexpr bool kPass8 = !(T == kIQ2_S && L == 16);
  auto pass8 = [&](uint32_t c0) __attribute__((always_inline)) {
    const bool lives = (col % 2 == 0) == (quad < 2);
    const uint32_t t = c0 + col / 2, to = c0 + 2 * quad + (col & 1);
    const uint32_t voff = lives && t < n ? t * cols + 8 * quad : 0x80000000u;
    const uint32_t xoff = to < n ? to * nblk * 4 : 0x80000000u;
    const uint32_t kc8 = (uint32_t) (col / 2) < (uint32_t) C ? (uint32_t) (col / 2) : (uint32_t) (C - 1);
    float acc[C][2];
#pragma unroll
    for (int c = 0; c < C; c++) acc[c][0] = acc[c][1] = 0.0f;
    long an[PD];
    auto aload = [&](int slot, uint32_t s) __attribute__((always_inline)) {
      an[slot] = __builtin_bit_cast(long, __builtin_amdgcn_raw_buffer_load_b64(qr, voff, s * 32, 0));
    };
    auto sload = [&](uint32_t s0) __attribute__((always_inline)) {
      const uint32_t sb = s0 + W * kc8 < nblk ? s0 + W * kc8 : nblk - 1;
      return __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(dr, xoff == 0x80000000u ? xoff : xoff + sb * 4, 0, 0));
    };
    float sa = sload((uint32_t) wave), sb2;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < PD; i++) {
      aload(i, wave + W * i < nblk ? wave + W * i : nblk - 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    auto round = [&](uint32_t s0, float& sc, float& nx_sc) __attribute__((always_inline)) {
      nx_sc = sload(s0 + L < nblk ? s0 + L : s0);
#pragma unroll
      for (int c = 0; c < C; c++) {
        const uint32_t s = s0 + W * c;
        if (!FULL && s >= nblk) break;  // (uniform)
        const uint8_t* blk = brow + (s / per) * Block<T>::bytes;
        const int j = (int) (s % per);
        uint32_t w0, w1;
        chunk<T>((lbytes) blk, j, quad, grid, sm, w0, w1);
        const long b = (long) (((uint64_t) w1 << 32) | w0);
        float f0, f1;
        factors<T>((lbytes) blk, j, f0, f1);
        const float n0 = -__fmul_rn(f0, kBiasF), n1 = -__fmul_rn(f1, kBiasF);
        const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(an[c % PD], b, bias, 0, 0, 0);
        aload(c % PD, s + W * PD < nblk ? s + W * PD : s);
        const float s0_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(D[0]), n0), __builtin_fmaf(f1, __int_as_float(D[1]), n1));
        const float s1_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(D[2]), n0), __builtin_fmaf(f1, __int_as_float(D[3]), n1));
        acc[c][0] = fmac_bcast(acc[c][0], sc, s0_, 2 * c);
        acc[c][1] = fmac_bcast(acc[c][1], sc, s1_, 2 * c + 1);
      }
    };
    for (uint32_t s0 = (uint32_t) wave; s0 < nblk; s0 += 2 * L) {
      round(s0, sa, sb2);
      if (s0 + L >= nblk) break;
      round(s0 + L, sb2, sa);
    }
#pragma unroll
    for (int o = C / 2; o > 0; o >>= 1)
#pragma unroll
      for (int c = 0; c < o; c++)
#pragma unroll
        for (int p = 0; p < 2; p++) acc[c][p] = __fadd_rn(acc[c][p], acc[c + o][p]);
#pragma unroll
    for (int p = 0; p < 2; p++) part[(wave * 2 + p) * kWave + lane] = acc[0][p];
    __syncthreads();
    for (int p = (int) wave; p < 2; p += W) {
      float tv[W];
#pragma unroll
      for (int v = 0; v < W; v++) tv[v] = part[(v * 2 + p) * kWave + lane];
#pragma unroll
      for (int o = W / 2; o > 0; o >>= 1)
#pragma unroll
        for (int v = 0; v < o; v++) tv[v] = __fadd_rn(tv[v], tv[v + o]);
      const uint32_t tk = c0 + 2 * quad + p;
      if (tk < n) y[(uint64_t) (r0 + tk) * ys + row0 + col] = tv[0];
    }
  };
  auto pass8s = [&](uint32_t c0) __attribute__((always_inline)) {
    const bool lives = (col % 2 == 0) == (quad < 2);
    const uint32_t t = c0 + col / 2, to = c0 + 2 * quad + (col & 1);
    (void) t;
    const uint32_t xoff = to < n ? to * nblk * 4 : 0x80000000u;
    const uint32_t kc8 = (uint32_t) (col / 2) < (uint32_t) C ? (uint32_t) (col / 2) : (uint32_t) (C - 1);
    float acc[C][2];
#pragma unroll
    for (int c = 0; c < C; c++) acc[c][0] = acc[c][1] = 0.0f;
    // the round's A rows (8 tokens x L blocks x 32 bytes: one 16-byte word a thread) staged in LDS as in the 16-token
    // pass; lane l reads its token's 8 bytes there where its half lives, zeros elsewhere
    constexpr uint32_t kAS = 32 * L + 16;
    static_assert(C != 4 || 16 * L == kThreads, "one word a thread");
    uint8_t* abuf = smem + L_.part;
    const uint32_t tk = threadIdx.x / (2 * L), o16 = threadIdx.x % (2 * L);
    const uint32_t gof = c0 + tk < n ? (c0 + tk) * cols + o16 * 16 : 0x80000000u, lof = tk * kAS + o16 * 16;
    u32x4 st;
    auto gstage = [&](uint32_t b0) __attribute__((always_inline)) {
      st = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, gof + b0 * 32, 0, 0));
    };
    const uint32_t nr = (nblk + L - 1) / L;
    gstage(0);
    auto sload = [&](uint32_t s0) __attribute__((always_inline)) {
      const uint32_t sb = s0 + W * kc8 < nblk ? s0 + W * kc8 : nblk - 1;
      return __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(dr, xoff == 0x80000000u ? xoff : xoff + sb * 4, 0, 0));
    };
    float sa = sload((uint32_t) wave), sb2;
    auto round = [&](uint32_t r, float& sc, float& nx_sc) __attribute__((always_inline)) {
      __syncthreads();  // (the round before read by every wave)
      *(u32x4*) (abuf + lof) = st;
      __syncthreads();
      gstage(r + 1 < nr ? (r + 1) * L : r * L);
      const uint32_t s0 = r * L + wave;
      nx_sc = sload(s0 + L < nblk ? s0 + L : s0);
#pragma unroll
      for (int c = 0; c < C; c++) {
        const uint32_t s = s0 + W * c;
        if (!FULL && s >= nblk) break;  // (uniform)
        const uint8_t* blk = brow + (s / per) * Block<T>::bytes;
        const int j = (int) (s % per);
        uint32_t w0, w1;
        chunk<T>((lbytes) blk, j, quad, grid, sm, w0, w1);
        const long b = (long) (((uint64_t) w1 << 32) | w0);
        float f0, f1;
        factors<T>((lbytes) blk, j, f0, f1);
        const float n0 = -__fmul_rn(f0, kBiasF), n1 = -__fmul_rn(f1, kBiasF);
        const long av = *(const long*) (abuf + (col / 2) * kAS + (wave + W * c) * 32 + 8 * quad);
        const v4i D = __builtin_amdgcn_mfma_i32_16x16x32_i8(lives ? av : 0, b, bias, 0, 0, 0);
        const float s0_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(D[0]), n0), __builtin_fmaf(f1, __int_as_float(D[1]), n1));
        const float s1_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(D[2]), n0), __builtin_fmaf(f1, __int_as_float(D[3]), n1));
        acc[c][0] = fmac_bcast(acc[c][0], sc, s0_, 2 * c);
        acc[c][1] = fmac_bcast(acc[c][1], sc, s1_, 2 * c + 1);
      }
    };
    for (uint32_t r = 0; r < nr; r += 2) {  // (uniform: every wave meets every barrier)
      round(r, sa, sb2);
      if (r + 1 >= nr) break;
      round(r + 1, sb2, sa);
    }
    __syncthreads();  // (the last round's A rows read: the partial trees go where they were)
#pragma unroll
    for (int o = C / 2; o > 0; o >>= 1)
#pragma unroll
      for (int c = 0; c < o; c++)
#pragma unroll
        for (int p = 0; p < 2; p++) acc[c][p] = __fadd_rn(acc[c][p], acc[c + o][p]);
#pragma unroll
    for (int p = 0; p < 2; p++) part[(wave * 2 + p) * kWave + lane] = acc[0][p];
    __syncthreads();
    for (int p = (int) wave; p < 2; p += W) {
      float tv[W];
#pragma unroll
      for (int v = 0; v < W; v++) tv[v] = part[(v * 2 + p) * kWave + lane];
#pragma unroll
      for (int o = W / 2; o > 0; o >>= 1)
#pragma unroll
        for (int v = 0; v < o; v++) tv[v] = __fadd_rn(tv[v], tv[v + o]);
      const uint32_t tk = c0 + 2 * quad + p;
      if (tk < n) y[(uint64_t) (r0 + tk) * ys + row0 + col] = tv[0];
    }
  };
  for (uint32_t c0 = 0; c0 < n; c0 += TOK) {
    __syncthreads();  // (the slab's first pass; then the last pass's partial trees read before they are rewritten)
    if constexpr (kPass8) {
      if (n - c0 <= 8) {  // (uniform)
        if constexpr (kStageA && C == 4 && L == 32) pass8s(c0);  // (staged: IQ2_XXS 951-980 -> 932-967 us; slower at 16)
        else pass8(c0);
        continue;
      }
    }
    float acc[C][4];
#pragma unroll
    for (int c = 0; c < C; c++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[c][i] = 0.0f;
    if constexpr (kStageA) {
      // the round's A bytes (the pass's 16 tokens x L blocks x 32 bytes) staged in LDS by the whole workgroup with
      // 16-byte loads, the next round's in registers meanwhile; row t of the buffer token c0 + t's, kAS bytes apart
      const uint32_t to = c0 + 4 * quad + (col & 3);
      const uint32_t xoff = to < n ? to * nblk * 4 : 0x80000000u;
      constexpr int PW = C / 2;  // 16-byte words a thread stages a round: 16 x 2L words over W waves
      static_assert(C % 2 == 0, "whole words a thread");
      constexpr uint32_t kAS = 32 * L + 16;
      uint8_t* abuf = smem + L_.part;
      uint32_t gof[PW], lof[PW];
#pragma unroll
      for (int u = 0; u < PW; u++) {
        const uint32_t wi = threadIdx.x + u * kThreads, tk = wi / (2 * L), o16 = wi % (2 * L);
        gof[u] = c0 + tk < n ? (c0 + tk) * cols + o16 * 16 : 0x80000000u;
        lof[u] = tk * kAS + o16 * 16;
      }
      u32x4 st[PW];
      auto gstage = [&](uint32_t b0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < PW; u++)
          st[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qr, gof[u] + b0 * 32, 0, 0));
      };
      auto sload = [&](uint32_t s0) __attribute__((always_inline)) {
        const uint32_t sb = s0 + W * kc < nblk ? s0 + W * kc : nblk - 1;  // (per lane: a vector offset)
        return __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(dr, xoff == 0x80000000u ? xoff : xoff + sb * 4, 0, 0));
      };
      const uint32_t nr = (nblk + L - 1) / L;
      gstage(0);
      float sa = sload((uint32_t) wave), sb2;
      auto round = [&](uint32_t r, float& sc, float& nx_sc) __attribute__((always_inline)) {
        __syncthreads();  // (the round before read by every wave)
#pragma unroll
        for (int u = 0; u < PW; u++) *(u32x4*) (abuf + lof[u]) = st[u];
        __syncthreads();
        gstage(r + 1 < nr ? (r + 1) * L : r * L);  // (past the last round: the last again, unused)
        const uint32_t s0 = r * L + wave;
        nx_sc = sload(s0 + L < nblk ? s0 + L : s0);
#pragma unroll
        for (int c = 0; c < C; c++) {
          const uint32_t s = s0 + W * c;  // logical lane wave + W c
          if (!FULL && s >= nblk) break;  // (uniform in the wave)
          const long a = *(const long*) (abuf + col * kAS + (wave + W * c) * 32 + 8 * quad);
          const uint8_t* blk = brow + (s / per) * Block<T>::bytes;
          const int j = (int) (s % per);
          uint32_t w0, w1;
          chunk<T>((lbytes) blk, j, quad, grid, sm, w0, w1);
          const long b = (long) (((uint64_t) w1 << 32) | w0);
          const long blo = quad < 2 ? b : 0, bhi = quad < 2 ? 0 : b;  // (k 0 .. 15: the first half, 16 .. 31 the second)
          float f0, f1;
          factors<T>((lbytes) blk, j, f0, f1);
          const float n0 = -__fmul_rn(f0, kBiasF), n1 = -__fmul_rn(f1, kBiasF);
          const v4i Dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, blo, bias, 0, 0, 0);
          const v4i Dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bhi, bias, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float s_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(Dl[i]), n0),
                                       __builtin_fmaf(f1, __int_as_float(Dh[i]), n1));
            acc[c][i] = fmac_bcast(acc[c][i], sc, s_, 4 * c + i);
          }
        }
      };
      for (uint32_t r = 0; r < nr; r += 2) {  // (uniform: every wave meets every barrier)
        round(r, sa, sb2);
        if (r + 1 >= nr) break;
        round(r + 1, sb2, sa);
      }
      __syncthreads();  // (the last round's A rows read: the partial trees go where they were)
    } else {
      // every load made on every path (a token past the count at an offset past the descriptor's end: zeros, no access)
      const uint32_t voff = c0 + col < n ? (c0 + col) * cols + 8 * quad : 0x80000000u;
      const uint32_t to = c0 + 4 * quad + (col & 3);
      const uint32_t xoff = to < n ? to * nblk * 4 : 0x80000000u;
      long an[PD];
      auto aload = [&](int slot, uint32_t s) __attribute__((always_inline)) {
        an[slot] = __builtin_bit_cast(long, __builtin_amdgcn_raw_buffer_load_b64(qr, voff, s * 32, 0));
      };
      auto sload = [&](uint32_t s0) __attribute__((always_inline)) {
        const uint32_t sb = s0 + W * kc < nblk ? s0 + W * kc : nblk - 1;  // (per lane: a vector offset)
        return __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(dr, xoff == 0x80000000u ? xoff : xoff + sb * 4, 0, 0));
      };
      // (the first round's scales, then the ring in slot order: the order every round issues them)
      float sa = sload((uint32_t) wave), sb2;
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < PD; i++) {
        aload(i, wave + W * i < nblk ? wave + W * i : nblk - 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      auto round = [&](uint32_t s0, float& sc, float& nx_sc) __attribute__((always_inline)) {
        nx_sc = sload(s0 + L < nblk ? s0 + L : s0);  // (the next round's, a round ahead, into the other register)
#pragma unroll
        for (int c = 0; c < C; c++) {
          const uint32_t s = s0 + W * c;  // logical lane wave + W c
          if (!FULL && s >= nblk) break;  // (uniform; FULL: every round whole)
          const uint8_t* blk = brow + (s / per) * Block<T>::bytes;
          const int j = (int) (s % per);
          uint32_t w0, w1;
          chunk<T>((lbytes) blk, j, quad, grid, sm, w0, w1);
          const long b = (long) (((uint64_t) w1 << 32) | w0);
          const long blo = quad < 2 ? b : 0, bhi = quad < 2 ? 0 : b;  // (k 0 .. 15: the first half, 16 .. 31 the second)
          float f0, f1;
          factors<T>((lbytes) blk, j, f0, f1);
          const float n0 = -__fmul_rn(f0, kBiasF), n1 = -__fmul_rn(f1, kBiasF);
          const v4i Dl = __builtin_amdgcn_mfma_i32_16x16x32_i8(an[c % PD], blo, bias, 0, 0, 0);
          const v4i Dh = __builtin_amdgcn_mfma_i32_16x16x32_i8(an[c % PD], bhi, bias, 0, 0, 0);
          aload(c % PD, s + W * PD < nblk ? s + W * PD : s);  // (past the last block: loaded again, unused)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float s_ = __fadd_rn(__builtin_fmaf(f0, __int_as_float(Dl[i]), n0),
                                       __builtin_fmaf(f1, __int_as_float(Dh[i]), n1));
            acc[c][i] = fmac_bcast(acc[c][i], sc, s_, 4 * c + i);
          }
        }
      };
      for (uint32_t s0 = (uint32_t) wave; s0 < nblk; s0 += 2 * L) {
        round(s0, sa, sb2);
        if (s0 + L >= nblk) break;
        round(s0 + L, sb2, sa);
      }
    }
    // the tree's levels L/2 .. W within the wave: chains c and c + o (logical lanes ll and ll ^ W o)
#pragma unroll
    for (int o = C / 2; o > 0; o >>= 1)
#pragma unroll
      for (int c = 0; c < o; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[c][i] = __fadd_rn(acc[c][i], acc[c + o][i]);
    // levels W/2 .. 1 across the waves through LDS, two of the lane's four outputs at a time
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      if (hh) __syncthreads();  // (the first pair read)
#pragma unroll
      for (int p = 0; p < 2; p++) part[(wave * 2 + p) * kWave + lane] = acc[0][2 * hh + p];
      __syncthreads();
      for (int p = (int) wave; p < 2; p += W) {
        float t[W];
#pragma unroll
        for (int v = 0; v < W; v++) t[v] = part[(v * 2 + p) * kWave + lane];
#pragma unroll
        for (int o = W / 2; o > 0; o >>= 1)
#pragma unroll
          for (int v = 0; v < o; v++) t[v] = __fadd_rn(t[v], t[v + o]);
        const uint32_t tk = c0 + 4 * quad + 2 * hh + p;
        if (tk < n) y[(uint64_t) (r0 + tk) * ys + row0 + col] = t[0];
      }
    }
  }
}

template <uint32_t T, int L, int G, int W>
bool launch(const void* const* w, const int32_t* cnt, const int32_t* xrow, uint32_t n_mat, uint32_t rows,
            uint32_t cols, const int8_t* q, const float* d, float* y, uint32_t ys, hipStream_t s) {
  const Lds<G, W, G == 1 && stage_a<T, L>() ? L : 0> l((uint32_t) row_bytes<T>(cols), grid_bytes_of<T>());
  if (l.total > 160 * 1024) return false;
  auto pick = [&]() {
    if constexpr (G == 1) return (cols / 32) % L == 0 ? kernel16<T, L, W, true> : kernel16<T, L, W, false>;
    else return (cols / 32) % L == 0 ? kernel<T, L, G, W, true> : kernel<T, L, G, W, false>;
  };
  auto k = pick();
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
  constexpr Shape s32 = shape<T, 32>(), s16 = shape<T, 16>();
  return cols >= 4096 ? launch<T, 32, s32.g, s32.w>(w, cnt, xrow, n_mat, rows, cols, q, d, y, ys, s)
                      : launch<T, 16, s16.g, s16.w>(w, cnt, xrow, n_mat, rows, cols, q, d, y, ys, s);
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
