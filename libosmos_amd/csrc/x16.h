// libosmos MI355X - the f16 activations' tiled layout that mm reads (reference include/osmos/gpu/mm.h:122-124): token
// t's column c of a matrix xts columns wide at (t / 16) 16 xts + (c / 16) 256 + (t % 16) 16 + c % 16 halves - each
// 16 x 16 fragment contiguous, a lane's 8 columns one 16-byte load. shared by mm.hip (mm_x16, mm_x16_rows, the
// kernels' B operand) and moe.hip (q4x_swiglu_rows).
#pragma once
#include "common.h"

namespace osm {

constexpr uint32_t kX16Tile = 16;

__host__ __device__ inline uint64_t x16_at(uint32_t t, uint32_t c, uint32_t xts) {
  return (uint64_t) (t / kX16Tile) * kX16Tile * xts + (c / 16) * 256 + (t % kX16Tile) * 16 + c % 16;
}

// a value's f16 (nearest, ties to even) and whether the value is past f16's largest finite, 65504, or not a number
// (the reference's overflow rule, kernels/mm.h:47-50: the value itself, before rounding - 65510 is flagged though it
// rounds to 65504)
__device__ inline _Float16 x16_round(float v, bool& over) {
  over |= !(__builtin_fabsf(v) <= 65504.0f);
  return (_Float16) v;
}

}  // namespace osm
