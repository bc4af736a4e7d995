// Exact float32 16 x 16 tile products (v_mfma_f32_16x16x4_f32) with operand
// accessors, for the float32 paths: the Level B matrix form on float32 token
// streams (chunk_f32.hip) and the exact WY/UT mode (wy.hip).
//
// Lane layout of v_mfma_f32_16x16x4_f32 (lane l, i = l % 16, G = l / 16):
// A operand A[i][G], B operand B[G][i], result D[4G + j][i] in register j.
#pragma once
#include "tile.h"

namespace gmdn {

// acc += sum_k A(r, k) B(k, c) over a 16 x 16 tile, k = 0 .. K-1 in steps
// of 4; a(r, k) / b(k, c) return the lane's operand element for tile row r /
// tile column c.
template <int K, class FA, class FB>
GMDN_DEV f32x4 mm16(FA a, FB b, f32x4 acc) {
  const int l = lane_id(), i = l & 15, G = l >> 4;
#pragma unroll 4
  for (int k = 0; k < K; k += 4) acc = mfma_f32(a(i, k + G), b(k + G, i), acc);
  return acc;
}

// D-layout tile -> row-major float matrix X (row stride ld) at (r0, c0)
GMDN_DEV void st_tile(float* X, int64_t ld, int r0, int c0, const f32x4& t) {
  const int l = lane_id(), c = l & 15, G = l >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) X[(int64_t)(r0 + 4 * G + j) * ld + c0 + c] = t[j];
}

// row-major float matrix X at (r0, c0) -> D-layout tile
GMDN_DEV f32x4 ld_tile(const float* X, int64_t ld, int r0, int c0) {
  const int l = lane_id(), c = l & 15, G = l >> 4;
  f32x4 t;
#pragma unroll
  for (int j = 0; j < 4; ++j) t[j] = X[(int64_t)(r0 + 4 * G + j) * ld + c0 + c];
  return t;
}

// Sum over the 16 lanes of each lane group (l / 16): every lane of the group
// receives the group's sum.  Every lane of the wave must be active.
GMDN_DEV float row16_sum(float x) {
  x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_mov<0x124>(x);  // row_ror:4
  x += dpp_mov<0x128>(x);  // row_ror:8
  return x;
}

// Inclusive prefix sum over the 64 lanes of a wave.
GMDN_DEV float wave_incl_scan(float x) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o, 64);
    if (l >= o) x += y;
  }
  return x;
}

}  // namespace gmdn
