// Wave64 MFMA tile primitives for gfx950 (CDNA4).
//
// Every product in the scan kernels is built from 16x16 output tiles of
// v_mfma_f32_16x16x32_bf16 (or v_mfma_f32_16x16x4_f32 for the exact-fp32
// mode).  Lane layouts, checked on MI355X hardware:
//
//   16x16x32 bf16   A: lane l holds A[l%16][8(l/16)+i], i=0..7
//                   B: lane l holds B[8(l/16)+i][l%16]
//                   D: lane l holds D[4(l/16)+j][l%16], j=0..3
//   16x16x4  f32    A: A[l%16][l/16]  B: B[l/16][l%16]  D as above
//
// "D layout": a 16x16 fp32 tile with lane <-> column (l%16) and the four
// accumulator registers <-> rows 4G+j (G = l/16).
//
// Chaining without a shuffle.  The contraction index of an MFMA may be
// permuted freely as long as both operands use the same permutation.  All
// 32-wide k-blocks here use the "pair order": lane group G holds the k
// indices {4G..4G+3} in slots 0..3 and {16+4G..16+4G+3} in slots 4..7.  Then
// two D-layout tiles stacked along k (rows 0..15 and 16..31) ARE an operand
// whose free index is the tile column: no LDS round trip is needed to feed
// one product's result into the next as the k side.  Operands read from
// memory use the same pair order (two 8-byte reads per lane, or two
// ds_read_b64_tr_b16 transposing reads for a k-major source).
//
// ds_read_b64_tr_b16 (checked on hardware): within each 16-lane group,
// output lane i element j is element i%4 of the 8-byte vector addressed by
// lane 4j+i/4.  So if lane (i, G) passes &X[r0 + i/4][c0 + 4(i%4)], it
// receives X[r0 + j][c0 + i] for j = 0..3: a column of a row-major tile.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gmdn {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define GMDN_DEV __device__ __forceinline__

GMDN_DEV int lane_id() { return threadIdx.x & 63; }
GMDN_DEV int wave_id() { return threadIdx.x >> 6; }

GMDN_DEV f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

GMDN_DEV f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
GMDN_DEV f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- operands
// An operand in split precision: value ~= hi + lo, both bf16.  P = 1 keeps
// only hi (inputs that are exact bf16); P = 2 keeps both.
template <int P>
struct Op {
  bf16x8 v[P];
};

// acc += a * b with split operands; the lo*lo term (2^-16 relative) is dropped.
template <int PA, int PB>
GMDN_DEV f32x4 mma(const Op<PA>& a, const Op<PB>& b, f32x4 acc) {
  acc = mfma(a.v[0], b.v[0], acc);
  if constexpr (PB == 2) acc = mfma(a.v[0], b.v[1], acc);
  if constexpr (PA == 2) acc = mfma(a.v[1], b.v[0], acc);
  return acc;
}

GMDN_DEV bf16 to_bf16(float x) { return (bf16)x; }
GMDN_DEV float from_bf16(bf16 x) { return (float)x; }

// Split x into hi + lo (both bf16).
GMDN_DEV void split2(float x, bf16& hi, bf16& lo) {
  hi = (bf16)x;
  lo = (bf16)(x - (float)hi);
}

// Two D-layout tiles stacked along k (t0: k rows 0..15, t1: rows 16..31),
// scaled per k-row by s0/s1 (lane's four rows each) -> pair-order operand.
template <int P>
GMDN_DEV Op<P> pack_tiles(const f32x4& t0, const f32x4& t1) {
  Op<P> r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (P == 1) {
      r.v[0][j] = (bf16)t0[j];
      r.v[0][4 + j] = (bf16)t1[j];
    } else {
      bf16 h, l;
      split2(t0[j], h, l);
      r.v[0][j] = h;
      r.v[1][j] = l;
      split2(t1[j], h, l);
      r.v[0][4 + j] = h;
      r.v[1][4 + j] = l;
    }
  }
  return r;
}

template <int P>
GMDN_DEV Op<P> pack_tiles_scaled(const f32x4& t0, const f32x4& t1, const f32x4& s0, const f32x4& s1) {
  return pack_tiles<P>(t0 * s0, t1 * s1);
}

// ------------------------------------------------------------ LDS readers
// Row read: lane (r = l%16, G) takes X[r][k] for k in pair order of the
// 32-wide block starting at column k0.  X is row-major bf16 with leading
// dimension ld (elements).  Two 8-byte reads.
GMDN_DEV bf16x8 lds_row(const bf16* X, int ld, int r0, int k0) {
  const int l = lane_id();
  const bf16* p = X + (r0 + (l & 15)) * ld + k0 + 4 * (l >> 4);
  bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
  bf16x4 b = *reinterpret_cast<const bf16x4*>(p + 16);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Column read: lane (c = l%16, G) takes X[k][c0 + c] for k in pair order of
// the 32-row block starting at row k0 (X row-major, leading dim ld).  Two
// ds_read_b64_tr_b16.
GMDN_DEV bf16x8 lds_col(const bf16* X, int ld, int k0, int c0) {
  const int l = lane_id();
  const int i = l & 15, G = l >> 4;
  const bf16* p0 = X + (k0 + 4 * G + (i >> 2)) * ld + c0 + 4 * (i & 3);
  const bf16* p1 = p0 + 16 * ld;
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
  s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
  bf16x4 ab = __builtin_bit_cast(bf16x4, a);
  bf16x4 bb = __builtin_bit_cast(bf16x4, b);
  return bf16x8{ab[0], ab[1], ab[2], ab[3], bb[0], bb[1], bb[2], bb[3]};
}

// D-layout tile from a row-major bf16 LDS tile X[row][col]: lane (c, G)
// gets X[r0 + 4G + j][c0 + c] (one transposing read).
GMDN_DEV f32x4 lds_dtile(const bf16* X, int ld, int r0, int c0) {
  const int l = lane_id();
  const int i = l & 15, G = l >> 4;
  const bf16* p = X + (r0 + 4 * G + (i >> 2)) * ld + c0 + 4 * (i & 3);
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  bf16x4 ab = __builtin_bit_cast(bf16x4, a);
  return f32x4{(float)ab[0], (float)ab[1], (float)ab[2], (float)ab[3]};
}

template <int P>
GMDN_DEV Op<P> lds_row_op(const bf16* const* planes, int ld, int r0, int k0) {
  Op<P> r;
#pragma unroll
  for (int p = 0; p < P; ++p) r.v[p] = lds_row(planes[p], ld, r0, k0);
  return r;
}
template <int P>
GMDN_DEV Op<P> lds_col_op(const bf16* const* planes, int ld, int k0, int c0) {
  Op<P> r;
#pragma unroll
  for (int p = 0; p < P; ++p) r.v[p] = lds_col(planes[p], ld, k0, c0);
  return r;
}

// ------------------------------------------------------------ reductions
GMDN_DEV float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

// Sum over the 4 lane groups (G) of a value held per lane: result equal in
// all lanes sharing l%16.
GMDN_DEV float group_sum(float x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

}  // namespace gmdn
