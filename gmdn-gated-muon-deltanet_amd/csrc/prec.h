// Precision policies and swizzled fp32 LDS matrices for the fp32-state
// kernels (the drop-in chunk scan and the Newton-Schulz engine).
//
// A "k-block" is 32 contraction indices in the pair order of tile.h
// (lane group G holds k = 4G..4G+3 and 16+4G..16+4G+3).  Every policy
// exposes
//   Op                 one lane's share of a 16x32 (or 32x16) operand
//   from8(float[8])    operand from the lane's 8 fp32 values in pair order
//   pack(t0, t1)       operand from two D-layout tiles stacked along k
//   mma(a, b, acc)     acc += a * b over the k-block
//
//   PrecX3   bf16x3 split products: x = hi + lo, a*b ~ ah*bh + ah*bl + al*bh
//            (three v_mfma_f32_16x16x32_bf16; ~2^-16 relative per product).
//            The build's mapping of the reference's 'tf32' precision.
//   PrecF32  eight v_mfma_f32_16x16x4_f32 (exact fp32 products), the
//            mapping of 'ieee'.  MFMA s (0..7) takes pair slot s, so the
//            same D-layout chaining applies.
#pragma once
#include "tile.h"

namespace gmdn {

struct PrecX3 {
  struct Op {
    bf16x8 hi, lo;
  };
  static GMDN_DEV Op from8(const float (&x)[8]) {
    Op r;
    bf16x4 h0, l0, h1, l1;
    split4(f32x4{x[0], x[1], x[2], x[3]}, h0, l0);
    split4(f32x4{x[4], x[5], x[6], x[7]}, h1, l1);
    r.hi = cat8(h0, h1);
    r.lo = cat8(l0, l1);
    return r;
  }
  static GMDN_DEV Op pack(const f32x4& t0, const f32x4& t1) {
    float x[8] = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
    return from8(x);
  }
  static GMDN_DEV f32x4 mma(const Op& a, const Op& b, f32x4 acc) {
    acc = mfma(a.hi, b.hi, acc);
    acc = mfma(a.hi, b.lo, acc);
    acc = mfma(a.lo, b.hi, acc);
    return acc;
  }
};

struct PrecF32 {
  struct Op {
    float v[8];
  };
  static GMDN_DEV Op from8(const float (&x)[8]) {
    Op r;
#pragma unroll
    for (int s = 0; s < 8; ++s) r.v[s] = x[s];
    return r;
  }
  static GMDN_DEV Op pack(const f32x4& t0, const f32x4& t1) {
    Op r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      r.v[j] = t0[j];
      r.v[4 + j] = t1[j];
    }
    return r;
  }
  static GMDN_DEV f32x4 mma(const Op& a, const Op& b, f32x4 acc) {
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = mfma_f32(a.v[s], b.v[s], acc);
    return acc;
  }
};

template <int PREC>
struct PrecSel;
template <>
struct PrecSel<0> {
  using T = PrecX3;
};
template <>
struct PrecSel<1> {
  using T = PrecF32;
};

// ------------------------------------------------ swizzled fp32 LDS matrix
// Row-major D x D fp32 in LDS without padding.  The 16-byte group q of row
// r is stored at group q ^ (r & SW) with SW = min(16, D/4) - 1: 16 rows read
// at one column group (row reads) hit 16 different bank groups, and 4 rows
// 4 apart read at 4 consecutive groups (column reads) hit 4 disjoint ranges.
template <int D>
struct SwzMat {
  static constexpr int SW = (D / 4 < 16 ? D / 4 : 16) - 1;
  static GMDN_DEV int off(int r, int c) {
    return r * D + ((((c >> 2) ^ (r & SW)) << 2) | (c & 3));
  }
  // physical 16-byte group p of row r holds logical group p ^ (r & SW)
  static GMDN_DEV int logical_group(int r, int p) { return p ^ (r & SW); }
};

// Plain row-major D x D fp32 matrix (global-memory workspaces).
template <int D>
struct PlainMat {
  static GMDN_DEV int off(int r, int c) { return r * D + c; }
};

// Operand whose k runs down the rows: lane (c, G) takes X[k0 + pair(G, s)][c0 + c].
template <class L>
GMDN_DEV void mat_colf(const float* X, int k0, int c0, float (&x)[8]) {
  const int l = lane_id(), c = l & 15, G = l >> 4;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int k = k0 + (s < 4 ? 4 * G + s : 16 + 4 * G + (s - 4));
    x[s] = X[L::off(k, c0 + c)];
  }
}

// Operand whose k runs along a row: lane (r, G) takes X[r0 + r][k0 + pair(G, s)].
template <class L>
GMDN_DEV void mat_rowf(const float* X, int r0, int k0, float (&x)[8]) {
  const int l = lane_id(), r = r0 + (l & 15), G = l >> 4;
  const f32x4 a = *reinterpret_cast<const f32x4*>(X + L::off(r, k0 + 4 * G));
  const f32x4 b = *reinterpret_cast<const f32x4*>(X + L::off(r, k0 + 16 + 4 * G));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    x[j] = a[j];
    x[4 + j] = b[j];
  }
}

// Store a D-layout tile t of M^T (rows = columns of M) as rows of M: lane
// (r, G) writes M[r0 + r][c0 + 4G .. c0 + 4G + 3] (one 16-byte write).
template <class L>
GMDN_DEV void mat_store_tileT(float* X, int r0, int c0, const f32x4& t) {
  const int l = lane_id();
  *reinterpret_cast<f32x4*>(X + L::off(r0 + (l & 15), c0 + 4 * (l >> 4))) = t;
}

template <class P, class L>
GMDN_DEV typename P::Op col_op(const float* X, int k0, int c0) {
  float x[8];
  mat_colf<L>(X, k0, c0, x);
  return P::from8(x);
}
template <class P, class L>
GMDN_DEV typename P::Op row_op(const float* X, int r0, int k0) {
  float x[8];
  mat_rowf<L>(X, r0, k0, x);
  return P::from8(x);
}

// Asynchronous copy of a contiguous D x D fp32 matrix from global memory into
// a swizzled LDS matrix with gfx950's global_load_lds_dwordx4 (lds_dma16):
// each wave instruction writes 64 consecutive 16-byte LDS groups, and each
// lane fetches the global group that belongs at its slot.  Caller waits
// (wait_vmem) and synchronises before reading.
template <int D, int NTHREADS>
GMDN_DEV void lds_dma_matrix(float* lds, const float* g) {
  constexpr int GROUPS = D * D / 4;        // 16-byte groups in the matrix
  constexpr int PER_ROW = D / 4;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  static_assert(GROUPS % NTHREADS == 0, "matrix must split evenly over the block");
#pragma unroll
  for (int base = 0; base < GROUPS; base += NTHREADS) {
    const int p = base + w * 64 + l;       // physical group this lane fills
    const int r = p / PER_ROW;
    const int q = SwzMat<D>::logical_group(r, p % PER_ROW);
    lds_dma16(g + r * D + q * 4, lds + (base + w * 64) * 4);
  }
}

}  // namespace gmdn
