// Block-cooperative Newton-Schulz msign and its VJP for a D x D fp32 matrix
// (reference fast_scan.py:63-69 forward, :107-131 VJP).
//
// D/16 waves; wave w owns rows 16w..16w+15 of every matrix and holds them as
// D-layout tiles of the transpose (lane <-> row, registers <-> columns), the
// same layout as the scan state.  Matrices that every wave reads in full are
// published through a shared D x D store of layout L (swizzled LDS or a plain
// global workspace), one barrier per publication.
//
// Forward step (P = X X^T is symmetric, so each wave's column block of P is
// computable from the published X and its own rows):
//   Pc  = P[:, rows]  = X_pub (row reads) x X^T_own
//   P2c = (P P)[:, rows] = P_pub (row reads) x Pc
//   X^T <- a X^T + X^T Z,  Z = b P + c P^2  (X_pub column reads x Zc)
//
// VJP step for iterate X_k with incoming Xbar (see oracle/scan.py msign_vjp):
//   Bbar = Xbar X_k^T, Abar = b Bbar + c (Bbar P + P Bbar)
//   Xbar <- a Xbar + Bm Xbar + (Abar + Abar^T) X_k,  Bm = b P + c P^2
// Each wave forms the column block [:, rows] of Bm and of Abar + Abar^T from
// its own rows plus the published X_k, Xbar, P and Bbar.
#pragma once
#include "prec.h"

namespace gmdn {

constexpr float NS_A = 3.4445f, NS_B = -4.7750f, NS_C = 2.0315f;  // fast_scan.py:32

template <int NW>
GMDN_DEV float block_sum(float x, float* red) {
  x = wave_sum(x);
  if (lane_id() == 0) red[wave_id()] = x;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int q = 0; q < NW; ++q) t += red[q];
  __syncthreads();
  return t;
}

// block_sum of two values under one pair of barriers (red: 2 NW floats); each
// sum is formed in the order block_sum uses
template <int NW>
GMDN_DEV f32x2 block_sum2(float x, float y, float* red) {
  const f32x2 s = wave_sum2(x, y);
  if (lane_id() == 0) {
    red[2 * wave_id()] = s[0];
    red[2 * wave_id() + 1] = s[1];
  }
  __syncthreads();
  f32x2 t = {0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    t[0] += red[2 * q];
    t[1] += red[2 * q + 1];
  }
  __syncthreads();
  return t;
}

template <class P, class L, int D>
struct NSBlock {
  static constexpr int NT = D / 16;
  static constexpr int NKB = D / 32;
  using Op = typename P::Op;

  template <int N>
  static GMDN_DEV void pack_all(const f32x4 (&t)[N], Op (&o)[N / 2]) {
#pragma unroll
    for (int kb = 0; kb < N / 2; ++kb) o[kb] = P::pack(t[2 * kb], t[2 * kb + 1]);
  }

  static GMDN_DEV void publish(float* M, const f32x4 (&t)[NT]) {
    const int r0 = 16 * wave_id();
#pragma unroll
    for (int c = 0; c < NT; ++c) mat_store_tileT<L>(M, r0, 16 * c, t[c]);
  }

  // own rows of `pub` times the wave's operand: tile [r'][r] = sum_k pub[r'][k] B[k][r]
  static GMDN_DEV f32x4 rowprod(const float* pub, int tr, const Op (&B)[NKB]) {
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc = P::mma(row_op<P, L>(pub, 16 * tr, 32 * kb), B[kb], acc);
    return acc;
  }
  // tile [c][r] = sum_k pub[k][c] B[k][r]
  static GMDN_DEV f32x4 colprod(const float* pub, int tc, const Op (&B)[NKB], f32x4 acc) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc = P::mma(col_op<P, L>(pub, 32 * kb, 16 * tc), B[kb], acc);
    return acc;
  }

  // One quintic step on the wave's rows XT (D-layout tiles of X^T).
  static GMDN_DEV void step(f32x4 (&XT)[NT], float* XM, float* PM) {
    const int r0 = 16 * wave_id();
    publish(XM, XT);
    __syncthreads();
    Op Bx[NKB];
    pack_all(XT, Bx);
    f32x4 Pc[NT];
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) Pc[tr] = rowprod(XM, tr, Bx);
    // P is symmetric: the column block is also the wave's rows of P
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) mat_store_tileT<L>(PM, r0, 16 * tr, Pc[tr]);
    __syncthreads();
    Op Bp[NKB];
    pack_all(Pc, Bp);
    f32x4 Z[NT];
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) Z[tr] = NS_B * Pc[tr] + NS_C * rowprod(PM, tr, Bp);
    Op Bz[NKB];
    pack_all(Z, Bz);
#pragma unroll
    for (int tc = 0; tc < NT; ++tc) XT[tc] = colprod(XM, tc, Bz, NS_A * XT[tc]);
    __syncthreads();
  }

  // One reverse step: XbT (D-layout tiles of Xbar^T, own rows) updated in
  // place given iterate XkT (own rows).  Uses four shared stores.
  static GMDN_DEV void vjp_step(const f32x4 (&XkT)[NT], f32x4 (&XbT)[NT], float* XM, float* PM,
                                float* XbM, float* BM) {
    const int r0 = 16 * wave_id();
    publish(XM, XkT);
    publish(XbM, XbT);
    __syncthreads();
    Op Bk[NKB], Bxb[NKB];
    pack_all(XkT, Bk);
    pack_all(XbT, Bxb);
    f32x4 Pc[NT], BR[NT], BC[NT];
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) {
      Pc[tr] = rowprod(XM, tr, Bk);    // P[r'][r]
      BR[tr] = rowprod(XM, tr, Bxb);   // Bbar[r][r'] (own row block, transposed)
      BC[tr] = rowprod(XbM, tr, Bk);   // Bbar[r'][r] (own column block)
    }
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) {
      mat_store_tileT<L>(PM, r0, 16 * tr, Pc[tr]);
      mat_store_tileT<L>(BM, r0, 16 * tr, BR[tr]);  // rows of Bbar
    }
    __syncthreads();
    Op Bp[NKB], Bbr[NKB], Bbc[NKB];
    pack_all(Pc, Bp);
    pack_all(BR, Bbr);
    pack_all(BC, Bbc);
    f32x4 Bm[NT], Ssym[NT];
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) {
      Bm[tr] = NS_B * Pc[tr] + NS_C * rowprod(PM, tr, Bp);
      f32x4 t = rowprod(BM, tr, Bp);                      // sum Bbar[r'][r''] P[r''][r]
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const Op pr = row_op<P, L>(PM, 16 * tr, 32 * kb);  // P[r'][r'']
        acc = P::mma(pr, Bbc[kb], acc);                  // sum P[r'][r''] Bbar[r''][r]
        acc = P::mma(pr, Bbr[kb], acc);                  // sum P[r'][r''] Bbar[r][r'']
        acc = P::mma(col_op<P, L>(BM, 32 * kb, 16 * tr), Bp[kb], acc);  // sum Bbar[r''][r'] P[r''][r]
      }
      Ssym[tr] = NS_B * (BC[tr] + BR[tr]) + NS_C * (t + acc);
    }
    Op Bbm[NKB], Bs[NKB];
    pack_all(Bm, Bbm);
    pack_all(Ssym, Bs);
#pragma unroll
    for (int tc = 0; tc < NT; ++tc) {
      f32x4 acc = colprod(XbM, tc, Bbm, NS_A * XbT[tc]);
      XbT[tc] = colprod(XM, tc, Bs, acc);
    }
    __syncthreads();
  }
};

// The forward quintic step with bf16x3 products and the shared matrices kept
// as split bf16 planes in LDS (hi plane then lo plane, each D x D in the
// 16-byte-group XOR swizzle RowSwz).  Within every 32 columns
// the 4-column blocks are stored in the order 0 4 1 5 2 6 3 7, so the eight
// values of a row operand in the pair k order of the register operands
// (columns 4G .. 4G+3 and 16+4G .. 16+4G+3) are one 16-byte row read per
// plane; column operands are two transposing reads per plane.  The
// publishing wave splits its own rows once.  A row's swizzle depends only on
// the row modulo 16, so each lane keeps one LDS base per distinct column
// pattern and row tiles are immediate offsets.
template <int D>
struct NSSplit {
  static constexpr int NT = D / 16;
  static constexpr int NKB = D / 32;
  static constexpr uint32_t PLANE = (uint32_t)D * D * 2;  // bytes of one plane
  static constexpr uint32_t BYTES = 2 * PLANE;             // one published matrix
  static constexpr uint32_t ROWB = D * 2;                  // bytes per row of a plane
  using L = RowSwz<D>;
  using P = PrecX3;
  using Op = P::Op;
  static_assert(L::MASK < 16, "row tiles of 16 must keep the swizzle");

  uint32_t prow[NKB];  // row reads: row lc, columns 32 kb + {4G .. 4G+3, 16+4G .. 16+4G+3}
  uint32_t pcol[NT];   // column reads: row 4G + lc/4, columns 16 tc + 4 (lc & 3) ..
  uint32_t ppub[NT];   // publishing: row 16 w + lc, columns 16 c + 4G ..

  // stored column of the 4-column block that starts at column c
  static GMDN_DEV int scol(int c) {
    const int b = (c >> 2) & 7;
    return (c & ~31) + 4 * (2 * (b & 3) + (b >> 2));
  }
  // LDS byte offset of (row r, the block starting at column c) in a plane
  static GMDN_DEV uint32_t off(int r, int c) { return swz_off<L>(r, scol(c)); }

  GMDN_DEV NSSplit() {
    const int l = lane_id(), lc = l & 15, G = l >> 4, w = wave_id();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) prow[kb] = swz_off<L>(lc, 32 * kb + 8 * G);  // stored slots 2G, 2G+1
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      pcol[t] = off(4 * G + (lc >> 2), 16 * t + 4 * (lc & 3));
      ppub[t] = off(16 * w + lc, 16 * t + 4 * G);
    }
  }

  template <int N>
  static GMDN_DEV void pack_all(const f32x4 (&t)[N], Op (&o)[N / 2]) {
#pragma unroll
    for (int kb = 0; kb < N / 2; ++kb) o[kb] = P::pack(t[2 * kb], t[2 * kb + 1]);
  }
  // All NTHR threads: a row-major fp32 D x D matrix in global memory -> split
  // planes at m (16-byte loads; thread j takes pieces j, j + NTHR, ...).
  template <int NTHR>
  static GMDN_DEV void stage(lds_ptr m, const float* g) {
    constexpr int PR = D / 4;  // 4-float pieces per row
    static_assert((D * PR) % NTHR == 0 && NTHR % PR == 0 && (NTHR / PR) % 16 == 0,
                  "pieces split evenly, in row steps that keep the swizzle");
    const int j = threadIdx.x, r = j / PR, c = (j % PR) * 4;
    const float* src = g + r * D + c;
    const uint32_t dst = off(r, c);
    constexpr int NQ = D * PR / NTHR, RSTEP = NTHR / PR;
    f32x4 x[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) x[q] = *reinterpret_cast<const f32x4*>(src + q * RSTEP * D);
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      bf16x4 hi, lo;
      split4(x[q], hi, lo);
      lds_st<bf16x4>(m + (dst + q * RSTEP * ROWB), hi);
      lds_st<bf16x4>(m + (dst + q * RSTEP * ROWB + PLANE), lo);
    }
  }
  // the wave's rows 16 w .. 16 w + 15 (D-layout tiles t of M^T) -> planes at m.
  // In the stored block order a lane's columns of tiles 2k and 2k+1 are
  // adjacent (blocks G and 4+G of a 32-column group sit at 8G and 8G+4), so
  // each pair leaves as one 16-byte store per plane.
  GMDN_DEV void publish(lds_ptr m, const f32x4 (&t)[NT]) const {
#pragma unroll
    for (int c = 0; c < NT; c += 2) {
      bf16x4 h0, l0, h1, l1;
      split4(t[c], h0, l0);
      split4(t[c + 1], h1, l1);
      const bf16x8 hi = cat8(h0, h1), lo = cat8(l0, l1);
      lds_st<bf16x8>(m + ppub[c], hi);
      lds_st<bf16x8>(m + (ppub[c] + PLANE), lo);
    }
  }
  // lane (r, G) takes M[16 tr + r][32 kb + pair(G, s)]
  GMDN_DEV Op row(lds_cptr m, int tr, int kb) const {
    const lds_cptr a = m + prow[kb] + tr * 16 * ROWB;
    Op o;
    o.hi = lds_ld<bf16x8>(a);
    o.lo = lds_ld<bf16x8>(a + PLANE);
    return o;
  }
  // lane (c, G) takes M[32 kb + pair(G, s)][16 tc + c]
  GMDN_DEV Op col(lds_cptr m, int kb, int tc) const {
    const lds_cptr a = m + pcol[tc] + kb * 32 * ROWB, b = a + 16 * ROWB;
    Op o;
    o.hi = cat8(lds_tr16(a), lds_tr16(b));
    o.lo = cat8(lds_tr16(a + PLANE), lds_tr16(b + PLANE));
    return o;
  }
  GMDN_DEV f32x4 rowprod(lds_cptr pub, int tr, const Op (&B)[NKB]) const {
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc = P::mma(row(pub, tr, kb), B[kb], acc);
    return acc;
  }
  GMDN_DEV f32x4 colprod(lds_cptr pub, int tc, const Op (&B)[NKB], f32x4 acc) const {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc = P::mma(col(pub, kb, tc), B[kb], acc);
    return acc;
  }
  // All NT tiles of a product at once, k-block outer: consecutive MFMAs go
  // to independent accumulators.  The operands are software-pipelined PIPE
  // ahead of their MFMAs (a scheduling barrier per step keeps the order): left
  // to itself, at the register pressure of the scan kernels, the compiler
  // waits for each operand read right before its MFMAs, exposing the LDS
  // latency on every read.
  static constexpr int PIPE = 2;
  // acc[tr] += tile [r'][r] = sum_k pub[r'][k] B[k][r]
  GMDN_DEV void rowprod_all(lds_cptr pub, const Op (&B)[NKB], f32x4 (&acc)[NT]) const {
    constexpr int NJ = NKB * NT;
    Op a[PIPE];
#pragma unroll
    for (int j = 0; j < PIPE; ++j) a[j] = row(pub, j % NT, j / NT);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const Op cur = a[j % PIPE];
      if (j + PIPE < NJ) a[j % PIPE] = row(pub, (j + PIPE) % NT, (j + PIPE) / NT);
      __builtin_amdgcn_sched_barrier(0);
      acc[j % NT] = P::mma(cur, B[j / NT], acc[j % NT]);
    }
  }
  // rowprod_all with the B operand the wave's own rows of the planes at bm
  // (row tile w), each k-block's read one k-block ahead
  GMDN_DEV void rowprod_own(lds_cptr pub, lds_cptr bm, f32x4 (&acc)[NT]) const {
    const int w = wave_id();
    constexpr int NJ = NKB * NT;
    Op a[PIPE], b[2];
    b[0] = row(bm, w, 0);
#pragma unroll
    for (int j = 0; j < PIPE; ++j) a[j] = row(pub, j % NT, j / NT);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const Op cur = a[j % PIPE];
      if (j + PIPE < NJ) a[j % PIPE] = row(pub, (j + PIPE) % NT, (j + PIPE) / NT);
      if (j % NT == 0 && j / NT + 1 < NKB) b[(j / NT + 1) & 1] = row(bm, w, j / NT + 1);
      __builtin_amdgcn_sched_barrier(0);
      acc[j % NT] = P::mma(cur, b[(j / NT) & 1], acc[j % NT]);
    }
  }
  // acc[tc] += tile [c][r] = sum_k pub[k][c] B[k][r]
  GMDN_DEV void colprod_all(lds_cptr pub, const Op (&B)[NKB], f32x4 (&acc)[NT]) const {
    constexpr int NJ = NKB * NT;
    Op a[PIPE];
#pragma unroll
    for (int j = 0; j < PIPE; ++j) a[j] = col(pub, j / NT, j % NT);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const Op cur = a[j % PIPE];
      if (j + PIPE < NJ) a[j % PIPE] = col(pub, (j + PIPE) / NT, (j + PIPE) % NT);
      __builtin_amdgcn_sched_barrier(0);
      acc[j % NT] = P::mma(cur, B[j / NT], acc[j % NT]);
    }
  }
  // stage_own in two halves, so that the loads can be issued early
  static GMDN_DEV void load_pieces(const float* g, bf16x8 (&pc)[NT]) {
    const int l = lane_id(), row = 16 * wave_id() + (l & 15);
#pragma unroll
    for (int c = 0; c < NT; ++c) pc[c] = *reinterpret_cast<const bf16x8*>(g + row * D + 16 * c + 4 * (l >> 4));
  }
  GMDN_DEV void store_pieces(lds_ptr m, const bf16x8 (&pc)[NT]) const {
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      lds_st<bf16x4>(m + ppub[c], __builtin_shufflevector(pc[c], pc[c], 0, 1, 2, 3));
      lds_st<bf16x4>(m + (ppub[c] + PLANE), __builtin_shufflevector(pc[c], pc[c], 4, 5, 6, 7));
    }
  }
  // The wave's rows of a matrix kept in global memory as split pieces (the
  // layout `store_own` writes) -> planes at m
  GMDN_DEV void stage_own(lds_ptr m, const float* g) const {
    const int l = lane_id(), row = 16 * wave_id() + (l & 15);
    bf16x8 pc[NT];
#pragma unroll
    for (int c = 0; c < NT; ++c) pc[c] = *reinterpret_cast<const bf16x8*>(g + row * D + 16 * c + 4 * (l >> 4));
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      lds_st<bf16x4>(m + ppub[c], __builtin_shufflevector(pc[c], pc[c], 0, 1, 2, 3));
      lds_st<bf16x4>(m + (ppub[c] + PLANE), __builtin_shufflevector(pc[c], pc[c], 4, 5, 6, 7));
    }
  }
  // the wave's rows (D-layout tiles t of M^T) -> split pieces in global memory
  static GMDN_DEV void store_own(float* g, const f32x4 (&t)[NT]) {
    const int l = lane_id(), row = 16 * wave_id() + (l & 15);
#pragma unroll
    for (int c = 0; c < NT; ++c) *reinterpret_cast<bf16x8*>(g + row * D + 16 * c + 4 * (l >> 4)) = split_piece(t[c]);
  }
  // operands of the wave's rows from pieces already loaded by load_pieces
  // (register moves only: placed right before their product, they do not
  // make the loads wait early)
  static GMDN_DEV void own_ops(const bf16x8 (&pc)[NT], Op (&o)[NKB]) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      o[kb].hi = __builtin_shufflevector(pc[2 * kb], pc[2 * kb + 1], 0, 1, 2, 3, 8, 9, 10, 11);
      o[kb].lo = __builtin_shufflevector(pc[2 * kb], pc[2 * kb + 1], 4, 5, 6, 7, 12, 13, 14, 15);
    }
  }
  // operands of the wave's rows from those pieces (the split of pack_all)
  static GMDN_DEV void load_own(const float* g, Op (&o)[NKB]) {
    const int l = lane_id(), row = 16 * wave_id() + (l & 15);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(g + row * D + 32 * kb + 4 * (l >> 4));
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(g + row * D + 32 * kb + 16 + 4 * (l >> 4));
      o[kb].hi = __builtin_shufflevector(a, b, 0, 1, 2, 3, 8, 9, 10, 11);
      o[kb].lo = __builtin_shufflevector(a, b, 4, 5, 6, 7, 12, 13, 14, 15);
    }
  }
  // D-layout tile [r'][r] (r' = 16 tr + .., r = the wave's rows) of the
  // transpose of the matrix at m: transposing reads at the wave's columns
  // (tb = the lane's base for them, `tbase`)
  GMDN_DEV static uint32_t tbase() {
    const int l = lane_id(), lc = l & 15;
    return off(4 * (l >> 4) + (lc >> 2), 16 * wave_id() + 4 * (lc & 3));
  }
  static GMDN_DEV f32x4 tview(lds_cptr m, uint32_t tb, int tr) {
    const lds_cptr a = m + tb + tr * 16 * ROWB;
    const bf16x4 h = lds_tr16(a), o = lds_tr16(a + PLANE);
    return f32x4{(float)h[0] + (float)o[0], (float)h[1] + (float)o[1], (float)h[2] + (float)o[2],
                 (float)h[3] + (float)o[3]};
  }
  // One quintic step on the wave's rows XT (D-layout tiles of X^T); the same
  // products as NSBlock::step.  With zst / pst, Z = b P + c P^2 and P = X X^T
  // (both symmetric) are also stored as the wave's rows in split pieces.
  GMDN_DEV void step(f32x4 (&XT)[NT], lds_ptr XM, lds_ptr PM, float* zst = nullptr, float* pst = nullptr) const {
    publish(XM, XT);
    __syncthreads();
    Op Bx[NKB];
    pack_all(XT, Bx);
    f32x4 Pc[NT];
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) Pc[tr] = zero4();
    rowprod_all(XM, Bx, Pc);
    // P is symmetric: the column block is also the wave's rows of P
    publish(PM, Pc);
    if (pst) store_own(pst, Pc);
    __syncthreads();
    Op Bp[NKB];
    pack_all(Pc, Bp);
    // Z = b P + c P^2, in place of the wave's block of P (now held by Bp)
    // as c ((b / c) P + P^2), accumulating P^2 onto the scaled block
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) Pc[tr] = (NS_B / NS_C) * Pc[tr];
    rowprod_all(PM, Bp, Pc);
#pragma unroll
    for (int tr = 0; tr < NT; ++tr) Pc[tr] = NS_C * Pc[tr];
    if (zst) store_own(zst, Pc);
    Op Bz[NKB];
    pack_all(Pc, Bz);
#pragma unroll
    for (int tc = 0; tc < NT; ++tc) XT[tc] = NS_A * XT[tc];
    colprod_all(XM, Bz, XT);
    __syncthreads();
  }
};

}  // namespace gmdn
