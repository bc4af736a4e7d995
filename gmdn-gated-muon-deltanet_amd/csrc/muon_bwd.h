// The bf16x3 muon reverse scan's stages as device functions over one
// workgroup each (reference fast_scan.py:107-131 and :158-166), shared by the
// drop-in scan's backward (scan_muon.hip) and the fused mixer core's muon
// backward (chunk_bwd.hip), which launch them side by side with their other
// stages.
#pragma once
#include "ns.h"
#include "scan_a.h"

#include <type_traits>

namespace gmdn {

// The backward with bf16x3 products, in two stages on the NSSplit engine
// (two LDS slots of one split matrix each, A and B).
//
// muon_pre_body, one workgroup per (b, h, chunk): the forward iterates do
// not depend on the cotangent, so they are rebuilt for every chunk at once
// across the chip.  K_i staged into B; G = U - S_i K_i; M_i = m M_{i-1} + G;
// X_0 = M_i / (|M_i| + eps); then the ns steps, storing each iterate X_k
// (k = 0 .. ns), each P_k = X_k X_k^T and Z_k = b P_k + c P_k^2 as the
// wave's rows in split pieces, M_i in fp32 and |M_i|.  Workspace per chunk:
// 3 ns + 2 matrices.
//
// muon_x3_body, one workgroup per (b, h), chunks in reverse order:
//   1. da_i = <Sb, S_i>, db_i = <Sb, X_ns> (S_i, X_ns and gS requested at
//      the end of the previous chunk); Xbar = b Sb; a Sb + gS parked in Sb's
//      workspace rows until the tail.
//   2. The VJP steps, k = ns-1 .. 0, with Xbar published in A and X_k in B:
//        Bbar = Xbar X_k^T                        (A and B row reads)
//        Q    = a Xbar + Z_k Xbar                 (A column reads, Z_k rows)
//        Bs   = Bbar + Bbar^T: Bbar published in A, read back transposed
//        Y    = Bs P_k                            (Bs published in A, P_k rows)
//        Y^T  read back transposed after publishing Y in A
//        Xbar <- Q + (b Bs + c (Y + Y^T)) X_k     (B column reads)
//      (P_k, Bs and Z_k are symmetric.)  Four D^3 products per step: the
//      transposes are LDS reads of the published copies, and P_k comes from
//      the iterate stage instead of X_k (X_k^T Bs).
//   3. The normalisation VJP, Gb = dU_i, and Sb <- (a Sb + gS) - Gb K_i^T
//      with K_i staged into B (row reads).  Each phase issues its global
//      loads together ahead of their first use.
// Mbar passes from chunk to chunk through the workspace as fp32 rows of their
// wave.
//
// Segments: the chunks are processed nseg at a time from the end, so the
// per-chunk workspace holds nseg chunks per (b, h) (per buffer) whatever N
// is; Sb and Mbar carry from one segment to the next through the workspace.
// With two iterate buffers a segment's iterates are formed in the launch
// that runs the previous segment's reverse pass.
template <int D>
struct MuonBwdWs {
  // nbuf iterate buffers, each with per (b, h) and chunk of a segment (local
  // index c = i - i0): X_0 .. X_ns, Z_0 .. Z_{ns-1}, P_0 .. P_{ns-1}, M_i;
  // then Mbar and Sb per (b, h); then |M_i| per buffer, (b, h) and chunk
  int64_t mat, per_chunk, BH, nseg, iters;
  GMDN_DEV MuonBwdWs(int64_t BH_, int64_t nseg_, int ns, int nbuf)
      : mat((int64_t)D * D), per_chunk((3 * ns + 2) * mat), BH(BH_), nseg(nseg_),
        iters(nbuf * BH_ * nseg_ * per_chunk) {}
  GMDN_DEV int64_t slot(int64_t bh, int c, int buf) const { return (buf * BH + bh) * nseg + c; }
  GMDN_DEV float* X(float* ws, int64_t sl, int k) const { return ws + sl * per_chunk + k * mat; }
  GMDN_DEV float* Z(float* ws, int64_t sl, int ns, int k) const { return ws + sl * per_chunk + (ns + 1 + k) * mat; }
  GMDN_DEV float* P(float* ws, int64_t sl, int ns, int k) const { return ws + sl * per_chunk + (2 * ns + 1 + k) * mat; }
  GMDN_DEV float* M(float* ws, int64_t sl, int ns) const { return ws + sl * per_chunk + (3 * ns + 1) * mat; }
  GMDN_DEV float* Mbar(float* ws, int64_t bh) const { return ws + iters + bh * mat; }
  GMDN_DEV float* Sbar(float* ws, int64_t bh) const { return ws + iters + (BH + bh) * mat; }
  GMDN_DEV float* norm(float* ws) const { return ws + iters + 2 * BH * mat; }
};

// One launch of the segmented backward: the reverse pass over segment
// [i0, i1) (blocks 0 .. nx3 - 1, nx3 = BH or 0) reading iterate buffer xbuf,
// and the iterates of segment [j0, j0 + jcur) (the next blocks, BH jcur of
// them, or none) written into buffer pbuf.  The two parts share nothing but
// the launch, so the chunk-parallel iterates of the next segment fill the CUs
// that the BH serial reverse scans leave idle.
struct MuonSegArgs {
  const float *U, *K, *av, *bv, *mv, *S_all, *M_all, *gS;
  float *dU, *da, *db, *dm, *dn, *ws;
  int64_t BH;
  int N, ns, nseg, nbuf;
  int nx3, i0, i1, xbuf;
  int j0, jcur, pbuf;
};

// The iterates of chunk j0 + blk % jcur of head blk / jcur.
template <int D>
GMDN_DEV void muon_pre_body(const MuonSegArgs& sa, int64_t blk) {
  const float* __restrict__ U = sa.U;
  const float* __restrict__ K = sa.K;
  const float* __restrict__ mv = sa.mv;
  const float* __restrict__ S_all = sa.S_all;
  const float* __restrict__ M_all = sa.M_all;
  float* __restrict__ ws = sa.ws;
  const int64_t BH = sa.BH;
  const int N = sa.N, ns = sa.ns, i0 = sa.j0, ncur = sa.jcur;
  using NSX = NSSplit<D>;
  using P = PrecX3;
  using Op = P::Op;
  constexpr int NT = D / 16, NKB = D / 32, NW = D / 16;
  extern __shared__ __align__(16) float msmem[];
  const lds_ptr SA = lds_base(msmem), SB = SA + NSX::BYTES;
  float* red = msmem + 2 * NSX::BYTES / 4;
  const NSX nsx;
  const MuonBwdWs<D> W(BH, sa.nseg, ns, sa.nbuf);
  const int64_t bh = blk / ncur;
  const int c = (int)(blk % ncur);  // chunk i0 + c of the segment
  const int64_t si = bh * N + i0 + c, sl = W.slot(bh, c, sa.pbuf);
  const int l = lane_id(), G = l >> 4, rl = l & 15;
  const int r0 = 16 * wave_id();
  const int64_t mat = (int64_t)D * D;
  auto roff = [&](int t) { return (int64_t)(r0 + rl) * D + 16 * t + 4 * G; };

  NSX::template stage<D * 4>(SB, K + si * mat);
  Op Bop[NKB];
  {
    f32x4 Si[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) Si[t] = *reinterpret_cast<const f32x4*>(S_all + si * mat + roff(t));
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Bop[kb] = P::pack(-Si[2 * kb], -Si[2 * kb + 1]);
  }
  __syncthreads();  // K_i staged
  const float gm = mv[si];
  float* WM = W.M(ws, sl, ns);
  f32x4 X[NT];
  float sq = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    f32x4 g = *reinterpret_cast<const f32x4*>(U + si * mat + roff(t));
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) g = P::mma(nsx.col(SB, kb, t), Bop[kb], g);
    const f32x4 Mp = *reinterpret_cast<const f32x4*>(M_all + si * mat + roff(t));
    X[t] = gm * Mp + g;
    *reinterpret_cast<f32x4*>(WM + roff(t)) = X[t];
    sq += X[t][0] * X[t][0] + X[t][1] * X[t][1] + X[t][2] * X[t][2] + X[t][3] * X[t][3];
  }
  const float nf = sqrtf(block_sum<NW>(sq, red));  // (its barriers also retire B's K_i reads)
  if (threadIdx.x == 0) W.norm(ws)[sl] = nf;
  const float scale = 1.f / (nf + 1e-7f);
#pragma unroll
  for (int t = 0; t < NT; ++t) X[t] = X[t] * scale;
  for (int k = 0; k < ns; ++k) {
    NSX::store_own(W.X(ws, sl, k), X);
    nsx.step(X, SA, SB, W.Z(ws, sl, ns, k), W.P(ws, sl, ns, k));
  }
  NSX::store_own(W.X(ws, sl, ns), X);
}

// The reverse pass of head bh over chunks i1 - 1 .. i0.
template <int D>
GMDN_DEV void muon_x3_body(const MuonSegArgs& sa, int64_t bh) {
  const float* __restrict__ K = sa.K;
  const float* __restrict__ av = sa.av;
  const float* __restrict__ bv = sa.bv;
  const float* __restrict__ mv = sa.mv;
  const float* __restrict__ S_all = sa.S_all;
  const float* __restrict__ M_all = sa.M_all;
  const float* __restrict__ gS = sa.gS;
  float* __restrict__ dU = sa.dU;
  float* __restrict__ da = sa.da;
  float* __restrict__ db = sa.db;
  float* __restrict__ dm = sa.dm;
  float* __restrict__ dn = sa.dn;
  float* __restrict__ ws = sa.ws;
  const int64_t BH = sa.BH;
  const int N = sa.N, ns = sa.ns, i0 = sa.i0, i1 = sa.i1, xbuf = sa.xbuf;
  using NSX = NSSplit<D>;
  using P = PrecX3;
  using Op = P::Op;
  constexpr int NT = D / 16, NKB = D / 32, NW = D / 16;
  extern __shared__ __align__(16) float msmem[];
  const lds_ptr SA = lds_base(msmem), SB = SA + NSX::BYTES;
  float* red = msmem + 2 * NSX::BYTES / 4;

  const NSX nsx;
  const uint32_t tb = NSX::tbase();
  const MuonBwdWs<D> W(BH, sa.nseg, ns, sa.nbuf);
  const int l = lane_id(), G = l >> 4, rl = l & 15;
  const int r0 = 16 * wave_id();
  const int64_t mat = (int64_t)D * D;
  float* WMb = W.Mbar(ws, bh);  // Mbar carried to chunk i-1
  // 32-bit lane offsets, opaque at every use: the loads and stores then take
  // a scalar base and one offset register; left visible, the compiler hoists
  // a 64-bit address pair per array out of the chunk loop and spills them
  const uint32_t lane_row = (uint32_t)((r0 + rl) * D + 4 * G);
  auto roff = [&](int t) {
    uint32_t o = lane_row;
    asm volatile("" : "+v"(o));
    return o + (uint32_t)(16 * t);
  };

  // Sb from the segment after this one (zero after the last chunk)
  float* WSb = W.Sbar(ws, bh);
  f32x4 Sb[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) Sb[t] = i1 == N ? zero4() : *reinterpret_cast<const f32x4*>(WSb + roff(t));

  // Chunk i's first-phase inputs S_i, X_ns's pieces and gS, requested
  // together and one chunk ahead (at the end of the previous chunk's tail),
  // so that their latency is not exposed at the chunk's start.
  f32x4 Si[NT], Gs[NT];
  bf16x8 Xn[NT];
  auto request_start = [&](int i) {
    const int64_t si = bh * N + i;
    const float* Xs = W.X(ws, W.slot(bh, i - i0, xbuf), ns);
#pragma unroll
    for (int t = 0; t < NT; ++t) Si[t] = *reinterpret_cast<const f32x4*>(S_all + si * mat + roff(t));
#pragma unroll
    for (int t = 0; t < NT; ++t) Xn[t] = *reinterpret_cast<const bf16x8*>(Xs + roff(t));
#pragma unroll
    for (int t = 0; t < NT; ++t) Gs[t] = *reinterpret_cast<const f32x4*>(gS + si * mat + roff(t));
  };
  request_start(i1 - 1);

  for (int i = i1 - 1; i >= i0; --i) {
    const int64_t si = bh * N + i, sl = W.slot(bh, i - i0, xbuf);
    const float ga = av[si], gb = bv[si], gm = mv[si];
    // ---- 1. da_i = <Sb, S_i>, db_i = <Sb, msign(M_i)>
    float pda = 0.f, pdb = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const f32x4 Xs = unsplit_piece(Xn[t]);
      pda += Sb[t][0] * Si[t][0] + Sb[t][1] * Si[t][1] + Sb[t][2] * Si[t][2] + Sb[t][3] * Si[t][3];
      pdb += Sb[t][0] * Xs[0] + Sb[t][1] * Xs[1] + Sb[t][2] * Xs[2] + Sb[t][3] * Xs[3];
    }
    const f32x2 dsum = block_sum2<NW>(pdb, pda, red);
    const float dbv = dsum[0], dav = dsum[1];
    // ---- 2. Xbar = b Sb pulled back through the ns steps (X is its register home)
    f32x4 X[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) X[t] = gb * Sb[t];
    // The tail's a Sb + gS waits in Sb's workspace rows through the VJP
    // steps (their registers are the scarce resource there).
    auto park_sb = [&] {
#pragma unroll
      for (int t = 0; t < NT; ++t) *reinterpret_cast<f32x4*>(WSb + roff(t)) = ga * Sb[t] + Gs[t];
    };
    if (ns > 0) {
      nsx.publish(SA, X);
      bf16x8 xs[NT];
      NSX::load_pieces(W.X(ws, sl, ns - 1), xs);
      park_sb();
      nsx.store_pieces(SB, xs);
      __syncthreads();
    } else {
      park_sb();
    }
    // the tail's M_i and Mbar rows, requested during the last VJP step
    const float* WM = W.M(ws, sl, ns);
    f32x4 Mi[NT], Mb[NT];
    auto request_tail = [&] {
#pragma unroll
      for (int t = 0; t < NT; ++t) Mi[t] = *reinterpret_cast<const f32x4*>(WM + roff(t));
#pragma unroll
      for (int t = 0; t < NT; ++t) Mb[t] = i == N - 1 ? zero4() : *reinterpret_cast<const f32x4*>(WMb + roff(t));
    };
    // One VJP step; the last one (k = 0) requests the tail's rows where the
    // others request the next step's.  (Peeled, so that no register array is
    // defined on one path of a step only: such an array stays live through
    // every step.)
    auto vjp_step = [&](int k, auto last_tag) {
      constexpr bool LAST = decltype(last_tag)::value;
      f32x4 Q[NT], Bs[NT];
      // Z_k's and P_k's own rows as pieces, P_k in flight through the first
      // two products (Z_k requested a step ahead, in flight through the last
      // product, measured slower: that product's operand reads wait behind it)
      bf16x8 zr[NT], pr[NT];
      NSX::load_pieces(W.Z(ws, sl, ns, k), zr);
      NSX::load_pieces(W.P(ws, sl, ns, k), pr);
      {
        // Bbar[r'][r] = sum_k Xbar[r'][k] X_k[r][k]: the wave's own rows of
        // X_k (B) as the B operand; LDS operands only, so Z_k's rows are in
        // flight through it
#pragma unroll
        for (int tr = 0; tr < NT; ++tr) Bs[tr] = zero4();
        nsx.rowprod_own(SA, SB, Bs);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the phases' operands apart
#pragma unroll
      for (int tc = 0; tc < NT; ++tc) Q[tc] = NS_A * X[tc];
      {
        Op Bz[NKB];
        NSX::own_ops(zr, Bz);
        nsx.colprod_all(SA, Bz, Q);
      }
      __syncthreads();  // every read of Xbar in A done
      nsx.publish(SA, Bs);
      __syncthreads();
      // Bs = Bbar + Bbar^T, the transpose read back from the published copy
#pragma unroll
      for (int tr = 0; tr < NT; ++tr) Bs[tr] += NSX::tview(SA, tb, tr);
      __syncthreads();  // every transposed read of A done
      nsx.publish(SA, Bs);  // Bs is symmetric
      __syncthreads();
      f32x4 Y[NT];
      {
        // Y[r'][r] = (Bs P_k)[r'][r]: P_k's own rows (= columns) as the B operand
#pragma unroll
        for (int tr = 0; tr < NT; ++tr) Y[tr] = zero4();
        Op Bp[NKB];
        __builtin_amdgcn_sched_barrier(0);
        NSX::own_ops(pr, Bp);
        nsx.rowprod_all(SA, Bp, Y);
      }
      // the next step's X_{k-1} pieces for B (after the last step: the tail's
      // rows), in flight through the Y exchange and the last product
      bf16x8 xn[NT];
      if constexpr (!LAST) {
        NSX::load_pieces(W.X(ws, sl, k - 1), xn);
      } else {
        request_tail();
      }
      __syncthreads();  // every read of Bs in A done
      nsx.publish(SA, Y);  // A holds Y^T
      __syncthreads();
      {
        Op So[NKB];
#pragma unroll
        for (int tr = 0; tr < NT; ++tr) Bs[tr] = NS_B * Bs[tr] + NS_C * (Y[tr] + NSX::tview(SA, tb, tr));
        NSX::pack_all(Bs, So);
        nsx.colprod_all(SB, So, Q);
#pragma unroll
        for (int tc = 0; tc < NT; ++tc) X[tc] = Q[tc];
      }
      __syncthreads();  // every read of A and B done
      if constexpr (!LAST) {
        nsx.publish(SA, X);
        nsx.store_pieces(SB, xn);
        __syncthreads();
      }
    };
    for (int k = ns - 1; k >= 1; --k) vjp_step(k, std::false_type{});
    if (ns > 0)
      vjp_step(0, std::true_type{});
    else
      request_tail();
    // ---- 3. normalisation: Mbar = Xbar/nrm - <Xbar, M_i>/nrm^2 * M_i/max(|M_i|, 1e-12)
    const float nf = W.norm(ws)[sl];
    const float nrm = nf + 1e-7f;
#pragma unroll
    for (int t = 0; t < NT; ++t) Sb[t] = *reinterpret_cast<const f32x4*>(WSb + roff(t));  // a Sb + gS
    NSX::template stage<D * 4>(SB, K + si * mat);  // K_i, for the row reads of the Sb update
    float pdot = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) pdot += X[t][0] * Mi[t][0] + X[t][1] * Mi[t][1] + X[t][2] * Mi[t][2] + X[t][3] * Mi[t][3];
    const float dot = block_sum<NW>(pdot, red);     // (its barriers also publish K_i in B)
    const float cM = dot / (nrm * nrm) / fmaxf(nf, 1e-12f);
    // M_{i-1} for dm, in flight through the Sb update
    f32x4 Mp[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) Mp[t] = *reinterpret_cast<const f32x4*>(M_all + si * mat + roff(t));
    f32x4 Mt[NT];  // dU_i = Gb_i, the total cotangent of M_i
    const float rn = 1.f / nrm;
#pragma unroll
    for (int t = 0; t < NT; ++t) Mt[t] = Mb[t] + X[t] * rn - cM * Mi[t];
    Op Bg[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Bg[kb] = P::pack(-Mt[2 * kb], -Mt[2 * kb + 1]);
    // Sb <- a Sb + gS - Gb K^T : A = K rows
    nsx.rowprod_all(SB, Bg, Sb);
    __builtin_amdgcn_sched_barrier(0);  // dm's wait for M_{i-1} after the product, not inside it
    float pdm = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) pdm += Mt[t][0] * Mp[t][0] + Mt[t][1] * Mp[t][1] + Mt[t][2] * Mp[t][2] + Mt[t][3] * Mp[t][3];
    // (chunk i0 requests itself again: a def on one path only would keep the
    // arrays live through the VJP steps)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      *reinterpret_cast<f32x4*>(WMb + roff(t)) = gm * Mt[t];
      *reinterpret_cast<f32x4*>(dU + si * mat + roff(t)) = Mt[t];
    }
    request_start(i > i0 ? i - 1 : i0);
    const float dmv = block_sum<NW>(pdm, red);
    if (threadIdx.x == 0) {
      da[si] = dav;
      db[si] = dbv;
      dm[si] = dmv;
      dn[si] = 0.f;
    }
    __syncthreads();  // B's K_i read by every wave before chunk i-1 publishes into A and B
  }
  if (i0 > 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t) *reinterpret_cast<f32x4*>(WSb + roff(t)) = Sb[t];
  }
}

}  // namespace gmdn
