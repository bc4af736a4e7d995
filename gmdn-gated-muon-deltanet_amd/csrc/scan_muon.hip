// Level A, muon rule (reference fast_scan.py:86-88 forward, :158-166 and
// :107-131 backward).  msign couples every entry of the state, so one
// workgroup of D/16 waves owns one (b, h): wave w keeps rows 16w.. of S and
// M (D-layout tiles of the transposes) and the waves cooperate on the
// Newton-Schulz iterations through shared matrices.
//
// Forward: X and P live in LDS (2 D^2 fp32 worth): as split bf16 planes for
// the bf16x3 precision, as swizzled fp32 for the exact one; K_i is read
// straight from global memory (it is used once per chunk).
// Backward with fp32 products (precision 'ieee'): X_k, P, Xbar and Bbar
// (4 D^2) exceed LDS at D = 128, so they live in a per-(b, h) global workspace
// (L2 resident), followed by the ns stored iterates X_0 .. X_{ns-1} (written
// and re-read by the same lanes).  The bf16x3 backward is described at its
// kernels.
#include "ns.h"
#include "scan_a.h"

#include <type_traits>

namespace gmdn {

template <int D, int PREC>
__global__ void __launch_bounds__(D * 4)
scan_fwd_muon(const float* __restrict__ U, const float* __restrict__ K,
              const float* __restrict__ av, const float* __restrict__ bv,
              const float* __restrict__ mv, float* __restrict__ S_all,
              float* __restrict__ M_all, int N, int ns) {
  using P = typename PrecSel<PREC>::T;
  constexpr int NT = D / 16, NKB = D / 32, NW = D / 16;
  using NS = NSBlock<P, SwzMat<D>, D>;
  extern __shared__ __align__(16) float smem[];
  float* XM = smem;
  float* PM = smem + D * D;
  __shared__ float red[NW];

  const int64_t bh = blockIdx.x;
  const int l = lane_id(), G = l >> 4, rl = l & 15;
  const int r0 = 16 * wave_id();
  const int64_t mat = (int64_t)D * D;
  auto roff = [&](int t) { return (int64_t)(r0 + rl) * D + 16 * t + 4 * G; };

  f32x4 S[NT], M[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) S[t] = M[t] = zero4();
  const NSSplit<D> nsx;  // per-lane LDS bases of the bf16x3 engine

  for (int i = 0; i < N; ++i) {
    const int64_t si = bh * N + i;
    const float* Ki = K + si * mat;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      *reinterpret_cast<f32x4*>((S_all + si * mat + roff(t))) = S[t];
      if (M_all) *reinterpret_cast<f32x4*>((M_all + si * mat + roff(t))) = M[t];
    }
    typename P::Op Bop[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Bop[kb] = P::pack(-S[2 * kb], -S[2 * kb + 1]);
    const float a = av[si], b = bv[si], m = mv[si];
    if constexpr (PREC == 0) {
      // K_i as split planes in the P store (free until the first NS step
      // publishes P), read back as column operands
      NSSplit<D>::template stage<D * 4>(lds_base(smem) + NSSplit<D>::BYTES, Ki);
      __syncthreads();
    }
    float sq = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 g = *reinterpret_cast<const f32x4*>((U + si * mat + roff(t)));
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        if constexpr (PREC == 0)
          g = P::mma(nsx.col(lds_base(smem) + NSSplit<D>::BYTES, kb, t), Bop[kb], g);
        else
          g = P::mma(col_op<P, PlainMat<D>>(Ki, 32 * kb, 16 * t), Bop[kb], g);
      }
      M[t] = m * M[t] + g;
      sq += M[t][0] * M[t][0] + M[t][1] * M[t][1] + M[t][2] * M[t][2] + M[t][3] * M[t][3];
    }
    const float scale = 1.f / (sqrtf(block_sum<NW>(sq, red)) + 1e-7f);
    f32x4 X[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) X[t] = M[t] * scale;
    if constexpr (PREC == 0) {
      const lds_ptr base = lds_base(smem);
      for (int s = 0; s < ns; ++s) nsx.step(X, base, base + NSSplit<D>::BYTES);
    } else {
      for (int s = 0; s < ns; ++s) NS::step(X, XM, PM);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) S[t] = a * S[t] + b * X[t];
  }
}

template <int D, int PREC>
__global__ void __launch_bounds__(D * 4)
scan_bwd_muon(const float* __restrict__ U, const float* __restrict__ K,
              const float* __restrict__ av, const float* __restrict__ bv,
              const float* __restrict__ mv, const float* __restrict__ S_all,
              const float* __restrict__ M_all, const float* __restrict__ gS,
              float* __restrict__ dU, float* __restrict__ da, float* __restrict__ db,
              float* __restrict__ dm, float* __restrict__ dn, float* __restrict__ ws, int N,
              int ns) {
  using P = typename PrecSel<PREC>::T;
  constexpr int NT = D / 16, NKB = D / 32, NW = D / 16;
  using NS = NSBlock<P, PlainMat<D>, D>;
  __shared__ float red[NW];

  const int64_t bh = blockIdx.x;
  const int l = lane_id(), G = l >> 4, rl = l & 15;
  const int r0 = 16 * wave_id();
  const int64_t mat = (int64_t)D * D;
  float* wsb = ws + bh * (4 + ns) * mat;
  float *XM = wsb, *PM = wsb + mat, *XbM = wsb + 2 * mat, *BM = wsb + 3 * mat, *IT = wsb + 4 * mat;
  auto roff = [&](int t) { return (int64_t)(r0 + rl) * D + 16 * t + 4 * G; };

  f32x4 Sb[NT], Mb[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) Sb[t] = Mb[t] = zero4();

  for (int i = N - 1; i >= 0; --i) {
    const int64_t si = bh * N + i;
    const float* Ki = K + si * mat;
    const float a = av[si], b = bv[si], m = mv[si];
    f32x4 Si[NT], Mp[NT], Mi[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      Si[t] = *reinterpret_cast<const f32x4*>((S_all + si * mat + roff(t)));
      Mp[t] = *reinterpret_cast<const f32x4*>((M_all + si * mat + roff(t)));
    }
    {
      typename P::Op Bop[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Bop[kb] = P::pack(-Si[2 * kb], -Si[2 * kb + 1]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 g = *reinterpret_cast<const f32x4*>((U + si * mat + roff(t)));
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) g = P::mma(col_op<P, PlainMat<D>>(Ki, 32 * kb, 16 * t), Bop[kb], g);
        Mi[t] = m * Mp[t] + g;
      }
    }
    float sq = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t) sq += Mi[t][0] * Mi[t][0] + Mi[t][1] * Mi[t][1] + Mi[t][2] * Mi[t][2] + Mi[t][3] * Mi[t][3];
    const float nf = sqrtf(block_sum<NW>(sq, red));
    const float nrm = nf + 1e-7f;
    f32x4 X[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) X[t] = Mi[t] / nrm;
    for (int s = 0; s < ns; ++s) {
#pragma unroll
      for (int t = 0; t < NT; ++t) mat_store_tileT<PlainMat<D>>(IT + s * mat, r0, 16 * t, X[t]);
      NS::step(X, XM, PM);
    }
    // db_i = <Sb, msign(M_i)>, da_i = <Sb, S_i>
    float pdb = 0.f, pda = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pdb += Sb[t][j] * X[t][j];
        pda += Sb[t][j] * Si[t][j];
      }
    const float dbv = block_sum<NW>(pdb, red);
    const float dav = block_sum<NW>(pda, red);
    // Xbar = b * Sb, pulled back through the ns steps
    f32x4 Xb[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) Xb[t] = b * Sb[t];
    for (int s = ns - 1; s >= 0; --s) {
      f32x4 Xk[NT];
      const int l2 = lane_id();
#pragma unroll
      for (int t = 0; t < NT; ++t)
        Xk[t] = *reinterpret_cast<const f32x4*>(IT + s * mat + PlainMat<D>::off(r0 + (l2 & 15), 16 * t + 4 * (l2 >> 4)));
      NS::vjp_step(Xk, Xb, XM, PM, XbM, BM);
    }
    // normalisation: Mbar = Xbar/nrm - <Xbar, Mi>/nrm^2 * Mi/max(|Mi|, 1e-12)
    float pdot = 0.f;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) pdot += Xb[t][j] * Mi[t][j];
    const float dot = block_sum<NW>(pdot, red);
    const float cM = dot / (nrm * nrm) / fmaxf(nf, 1e-12f);
    float pdm = 0.f;
    f32x4 Gb[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const f32x4 Mtot = Mb[t] + Xb[t] / nrm - cM * Mi[t];
#pragma unroll
      for (int j = 0; j < 4; ++j) pdm += Mtot[j] * Mp[t][j];
      Mb[t] = m * Mtot;
      Gb[t] = Mtot;
      *reinterpret_cast<f32x4*>((dU + si * mat + roff(t))) = Gb[t];
    }
    const float dmv = block_sum<NW>(pdm, red);
    // Sb <- a Sb - Gb K^T + gS
    typename P::Op Bg[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Bg[kb] = P::pack(-Gb[2 * kb], -Gb[2 * kb + 1]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 acc = a * Sb[t] + *reinterpret_cast<const f32x4*>((gS + si * mat + roff(t)));
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) acc = P::mma(row_op<P, PlainMat<D>>(Ki, 16 * t, 32 * kb), Bg[kb], acc);
      Sb[t] = acc;
    }
    if (threadIdx.x == 0) {
      da[si] = dav;
      db[si] = dbv;
      dm[si] = dmv;
      dn[si] = 0.f;
    }
  }
}

// The backward with bf16x3 products, in two kernels on the NSSplit engine
// (two LDS slots of one split matrix each, A and B).
//
// scan_bwd_muon_pre, one workgroup per (b, h, chunk): the forward iterates do
// not depend on the cotangent, so they are rebuilt for every chunk at once
// across the chip.  K_i staged into B; G = U - S_i K_i; M_i = m M_{i-1} + G;
// X_0 = M_i / (|M_i| + eps); then the ns steps, storing each iterate X_k
// (k = 0 .. ns), each P_k = X_k X_k^T and Z_k = b P_k + c P_k^2 as the
// wave's rows in split pieces, M_i in fp32 and |M_i|.  Workspace per chunk:
// 3 ns + 2 matrices.
//
// scan_bwd_muon_x3, one workgroup per (b, h), chunks in reverse order:
//   1. da_i = <Sb, S_i>, db_i = <Sb, X_ns> (S_i, X_ns and gS requested at
//      the end of the previous chunk); Xbar = b Sb; a Sb + gS parked in Sb's
//      workspace rows until the tail.
//   2. The VJP steps, k = ns-1 .. 0, with Xbar published in A and X_k in B:
//        Q    = a Xbar + Z_k Xbar                 (A column reads, Z_k rows)
//        Bbar = Xbar X_k^T                        (A and B row reads)
//        Bs   = Bbar + Bbar^T: Bbar published in A, read back transposed
//        Y    = Bs P_k                            (Bs published in A, P_k rows)
//        Y^T  read back transposed after publishing Y in A
//        Xbar <- Q + (b Bs + c (Y + Y^T)) X_k     (B column reads)
//      (P_k, Bs and Z_k are symmetric.)  Four D^3 products per step: the
//      transposes are LDS reads of the published copies, and P_k comes from
//      the first kernel instead of X_k (X_k^T Bs).
//   3. The normalisation VJP, Gb = dU_i, and Sb <- (a Sb + gS) - Gb K_i^T
//      with K_i staged into B (row reads).  Each phase issues its global
//      loads together ahead of their first use.
// Mbar passes from chunk to chunk through the workspace as fp32 rows of their
// wave.
//
// Segments: the chunks are processed NSEG at a time from the end (pre over
// the segment, then x3 over it), so the per-chunk workspace holds NSEG
// chunks per (b, h) whatever N is; Sb and Mbar carry from one segment to the
// next through the workspace.
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
  extern __shared__ __align__(16) float smem[];
  const lds_ptr SA = lds_base(smem), SB = SA + NSX::BYTES;
  float* red = smem + 2 * NSX::BYTES / 4;
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
  extern __shared__ __align__(16) float smem[];
  const lds_ptr SA = lds_base(smem), SB = SA + NSX::BYTES;
  float* red = smem + 2 * NSX::BYTES / 4;

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
#pragma unroll
      for (int tc = 0; tc < NT; ++tc) Q[tc] = NS_A * X[tc];
      {
        Op Bz[NKB];
        NSX::own_ops(zr, Bz);
        nsx.colprod_all(SA, Bz, Q);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the phases' operands apart
      {
        // Bbar[r'][r] = sum_k Xbar[r'][k] X_k[r][k]: the wave's own rows of
        // X_k (B) as the B operand
#pragma unroll
        for (int tr = 0; tr < NT; ++tr) Bs[tr] = zero4();
        nsx.rowprod_own(SA, SB, Bs);
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

// Blocks 0 .. nx3 - 1: the reverse pass of their head over segment [i0, i1);
// the rest: the iterates of one chunk of segment [j0, j0 + jcur) each.
template <int D>
__global__ void __launch_bounds__(D * 4) scan_bwd_muon_seg(MuonSegArgs sa) {
  const int64_t b = blockIdx.x;
  if (b < sa.nx3)
    muon_x3_body<D>(sa, b);
  else
    muon_pre_body<D>(sa, b - sa.nx3);
}

template <int D, int PREC>
static hipError_t launch_fwd_muon(const ScanArgs& s) {
  const size_t lds = 2 * (size_t)D * D * sizeof(float);
  auto kern = scan_fwd_muon<D, PREC>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)s.BH), dim3(D * 4), lds, s.stream, s.U, s.K, s.a, s.b, s.m,
                     s.S_all, s.M_all, (int)s.N, s.ns);
  return hipGetLastError();
}

template <int D, int PREC>
static hipError_t launch_bwd_muon(const ScanArgs& s, float* ws, int64_t ws_floats) {
  if constexpr (PREC == 0) {
    const int lds = 2 * NSSplit<D>::BYTES + 64;
    auto k = scan_bwd_muon_seg<D>;
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    // Segments of nseg chunks from the end; Sb and Mbar carry from one
    // segment's reverse pass to the next through the workspace.  With two
    // iterate buffers the iterates of segment k + 1 are formed in the launch
    // that runs segment k's reverse pass (only the first segment's run
    // alone); with one, each segment's iterates and then its reverse pass.
    const MuonBwdPlan plan = muon_bwd_plan(s.BH, s.N, D, s.ns, ws_floats);
    if (plan.nseg < 1) return hipErrorInvalidValue;
    const int nseg = (int)plan.nseg;
    MuonSegArgs sa{};
    sa.U = s.U; sa.K = s.K; sa.av = s.a; sa.bv = s.b; sa.mv = s.m; sa.S_all = s.S_all; sa.M_all = s.M_all;
    sa.gS = s.gS; sa.dU = s.dU; sa.da = s.da; sa.db = s.db; sa.dm = s.dm; sa.dn = s.dn; sa.ws = ws;
    sa.BH = s.BH; sa.N = (int)s.N; sa.ns = s.ns; sa.nseg = nseg; sa.nbuf = plan.nbuf;
    auto launch = [&](int nx3, int i0, int i1, int xbuf, int j0, int jcur, int pbuf) {
      sa.nx3 = nx3; sa.i0 = i0; sa.i1 = i1; sa.xbuf = xbuf;
      sa.j0 = j0; sa.jcur = jcur; sa.pbuf = pbuf;
      const int64_t blocks = (int64_t)nx3 + s.BH * jcur;
      hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(D * 4), lds, s.stream, sa);
      return hipGetLastError();
    };
    const int bh = (int)s.BH;
    int i1 = (int)s.N, i0 = i1 > nseg ? i1 - nseg : 0;
    if (plan.nbuf == 2) {
      e = launch(0, 0, 0, 0, i0, i1 - i0, 0);
      for (int seg = 0; e == hipSuccess && i1 > 0; ++seg) {
        const int j1 = i0, j0 = j1 > nseg ? j1 - nseg : 0;
        e = launch(bh, i0, i1, seg & 1, j0, j1 - j0, (seg + 1) & 1);
        i1 = i0;
        i0 = j0;
      }
    } else {
      for (; e == hipSuccess && i1 > 0; i1 = i0, i0 = i1 > nseg ? i1 - nseg : 0) {
        e = launch(0, 0, 0, 0, i0, i1 - i0, 0);
        if (e == hipSuccess) e = launch(bh, i0, i1, 0, 0, 0, 0);
      }
    }
    return e;
  } else {
    auto kern = scan_bwd_muon<D, PREC>;
    hipLaunchKernelGGL(kern, dim3((unsigned)s.BH), dim3(D * 4), 0, s.stream, s.U, s.K, s.a, s.b, s.m,
                       s.S_all, s.M_all, s.gS, s.dU, s.da, s.db, s.dm, s.dn, ws, (int)s.N, s.ns);
    return hipGetLastError();
  }
}

hipError_t scan_fwd_muon_launch(const ScanArgs& s) {
  const bool x3 = s.precision == 0;
  switch (s.dh) {
    case 32: return x3 ? launch_fwd_muon<32, 0>(s) : launch_fwd_muon<32, 1>(s);
    case 64: return x3 ? launch_fwd_muon<64, 0>(s) : launch_fwd_muon<64, 1>(s);
    case 128: return x3 ? launch_fwd_muon<128, 0>(s) : launch_fwd_muon<128, 1>(s);
  }
  return hipErrorInvalidValue;
}

hipError_t scan_bwd_muon_launch(const ScanArgs& s, float* ws, int64_t ws_floats) {
  const bool x3 = s.precision == 0;
  switch (s.dh) {
    case 32: return x3 ? launch_bwd_muon<32, 0>(s, ws, ws_floats) : launch_bwd_muon<32, 1>(s, ws, ws_floats);
    case 64: return x3 ? launch_bwd_muon<64, 0>(s, ws, ws_floats) : launch_bwd_muon<64, 1>(s, ws, ws_floats);
    case 128: return x3 ? launch_bwd_muon<128, 0>(s, ws, ws_floats) : launch_bwd_muon<128, 1>(s, ws, ws_floats);
  }
  return hipErrorInvalidValue;
}

}  // namespace gmdn
