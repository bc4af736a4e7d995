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
// and re-read by the same lanes).  The bf16x3 backward's stages (iterate
// rebuild, serial reverse scan) are in muon_bwd.h; scan_bwd_muon_seg runs
// them a segment at a time.
#include "muon_bwd.h"
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
