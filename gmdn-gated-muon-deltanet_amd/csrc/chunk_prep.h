// Level B: the per-chunk matrices of the reference's matrix form
// (train_ablation.py:161-167, :186), chunk-parallel, for the paths that run
// the drop-in scan kernels between chunk-parallel stages (muon's backward;
// adam's training at d = 128, whose scan runs in exact float32):
//
//   FWD: Kw = K^T diag(w) K,  Uv = V^T diag(w) K               (:164-165)
//   BWD: gS = dL/dS_i = dO^T Qt = dO^T Q - (A^T dO)^T K        (:166, :186)
//   a = exp(sum max(g, log 1e-6)), b = mean beta, m = exp(sum max(gmu, log 1e-6)),
//   n = exp(sum max(gnu, log 1e-6)) (adam; 1 for muon)
//
// with A = tril(Q K^T) diag(beta) and the rule's token weights w (muon:
// w_t = exp(sum_{s > t} max(gmu_s, log 1e-6)), :154-156; adam: 1, :158).
// One workgroup of D/16 waves per (b, h, chunk); every product contracts the
// chunk's 64 tokens.  Wave w forms rows 16w .. 16w+15 of each d x d output from
// transposed tiles (lane <-> output row, registers <-> four consecutive
// columns), so each lane stores 16 contiguous bytes per tile.
#pragma once
#include "chunk_b.h"
#include "scan_a.h"

namespace gmdn {

template <int D>
struct PrepLds {
  static constexpr int NW = D / 16;
  static constexpr int NTHR = 64 * NW;
  static constexpr int TILE = CB_C * D * 2;
  static constexpr int Q0 = 0, K0 = TILE, V0 = 2 * TILE, O0 = 3 * TILE;
  static constexpr int WH0 = 4 * TILE, WL0 = 5 * TILE;  // w K, split
  static constexpr int PH0 = 6 * TILE, PL0 = 7 * TILE;  // P = A^T dO as [s][r], split
  static constexpr int AP = CB_C * CB_C * 2;
  static constexpr int AH0 = 8 * TILE, AL0 = AH0 + AP;  // A^T (rows s), split
  static constexpr int R0 = AL0 + AP;                   // floats: beta, w
  static constexpr int BYTES = R0 + 2 * CB_C * 4;
  static_assert(BYTES <= 160 * 1024, "prep LDS exceeds the 160 KiB of a CU");
};

// The stage for chunk i of head bh (one workgroup of PrepLds<D>::NTHR
// threads with PrepLds<D>::BYTES of dynamic LDS).
template <int D, int RULE, bool FWD, bool BWD>
GMDN_DEV void chunk_prep_body(const ChunkArgs& p, float* __restrict__ Kw, float* __restrict__ Uv,
                              float* __restrict__ gS, float* __restrict__ abm, int64_t bh, int i) {
  static_assert(RULE == 1 || RULE == 2, "the matrix-form stages serve muon and adam");
  using LQ = BSwz<D>;
  using LA = BSwz<CB_C>;
  using L = PrepLds<D>;
  constexpr int NKB = D / 32, NT = D / 16, NW = L::NW, NTHR = L::NTHR;
  extern __shared__ __align__(16) char smem[];
  const bf16* Qs = reinterpret_cast<const bf16*>(smem + L::Q0);
  const bf16* Ks = reinterpret_cast<const bf16*>(smem + L::K0);
  const bf16* Vs = reinterpret_cast<const bf16*>(smem + L::V0);
  const bf16* Os = reinterpret_cast<const bf16*>(smem + L::O0);
  bf16* Wh = reinterpret_cast<bf16*>(smem + L::WH0);
  bf16* Wl = reinterpret_cast<bf16*>(smem + L::WL0);
  bf16* Ph = reinterpret_cast<bf16*>(smem + L::PH0);
  bf16* Pl = reinterpret_cast<bf16*>(smem + L::PL0);
  bf16* Ah = reinterpret_cast<bf16*>(smem + L::AH0);
  bf16* Al = reinterpret_cast<bf16*>(smem + L::AL0);
  float* rbeta = reinterpret_cast<float*>(smem + L::R0);
  float* rw = rbeta + CB_C;

  const int64_t bb = bh / p.H, hh = bh % p.H;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int64_t t0 = (int64_t)i * CB_C, si = bh * p.N + i;
  const int64_t mat = (int64_t)D * D;

  // ---- tiles and gates
  float gbeta = 0.f, gg = 0.f, gm = 0.f, gn = 0.f;
  if (w == 0) {
    const int64_t e = bh * p.T + t0 + l;
    gbeta = p.beta[e];
    gg = p.g[e];
    gm = p.gmu[e];
    if constexpr (RULE == 2) gn = p.gnu[e];
  }
  {
    DmaPlan<LQ, CB_C, NTHR> pk;
    pk.init(w, p.sk[2]);
    const uint32_t lds0 = lds_addr(smem);
    pk.issue(p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], lds0 + L::K0, w);
    if constexpr (FWD) {
      DmaPlan<LQ, CB_C, NTHR> pv;
      pv.init(w, p.sv[2]);
      pv.issue(p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2], lds0 + L::V0, w);
    }
    if constexpr (BWD) {
      DmaPlan<LQ, CB_C, NTHR> pq, po;
      pq.init(w, p.sq[2]);
      po.init(w, p.so[2]);
      pq.issue(p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2], lds0 + L::Q0, w);
      po.issue(p.o + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2], lds0 + L::O0, w);
    }
  }
  wait_vmem();
  if (w == 0) {
    const int64_t BHN = p.B * p.H * p.N;
    const float lg = fmaxf(gg, LOG_FLOOR), lm = fmaxf(gm, LOG_FLOOR);
    const float a = expf(wave_sum(lg));
    const float b = wave_sum(gbeta) * (1.f / CB_C);
    const float msum = wave_sum(lm);
    const float n = RULE == 2 ? expf(wave_sum(fmaxf(gn, LOG_FLOOR))) : 1.f;
    float incl = lm;  // inclusive prefix sum over the tokens
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(incl, o, 64);
      if (l >= o) incl += y;
    }
    rbeta[l] = gbeta;
    rw[l] = RULE == 1 ? expf(msum - incl) : 1.f;  // muon: w_t = exp(sum_{s > t} lm_s)
    if (l == 0) {
      abm[si] = a;
      abm[BHN + si] = b;
      abm[2 * BHN + si] = expf(msum);
      abm[3 * BHN + si] = n;
    }
  }
  __syncthreads();

  if constexpr (FWD) {
    // ---- w K (split planes)
    for (int e = threadIdx.x; e < CB_C * D / 8; e += NTHR) {
      const int t = e / (D / 8), c8 = (e % (D / 8)) * 8;
      const int off = LQ::off(t, c8);
      const bf16x8 kv = *reinterpret_cast<const bf16x8*>(Ks + off);
      const float wt = rw[t];
      bf16x4 h0, l0, h1, l1;
      split4(f32x4{wt * (float)kv[0], wt * (float)kv[1], wt * (float)kv[2], wt * (float)kv[3]}, h0, l0);
      split4(f32x4{wt * (float)kv[4], wt * (float)kv[5], wt * (float)kv[6], wt * (float)kv[7]}, h1, l1);
      const bf16x8 hi = cat8(h0, h1), lo = cat8(l0, l1);
      *reinterpret_cast<bf16x8*>(Wh + off) = hi;
      *reinterpret_cast<bf16x8*>(Wl + off) = lo;
    }
  }
  if constexpr (BWD) {
    // ---- A^T (split planes, tiles above the diagonal zero)
#pragma unroll
    for (int kk = 0; kk < 16 / NW; ++kk) {
      const int k = w + NW * kk, tt = k >> 2, st = k & 3;
      bf16x4 ah, al;
      if (tt < st) {
        ah = al = bf16x4{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
      } else {
        f32x4 X = zero4();
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
          X = mfma(row8<LQ>(Qs, 16 * tt + lc, 32 * kb), row8<LQ>(Ks, 16 * st + lc, 32 * kb), X);
        // lane (s, G) holds A[t = 16 tt + 4G + jj][s = 16 st + lc]
        const float bs = rbeta[16 * st + lc];
        f32x4 xv;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) xv[jj] = (tt > st || 4 * G + jj >= lc) ? X[jj] * bs : 0.f;
        split4(xv, ah, al);
      }
      const int ao = LA::off(16 * st + lc, 16 * tt + 4 * G);
      *reinterpret_cast<bf16x4*>(Ah + ao) = ah;
      *reinterpret_cast<bf16x4*>(Al + ao) = al;
    }
    __syncthreads();  // A^T published (w K too, when formed)

    // ---- P = A^T dO for this wave's 16 dO columns r0 .. : lane (s, G) of tile
    // st holds P^T[r0 + 4G + jj][16 st + s]; published as [s][r] split planes
    const int r0 = 16 * w;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      f32x4 Pt = zero4();
#pragma unroll
      for (int kbt = 0; kbt < 2; ++kbt) {
        if (32 * kbt + 31 < 16 * st) continue;
        const Op<1> dOt{{col8<LQ>(Os, 32 * kbt, r0)}};
        const Op<2> At{{row8<LA>(Ah, 16 * st + lc, 32 * kbt), row8<LA>(Al, 16 * st + lc, 32 * kbt)}};
        Pt = mma<1, 2>(dOt, At, Pt);
      }
      bf16x4 h4, l4;
      split4(Pt, h4, l4);
      const int po = LQ::off(16 * st + lc, r0 + 4 * G);
      *reinterpret_cast<bf16x4*>(Ph + po) = h4;
      *reinterpret_cast<bf16x4*>(Pl + po) = l4;
    }
  }
  __syncthreads();

  // ---- the d x d outputs, rows a0 + lc of each: out[a][b] = sum_t X[t][a] Y[t][b]
  // as transposed tiles D[b][a] (A operand: Y columns b, B operand: X columns a)
  const int a0 = 16 * w;
  const int64_t orow = si * mat + (int64_t)(a0 + lc) * D + 4 * G;
  if constexpr (FWD) {
    Op<1> Vc[2];
    Op<2> Wc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      Vc[kt].v[0] = col8<LQ>(Vs, 32 * kt, a0);
      Wc[kt] = Op<2>{{col8<LQ>(Wh, 32 * kt, a0), col8<LQ>(Wl, 32 * kt, a0)}};
    }
#pragma unroll
    for (int bt = 0; bt < NT; ++bt) {
      f32x4 kw = zero4(), uv = zero4();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const Op<2> wcol{{col8<LQ>(Wh, 32 * kt, 16 * bt), col8<LQ>(Wl, 32 * kt, 16 * bt)}};
        kw = mma<1, 2>(Op<1>{{col8<LQ>(Ks, 32 * kt, 16 * bt)}}, Wc[kt], kw);  // sum_t K[t][b] (w K)[t][a]
        uv = mma<2, 1>(wcol, Vc[kt], uv);                                     // sum_t (w K)[t][b] V[t][a]
      }
      *reinterpret_cast<f32x4*>(Kw + orow + 16 * bt) = kw;
      *reinterpret_cast<f32x4*>(Uv + orow + 16 * bt) = uv;
    }
  }
  if constexpr (BWD) {
    Op<1> Oc[2];
    Op<2> Pc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      Oc[kt].v[0] = col8<LQ>(Os, 32 * kt, a0);
      Pc[kt] = Op<2>{{col8<LQ>(Ph, 32 * kt, a0), col8<LQ>(Pl, 32 * kt, a0)}};
    }
#pragma unroll
    for (int bt = 0; bt < NT; ++bt) {
      f32x4 gs = zero4();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        gs = mma<1, 1>(Op<1>{{col8<LQ>(Qs, 32 * kt, 16 * bt)}}, Oc[kt], gs);           // sum_t Q[t][b] dO[t][a]
        gs = mma<1, 2>(Op<1>{{neg8(col8<LQ>(Ks, 32 * kt, 16 * bt))}}, Pc[kt], gs);     // - sum_t K[t][b] P[t][a]
      }
      *reinterpret_cast<f32x4*>(gS + orow + 16 * bt) = gs;
    }
  }
}

}  // namespace gmdn
