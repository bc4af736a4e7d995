// Exact WY/UT mode: the token-exact gated delta rule
//     S_t = alpha_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T,   o_t = S_t q_t
// chunked with the WY/UT transform (the reference trains the chunk-frozen
// E-form instead and leaves this mode out, train_ablation.py:12-18).
//
// Per (b, h) and chunk of C = 64 tokens, with gc_t the prefix sum of the
// clamped log-gates from the chunk start, gamma_t = exp(gc_t),
// Gamma[t, s] = exp(gc_t - gc_s) (formed on the causal entries s <= t only,
// so that no ratio of two underflowed products appears) and
// kd_t = gamma_C / gamma_t:
//     A = strict_lower(diag(beta) (K K^T * Gamma)),   T = (I + A)^-1
//     U = T diag(beta) V,  W = T diag(beta gamma) K,  X = U - W S^T
//     o = diag(gamma) Q S^T + M X,   M = lower_incl(Q K^T * Gamma)
//     S' = gamma_C S + X^T diag(kd) K
// The state recurrence is affine, S' = a S + U_A - S K_A, which is the
// drop-in delta scan's (fast_scan.py:82) with
//     a = gamma_C,  U_A = (diag(beta) V)^T P,  K_A = (diag(beta gamma) K)^T P,
//     P = T^T diag(kd) K,
// and the output is o = Qt S^T + Ov with
//     Qt = diag(gamma) Q - (M T diag(beta gamma)) K,  Ov = (M T diag(beta)) V.
//
// Forward: wy_prep (one workgroup of 8 waves per (b, h, chunk)) forms a, U_A,
// K_A, Qt and Ov: bf16 q, k, v enter the products exactly, float32
// intermediates as split hi + lo bf16 operands; T by blocked forward
// substitution in float32.  The drop-in delta scan kernels carry S
// (split-bf16 state products); wy_out forms o = Qt S_i^T + Ov (split-bf16).
// Its workspace [U_A | K_A | S_all | Qt | Ov | a] is the backward's checkpoint.
//
// Backward, given dO:
//   wy_gs     gS_i = dL/dS_i through o = dO^T Qt                 (chunk-parallel)
//   the drop-in delta scan's reverse kernel (split-bf16) on (U_A, K_A, a, S_all,
//             gS): its dU_i is Sb = dL/dS_{i+1}, the state cotangent after chunk i
//   wy_tok1 / wy_tok2: the VJP of the chunk algebra in the X-form above, per
//             chunk from S_i and Sb (chunk-parallel):
//     dX  = M^T dO + diag(kd) K Sb^T,  dQt~ = dO S_i,  dM = lower_incl(dO X^T),
//     dK~ = X Sb,  dW = -dX S_i,  dgamma_C = <Sb, S_i>,
//     dT  = dX (diag(beta) V)^T + dW (diag(beta gamma) K)^T,
//     d(diag(beta) V) = T^T dX,  d(diag(beta gamma) K) = T^T dW,
//     dA  = strict_lower(-T^T dT T^T),
//     then A, M, gamma, kd and Gamma back to q, k, v, beta and the log-gates
//     (Gamma's exponent differences give dgc_t as row minus column sums of
//     dGamma * Gamma; dg_u = sum_{t >= u} dgc_t where g_u is above its floor).
//   wy_tok1 runs up to dT (dv final; partial dq, dk; T, dT, dM and per-token
//   gate partials to the workspace), wy_tok2 the rest (dA, the A and M terms,
//   the gate gradients).
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"
#include "f32mm.h"
#include "scan_a.h"

namespace gmdn {
namespace {

constexpr int WY_THREADS = 256;

// Per-token gate quantities of the chunk (wave 0, lane = token): beta, gamma,
// beta gamma, kd = gamma_C / gamma and log gamma (the prefix sums of the
// clamped log-gates) into LDS; returns gamma of this lane's token.
GMDN_DEV float wy_gates(const float* beta, const float* g, int64_t e, float* bet, float* gam, float* bg,
                        float* kd, float* lgam) {
  const int l = lane_id();
  const float bt = beta[e];
  const float gc = wave_incl_scan(fmaxf(g[e], LOG_FLOOR));
  const float gC = __shfl(gc, 63, 64);
  const float g_ = expf(gc);
  bet[l] = bt;
  gam[l] = g_;
  bg[l] = bt * g_;
  kd[l] = expf(gC - gc);
  lgam[l] = gc;
  return g_;
}

// T = (I + A)^-1 for a strictly lower C x C matrix A (row stride LDC) into Ts,
// which must be zero on entry.  The four 16 x 16 diagonal blocks by forward
// substitution (wave w, lane j < 16 holds column j of block w), then the
// off-diagonal blocks T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj level by level
// (d = i - j; wave w takes the block with j = w).  Waves 0-3 work; any
// further waves of the workgroup only take part in the barriers.  Xw: 3 x 256
// floats of scratch.  Ends with a barrier.
template <int LDC>
GMDN_DEV void tri_inverse(const float* As, float* Ts, float* Xw_all) {
  const int w = wave_id(), l = lane_id();
  if (w < 4 && l < 16) {
    const int o = 16 * w;
    float x[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float s = t == l ? 1.f : 0.f;
#pragma unroll
      for (int u = 0; u < t; ++u) s -= As[(o + t) * LDC + o + u] * x[u];
      x[t] = s;
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) Ts[(o + t) * LDC + o + l] = x[t];
  }
  __syncthreads();
  float* Xw = Xw_all + 256 * (w < 3 ? w : 0);
  for (int d = 1; d < 4; ++d) {
    const int j = w, ii = w + d;
    const int r = l >> 2, c = 4 * (l & 3);
    if (ii < 4) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int kb = j; kb < ii; ++kb)
#pragma unroll 4
        for (int u = 0; u < 16; ++u) {
          const float a = As[(16 * ii + r) * LDC + 16 * kb + u];
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[q] += a * Ts[(16 * kb + u) * LDC + 16 * j + c + q];
        }
#pragma unroll
      for (int q = 0; q < 4; ++q) Xw[r * 16 + c + q] = acc[q];
    }
    __syncthreads();
    if (ii < 4) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
      for (int u = 0; u < 16; ++u) {
        const float a = Ts[(16 * ii + r) * LDC + 16 * ii + u];
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] += a * Xw[u * 16 + c + q];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) Ts[(16 * ii + r) * LDC + 16 * j + c + q] = -acc[q];
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ forward
// wy_prep: one workgroup of 8 waves per (b, h, chunk).  q, k, v stay bf16 in
// LDS (row swizzle BSwz) and enter the products exactly; A, T, M and the
// decays are float32, and every float32 operand of a product is split into
// hi + lo bf16 (three MFMAs for two split operands, two for one: about
// 2^-16 relative error per product).
//   A  = strict_lower(diag(beta)(K K^T * Gamma))     float32 tiles, for T
//   T  = (I + A)^-1                                 forward substitution (float32)
//   M  = lower_incl(Q K^T * Gamma)                  split planes, rows t
//   (M T)^T tiles [u][t], scaled by beta gamma_u (Qt) or beta_u (Ov) per
//       row, are directly the pair-order operand of the next product:
//   Qt = diag(gamma) Q - (M T diag(beta gamma)) K,  Ov = (M T diag(beta)) V
//   P  = T^T diag(kd) K, tiles [s][c], scaled by beta_s / beta gamma_s:
//   U_A = V^T (diag(beta) P),  K_A = K^T (diag(beta gamma) P)
// (the same algebra, with diag(beta) moved onto P.)
constexpr int WYP_THREADS = 512;

template <int D>
struct WyPrepLds {
  static constexpr int C = CB_C;
  static constexpr int TB = C * D * 2;    // bf16 token tile (bytes)
  static constexpr int CP = C * C * 2;    // one bf16 C x C plane
  static constexpr int LDC = C + 4;       // float stride of A and T rows
  static constexpr int CF = C * LDC * 4;  // float C x C
  static constexpr int K0 = 0, Q0 = TB, V0 = 2 * TB;
  static constexpr int A0 = 3 * TB, T0 = A0 + CF;
  static constexpr int X0 = T0 + CF;  // tri_inverse scratch, 3 x 256 floats
  // split planes (hi, lo) of T, diag(kd) T and M
  static constexpr int TH0 = X0 + 3 * 1024, TL0 = TH0 + CP, KH0 = TL0 + CP, KL0 = KH0 + CP, MH0 = KL0 + CP,
                       ML0 = MH0 + CP;
  static constexpr int R0 = ML0 + CP;  // beta, gamma, beta gamma, kd, log gamma
  static constexpr int BYTES = R0 + 5 * C * 4;
  static_assert(BYTES <= 160 * 1024, "WY prep LDS exceeds the 160 KiB of a CU");
};

// the causal 16 x 16 tiles (row tile >= column tile) of a C x C matrix
GMDN_DEV void causal_tile(int idx, int& tt, int& st) {
  tt = idx < 1 ? 0 : idx < 3 ? 1 : idx < 6 ? 2 : 3;
  st = idx - tt * (tt + 1) / 2;
}

// Staging through registers with every global load of a phase issued before
// the first LDS store (one memory latency per phase, not one per loop trip).
// Rows x W floats (row stride ld) -> split planes BSwz<W>.
template <int W, int ROWS, int NTHR>
struct SplitRows {
  static constexpr int PER = ROWS * (W / 8) / NTHR;
  static_assert(ROWS * (W / 8) % NTHR == 0, "whole 8-column groups per thread");
  f32x4 x[PER][2];
  GMDN_DEV void load(const float* src, int64_t ld) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = threadIdx.x + q * NTHR, r = e / (W / 8), c = (e % (W / 8)) * 8;
      x[q][0] = *reinterpret_cast<const f32x4*>(src + r * ld + c);
      x[q][1] = *reinterpret_cast<const f32x4*>(src + r * ld + c + 4);
    }
  }
  // zero the entries above the diagonal (square matrices)
  GMDN_DEV void lower() {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = threadIdx.x + q * NTHR, r = e / (W / 8), c = (e % (W / 8)) * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (c + j > r) x[q][0][j] = 0.f;
        if (c + 4 + j > r) x[q][1][j] = 0.f;
      }
    }
  }
  GMDN_DEV void store(bf16* hi, bf16* lo) const {
    using LW = BSwz<W>;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = threadIdx.x + q * NTHR, r = e / (W / 8), c = (e % (W / 8)) * 8;
      bf16x4 h0, o0, h1, o1;
      split4(x[q][0], h0, o0);
      split4(x[q][1], h1, o1);
      *reinterpret_cast<bf16x8*>(hi + LW::off(r, c)) = cat8(h0, h1);
      *reinterpret_cast<bf16x8*>(lo + LW::off(r, c)) = cat8(o0, o1);
    }
  }
};

// A chunk's bf16 token rows (row stride `stride`) -> BSwz<D> tile
template <int D, int NTHR>
struct TokRows {
  static constexpr int PER = CB_C * (D / 8) / NTHR;
  static_assert(CB_C * (D / 8) % NTHR == 0, "whole 8-column groups per thread");
  bf16x8 x[PER];
  GMDN_DEV void load(const bf16* src, int64_t stride) {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = threadIdx.x + q * NTHR, t = e / (D / 8), c = (e % (D / 8)) * 8;
      x[q] = *reinterpret_cast<const bf16x8*>(src + t * stride + c);
    }
  }
  GMDN_DEV void store(bf16* dst) const {
    using LT = BSwz<D>;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int e = threadIdx.x + q * NTHR, t = e / (D / 8), c = (e % (D / 8)) * 8;
      *reinterpret_cast<bf16x8*>(dst + LT::off(t, c)) = x[q];
    }
  }
};

template <int D>
__global__ void __launch_bounds__(WYP_THREADS)
wy_prep(ChunkArgs p, float* __restrict__ UA, float* __restrict__ KA, float* __restrict__ Qt,
        float* __restrict__ Ov, float* __restrict__ aout) {
  using L = WyPrepLds<D>;
  using LT = BSwz<D>;      // token tiles
  using LP = BSwz<CB_C>;   // C x C planes
  constexpr int C = CB_C, LDC = L::LDC, NT = D / 16, NKB = D / 32;
  extern __shared__ __align__(16) char smem[];
  bf16* Kb = reinterpret_cast<bf16*>(smem + L::K0);
  bf16* Qb = reinterpret_cast<bf16*>(smem + L::Q0);
  bf16* Vb = reinterpret_cast<bf16*>(smem + L::V0);
  float* As = reinterpret_cast<float*>(smem + L::A0);
  float* Ts = reinterpret_cast<float*>(smem + L::T0);
  bf16* Th = reinterpret_cast<bf16*>(smem + L::TH0);
  bf16* Tl = reinterpret_cast<bf16*>(smem + L::TL0);
  bf16* KTh = reinterpret_cast<bf16*>(smem + L::KH0);
  bf16* KTl = reinterpret_cast<bf16*>(smem + L::KL0);
  bf16* Mh = reinterpret_cast<bf16*>(smem + L::MH0);
  bf16* Ml = reinterpret_cast<bf16*>(smem + L::ML0);
  float* bet = reinterpret_cast<float*>(smem + L::R0);
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;

  // ---- bf16 tiles, gates; T and the M planes zeroed
  const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2];
  const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2];
  const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2];
  {
    TokRows<D, WYP_THREADS> tk, tq, tv;
    tk.load(kg, p.sk[2]);
    tq.load(qg, p.sq[2]);
    tv.load(vg, p.sv[2]);
    tk.store(Kb);
    tq.store(Qb);
    tv.store(Vb);
  }
  for (int e = threadIdx.x; e < C * LDC / 4; e += WYP_THREADS) reinterpret_cast<f32x4*>(Ts)[e] = zero4();
  for (int e = threadIdx.x; e < 2 * L::CP / 16; e += WYP_THREADS) reinterpret_cast<f32x4*>(Mh)[e] = zero4();
  if (w == 0) {
    const float g_ = wy_gates(p.beta, p.g, bh * p.T + t0 + l, bet, gam, bg, kd, lgam);
    if (l == 63) aout[bh * p.N + i] = g_;
  }
  __syncthreads();

  // ---- A's causal tiles (float32, for the substitution) and M's (split
  //      planes): jobs 0-9 and 10-19 over the waves
  for (int job = w; job < 20; job += WYP_THREADS / 64) {
    int tt, st;
    causal_tile(job % 10, tt, st);
    if (job < 10) {
      // A[t][s] = beta_t Gamma[t][s] sum_c K[t][c] K[s][c]
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        acc = mfma(row8<LT>(Kb, 16 * tt + lc, 32 * kb), row8<LT>(Kb, 16 * st + lc, 32 * kb), acc);
      const int s = 16 * st + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tt + 4 * G + j;
        acc[j] = s < t ? bet[t] * acc[j] * expf(lgam[t] - lgam[s]) : 0.f;
      }
      st_tile(As, LDC, 16 * tt, 16 * st, acc);
    } else {
      // M^T[s][t] = Gamma[t][s] sum_c K[s][c] Q[t][c], stored as rows t of M
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        acc = mfma(row8<LT>(Kb, 16 * st + lc, 32 * kb), row8<LT>(Qb, 16 * tt + lc, 32 * kb), acc);
      const int t = 16 * tt + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = 16 * st + 4 * G + j;
        acc[j] = s <= t ? acc[j] * expf(lgam[t] - lgam[s]) : 0.f;
      }
      bf16x4 h, o;
      split4(acc, h, o);
      *reinterpret_cast<bf16x4*>(Mh + LP::off(t, 16 * st + 4 * G)) = h;
      *reinterpret_cast<bf16x4*>(Ml + LP::off(t, 16 * st + 4 * G)) = o;
    }
  }
  __syncthreads();
  tri_inverse<LDC>(As, Ts, reinterpret_cast<float*>(smem + L::X0));

  // ---- split planes of T and diag(kd) T (one 8-column group per thread)
  {
    const int r = threadIdx.x >> 3, c = (threadIdx.x & 7) * 8;
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(Ts + r * LDC + c);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(Ts + r * LDC + c + 4);
    bf16x4 h0, o0, h1, o1;
    split4(x0, h0, o0);
    split4(x1, h1, o1);
    *reinterpret_cast<bf16x8*>(Th + LP::off(r, c)) = cat8(h0, h1);
    *reinterpret_cast<bf16x8*>(Tl + LP::off(r, c)) = cat8(o0, o1);
    const float k_ = kd[r];
    split4(k_ * x0, h0, o0);
    split4(k_ * x1, h1, o1);
    *reinterpret_cast<bf16x8*>(KTh + LP::off(r, c)) = cat8(h0, h1);
    *reinterpret_cast<bf16x8*>(KTl + LP::off(r, c)) = cat8(o0, o1);
  }
  __syncthreads();

  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D;
  // ---- Qt (waves 0-3) or Ov (waves 4-7) of token tile tt
  {
    const bool ov = w >= 4;
    const int tt = w & 3;
    // (M T)^T[u][t] = sum_s T[s][u] M[t][s], causal (u <= t)
    f32x4 mt[4];
#pragma unroll
    for (int ut = 0; ut < 4; ++ut) {
      mt[ut] = zero4();
      if (ut <= tt) {
        for (int kb = ut >> 1; kb <= (tt >> 1); ++kb)
          mt[ut] = mma<2, 2>(Op<2>{{col8<LP>(Th, 32 * kb, 16 * ut), col8<LP>(Tl, 32 * kb, 16 * ut)}},
                             Op<2>{{row8<LP>(Mh, 16 * tt + lc, 32 * kb), row8<LP>(Ml, 16 * tt + lc, 32 * kb)}},
                             mt[ut]);
        const float* sc = ov ? bet : bg;
#pragma unroll
        for (int j = 0; j < 4; ++j) mt[ut][j] *= sc[16 * ut + 4 * G + j];
      }
    }
    // pair order over u: the operand's free index is t
    const Op<2> a0 = pack_tiles<2>(mt[0], mt[1]), a1 = pack_tiles<2>(mt[2], mt[3]);
    const bf16* Bt = ov ? Vb : Kb;
    float* out = (ov ? Ov : Qt) + tokbase;
#pragma unroll 2
    for (int tc = 0; tc < NT; ++tc) {
      f32x4 acc = mma<2, 1>(a0, Op<1>{{b_col<LT>(Bt, 0, 16 * tc)}}, zero4());
      if (tt >= 2) acc = mma<2, 1>(a1, Op<1>{{b_col<LT>(Bt, 32, 16 * tc)}}, acc);
      const int c = 16 * tc + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tt + 4 * G + j;
        out[(int64_t)t * D + c] = ov ? acc[j] : gam[t] * (float)Qb[LT::off(t, c)] - acc[j];
      }
    }
  }

  // ---- P column tile ct, then U_A and K_A columns ct over the wave's row tiles
  {
    constexpr int WPC = (WYP_THREADS / 64) / NT;  // waves per column tile
    const int ct = w % NT, part = w / NT;
    f32x4 pt[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      // P[s][c] = sum_t kd_t T[t][s] K[t][c], T[t][s] = 0 for t < s
      pt[st] = zero4();
      for (int kb = st >> 1; kb < 2; ++kb)
        pt[st] = mma<2, 1>(Op<2>{{col8<LP>(KTh, 32 * kb, 16 * st), col8<LP>(KTl, 32 * kb, 16 * st)}},
                           Op<1>{{col8<LT>(Kb, 32 * kb, 16 * ct)}}, pt[st]);
    }
    f32x4 pb[4], pg[4];
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = 16 * st + 4 * G + j;
        pb[st][j] = bet[s] * pt[st][j];
        pg[st][j] = bg[s] * pt[st][j];
      }
    const Op<2> bp[2] = {pack_tiles<2>(pb[0], pb[1]), pack_tiles<2>(pb[2], pb[3])};
    const Op<2> bq[2] = {pack_tiles<2>(pg[0], pg[1]), pack_tiles<2>(pg[2], pg[3])};
    const int64_t mbase = (bh * p.N + i) * (int64_t)D * D;
    constexpr int RPW = NT / WPC;
#pragma unroll 2
    for (int rt = part * RPW; rt < (part + 1) * RPW; ++rt) {
      f32x4 ua = zero4(), ka = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        ua = mma<1, 2>(Op<1>{{b_col<LT>(Vb, 32 * kb, 16 * rt)}}, bp[kb], ua);
        ka = mma<1, 2>(Op<1>{{b_col<LT>(Kb, 32 * kb, 16 * rt)}}, bq[kb], ka);
      }
      st_tile(UA + mbase, D, 16 * rt, 16 * ct, ua);
      st_tile(KA + mbase, D, 16 * rt, 16 * ct, ka);
    }
  }
}

// o = Qt S_i^T + Ov for one (b, h, chunk): S_i as split planes in LDS (rows r),
// Qt rows of the wave's token tile split in registers
template <int D>
__global__ void __launch_bounds__(WY_THREADS)
wy_out(ChunkArgs p, const float* __restrict__ Qt, const float* __restrict__ Ov, const float* __restrict__ Sst) {
  using LS = BSwz<D>;
  constexpr int C = CB_C, NT = D / 16, NKB = D / 32;
  extern __shared__ __align__(16) char smem[];
  bf16* Sh = reinterpret_cast<bf16*>(smem);
  bf16* Sl = Sh + D * D;
  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D;
  const float* S = Sst + (bh * p.N + i) * (int64_t)D * D;
  SplitRows<D, D, WY_THREADS> sr;
  sr.load(S, D);
  // lane (t, G) of k-block kb: Qt[16 w + t][32 kb + 8G .. +7]
  Op<2> qa[NKB];
  {
    const float* qr = Qt + tokbase + (int64_t)(16 * w + lc) * D + 8 * G;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      bf16x4 h0, o0, h1, o1;
      split4(*reinterpret_cast<const f32x4*>(qr + 32 * kb), h0, o0);
      split4(*reinterpret_cast<const f32x4*>(qr + 32 * kb + 4), h1, o1);
      qa[kb] = Op<2>{{cat8(h0, h1), cat8(o0, o1)}};
    }
  }
  sr.store(Sh, Sl);
  __syncthreads();
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2];
#pragma unroll 2
  for (int rt = 0; rt < NT; ++rt) {
    // tile [t][r] = sum_c Qt[t][c] S[r][c]
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      acc = mma<2, 2>(qa[kb], Op<2>{{row8<LS>(Sh, 16 * rt + lc, 32 * kb), row8<LS>(Sl, 16 * rt + lc, 32 * kb)}}, acc);
    const int r = 16 * rt + lc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * w + 4 * G + j;
      og[t * p.so[2] + r] = (bf16)(acc[j] + Ov[tokbase + (int64_t)t * D + r]);
    }
  }
}

// ----------------------------------------------------------------- backward
// Chunk-parallel kernels of 8 waves; intermediates of one chunk pass
// through the workspace.  Split-bf16 products as in the forward; S_i and Sb
// are staged in LDS as split planes (rows r, BSwz), one of them per kernel.
// Wave w takes token tile tt = w % 4 and the feature half h = w / 4 of
// every C x d result.
//   wy_gs  gS = dO^T Qt
//   wy_ka  (S_i)  A, T (to the workspace); W, U; X = U - W S^T;
//                 dq1 = diag(gamma) dO S; Z = diag(beta) V - diag(beta gamma) K S^T
//   wy_kb  (Sb)   M; dM = lower_incl(dO X^T); dX = M^T dO + diag(kd) K Sb^T;
//                 dk2 = diag(kd) X Sb; <Sb, S_i>
//   wy_kc1 (S_i)  R = T^T dX: dv = diag(beta) R; dk2 -= diag(beta gamma) R S;
//                 dT = dX Z^T (the lower tiles; with dW = -dX S, dW (diag(beta gamma) K)^T
//                 = -dX (diag(beta gamma) K S^T)^T)
//   wy_kc2        dA = strict_lower(-T^T dT T^T); the A and M terms of dq, dk; the gates
// Per-token partial sums (one slot per feature half) go to the chunk's
// `tokp` record and are added in a fixed order: the gradients are bitwise
// reproducible.
struct WyBwd {
  const float *UA, *KA, *S_all, *Qt, *av;  // forward checkpoint
  const bf16* dO;                         // strides so
  float* gS;                              // wy_gs output
  const float* Sb;                        // the reverse scan's dU (= dL/dS_{i+1})
  float *T, *dM, *dT;                     // C x C per chunk
  float *X, *Z, *dX, *dq1, *dk2;          // B H T d each
  float* tokp;                            // per chunk, TOKP floats (below)
  bf16 *dq, *dk, *dv;
  float *dbeta, *dg;
};
// tokp record: [dgamma from q: 2 C][dkd: 2 C][beta-side of U: 2 C][beta gamma-side of W: 2 C][<Sb, S_i>]
constexpr int TOKP = 8 * CB_C + 4;
constexpr int TP_GQ = 0, TP_KD = 2 * CB_C, TP_SB = 4 * CB_C, TP_SBG = 6 * CB_C, TP_DA = 8 * CB_C;

constexpr int WYB_THREADS = 512;

// split operand from a float row in global memory: lane (i, G) takes
// X[r0 + i][k0 + 8G .. +7] (natural k order)
GMDN_DEV Op<2> gl_row_op(const float* X, int64_t ld, int r0, int k0) {
  const int l = lane_id();
  const float* s = X + (int64_t)(r0 + (l & 15)) * ld + k0 + 8 * (l >> 4);
  bf16x4 h0, o0, h1, o1;
  split4(*reinterpret_cast<const f32x4*>(s), h0, o0);
  split4(*reinterpret_cast<const f32x4*>(s + 4), h1, o1);
  return Op<2>{{cat8(h0, h1), cat8(o0, o1)}};
}

// split planes' natural-order row / column operands
template <class L>
GMDN_DEV Op<2> prow(const bf16* hi, const bf16* lo, int r, int k0) {
  return Op<2>{{row8<L>(hi, r, k0), row8<L>(lo, r, k0)}};
}
template <class L>
GMDN_DEV Op<2> pcol(const bf16* hi, const bf16* lo, int k0, int c0) {
  return Op<2>{{col8<L>(hi, k0, c0), col8<L>(lo, k0, c0)}};
}
// pair-order row / column operands
template <class L>
GMDN_DEV Op<2> prow_p(const bf16* hi, const bf16* lo, int r0, int k0) {
  return Op<2>{{b_row<L>(hi, r0, k0), b_row<L>(lo, r0, k0)}};
}
template <class L>
GMDN_DEV Op<2> pcol_p(const bf16* hi, const bf16* lo, int k0, int c0) {
  return Op<2>{{b_col<L>(hi, k0, c0), b_col<L>(lo, k0, c0)}};
}
// a natural-order split row operand scaled per k by sc[k0 + 8G + j]
GMDN_DEV Op<2> scale_op(const Op<2>& x, const float* sc, int k0) {
  const int G = lane_id() >> 4;
  f32x4 a, b;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a[j] = ((float)x.v[0][j] + (float)x.v[1][j]) * sc[k0 + 8 * G + j];
    b[j] = ((float)x.v[0][4 + j] + (float)x.v[1][4 + j]) * sc[k0 + 8 * G + 4 + j];
  }
  bf16x4 h0, o0, h1, o1;
  split4(a, h0, o0);
  split4(b, h1, o1);
  return Op<2>{{cat8(h0, h1), cat8(o0, o1)}};
}

// gS[r][c] = sum_t dO[t][r] Qt[t][c]
template <int D>
__global__ void __launch_bounds__(WY_THREADS) wy_gs(ChunkArgs p, WyBwd b) {
  using LT = BSwz<D>;
  constexpr int C = CB_C, NT = D / 16;
  extern __shared__ __align__(16) char smem[];
  bf16* Ob = reinterpret_cast<bf16*>(smem);
  bf16* Qh = Ob + C * D;
  bf16* Ql = Qh + C * D;
  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id();
  {
    TokRows<D, WY_THREADS> to;
    SplitRows<D, CB_C, WY_THREADS> sq;
    to.load(b.dO + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2], p.so[2]);
    sq.load(b.Qt + (bh * p.T + t0) * (int64_t)D, D);
    to.store(Ob);
    sq.store(Qh, Ql);
  }
  __syncthreads();
  float* gS = b.gS + si * (int64_t)D * D;
  for (int tile = w; tile < NT * NT; tile += WY_THREADS / 64) {
    const int rt = tile / NT, ct = tile % NT;
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      acc = mma<1, 2>(Op<1>{{col8<LT>(Ob, 32 * kb, 16 * rt)}}, pcol<LT>(Qh, Ql, 32 * kb, 16 * ct), acc);
    st_tile(gS, D, 16 * rt, 16 * ct, acc);
  }
}

template <int D>
struct WyKaLds {
  static constexpr int C = CB_C, TB = C * D * 2, CP = C * C * 2, LDC = C + 4, CF = C * LDC * 4;
  static constexpr int K0 = 0, V0 = TB, O0 = 2 * TB, R0 = 3 * TB;
  // region R: A, T (float32) and the substitution's scratch, then the S_i planes
  static constexpr int RB = 4 * D * D > 2 * CF + 3072 ? 4 * D * D : 2 * CF + 3072;
  static constexpr int TH0 = R0 + RB, TL0 = TH0 + CP, G0 = TL0 + CP;
  static constexpr int BYTES = G0 + 5 * C * 4;
  static_assert(BYTES <= 160 * 1024, "WY backward LDS exceeds the 160 KiB of a CU");
};

template <int D>
__global__ void __launch_bounds__(WYB_THREADS) wy_ka(ChunkArgs p, WyBwd b) {
  using L = WyKaLds<D>;
  using LT = BSwz<D>;
  using LP = BSwz<CB_C>;
  constexpr int C = CB_C, LDC = L::LDC, NT = D / 16, NKB = D / 32, NH = NT / 2;
  extern __shared__ __align__(16) char smem[];
  bf16* Kb = reinterpret_cast<bf16*>(smem + L::K0);
  bf16* Vb = reinterpret_cast<bf16*>(smem + L::V0);
  bf16* Ob = reinterpret_cast<bf16*>(smem + L::O0);
  float* As = reinterpret_cast<float*>(smem + L::R0);
  float* Ts = As + C * LDC;
  bf16* Sh = reinterpret_cast<bf16*>(smem + L::R0);
  bf16* Sl = Sh + D * D;
  bf16* Th = reinterpret_cast<bf16*>(smem + L::TH0);
  bf16* Tl = reinterpret_cast<bf16*>(smem + L::TL0);
  float* bet = reinterpret_cast<float*>(smem + L::G0);
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D;
  const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2];

  // S_i's loads stay in flight through A and T (its planes replace them in region R)
  SplitRows<D, D, WYB_THREADS> sr;
  {
    TokRows<D, WYB_THREADS> tk, tv, to;
    tk.load(p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], p.sk[2]);
    tv.load(p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2], p.sv[2]);
    to.load(b.dO + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2], p.so[2]);
    sr.load(b.S_all + si * (int64_t)D * D, D);
    tk.store(Kb);
    tv.store(Vb);
    to.store(Ob);
  }
  for (int e = threadIdx.x; e < C * LDC / 4; e += WYB_THREADS) reinterpret_cast<f32x4*>(Ts)[e] = zero4();
  if (w == 0) wy_gates(p.beta, p.g, bh * p.T + t0 + l, bet, gam, bg, kd, lgam);
  __syncthreads();
  // ---- A's causal tiles, T
  for (int job = w; job < 10; job += WYB_THREADS / 64) {
    int tt, st;
    causal_tile(job, tt, st);
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      acc = mfma(row8<LT>(Kb, 16 * tt + lc, 32 * kb), row8<LT>(Kb, 16 * st + lc, 32 * kb), acc);
    const int s = 16 * st + lc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j;
      acc[j] = s < t ? bet[t] * acc[j] * expf(lgam[t] - lgam[s]) : 0.f;
    }
    st_tile(As, LDC, 16 * tt, 16 * st, acc);
  }
  __syncthreads();
  tri_inverse<LDC>(As, Ts, Ts + C * LDC);
  {
    // T's split planes, and T itself for the later kernels
    const int r = threadIdx.x >> 3, c = (threadIdx.x & 7) * 8;
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(Ts + r * LDC + c);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(Ts + r * LDC + c + 4);
    bf16x4 h0, o0, h1, o1;
    split4(x0, h0, o0);
    split4(x1, h1, o1);
    *reinterpret_cast<bf16x8*>(Th + LP::off(r, c)) = cat8(h0, h1);
    *reinterpret_cast<bf16x8*>(Tl + LP::off(r, c)) = cat8(o0, o1);
    float* Tg = b.T + si * C * C + r * C + c;
    *reinterpret_cast<f32x4*>(Tg) = x0;
    *reinterpret_cast<f32x4*>(Tg + 4) = x1;
  }
  __syncthreads();  // region R is free: the S_i planes
  sr.store(Sh, Sl);
  __syncthreads();

  const int tt = w & 3, h = w >> 2;
  const int kbt = tt >> 1;  // T[t][s] = 0 for s > t: k-blocks 0 .. kbt
  // rows t of diag(beta)-, diag(beta gamma)-scaled T (k = s)
  Op<2> tb[2], tg[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const Op<2> x = prow<LP>(Th, Tl, 16 * tt + lc, 32 * kb);
    tb[kb] = scale_op(x, bet, 32 * kb);
    tg[kb] = scale_op(x, bg, 32 * kb);
  }
  // -W^T tiles [c][t] = -sum_s K[s][c] beta gamma_s T[t][s], packed: the
  // pair-order operand (k = c, free t) of X's W S^T term
  Op<2> wn[NKB];
#pragma unroll
  for (int kp = 0; kp < NKB; ++kp) {
    f32x4 a0 = zero4(), a1 = zero4();
    for (int kb = 0; kb <= kbt; ++kb) {
      a0 = mma<1, 2>(Op<1>{{col8<LT>(Kb, 32 * kb, 32 * kp)}}, tg[kb], a0);
      a1 = mma<1, 2>(Op<1>{{col8<LT>(Kb, 32 * kb, 32 * kp + 16)}}, tg[kb], a1);
    }
    wn[kp] = pack_tiles<2>(-a0, -a1);
  }
#pragma unroll 1
  for (int q = 0; q < NH; ++q) {
    const int rt = h * NH + q;
    // X = U - W S^T, U[t][r] = sum_s beta_s T[t][s] V[s][r]
    f32x4 x = zero4();
    for (int kb = 0; kb <= kbt; ++kb) x = mma<2, 1>(tb[kb], Op<1>{{col8<LT>(Vb, 32 * kb, 16 * rt)}}, x);
#pragma unroll
    for (int kp = 0; kp < NKB; ++kp) x = mma<2, 2>(wn[kp], prow_p<LT>(Sh, Sl, 16 * rt, 32 * kp), x);
    st_tile(b.X + tokbase, D, 16 * tt, 16 * rt, x);
    // Z = diag(beta) V - diag(beta gamma) K S^T
    f32x4 ks = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      ks = mma<1, 2>(Op<1>{{row8<LT>(Kb, 16 * tt + lc, 32 * kb)}}, prow<LT>(Sh, Sl, 16 * rt + lc, 32 * kb), ks);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j;
      ks[j] = bet[t] * (float)Vb[LT::off(t, 16 * rt + lc)] - bg[t] * ks[j];
    }
    st_tile(b.Z + tokbase, D, 16 * tt, 16 * rt, ks);
  }
  // dq1 = diag(gamma) dO S; dL/dgamma_t through diag(gamma) Q: sum_c (dO S)[t][c] q[t][c]
  float dgq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int q = 0; q < NH; ++q) {
    const int ct = h * NH + q;
    f32x4 y = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      y = mma<1, 2>(Op<1>{{row8<LT>(Ob, 16 * tt + lc, 32 * kb)}}, pcol<LT>(Sh, Sl, 32 * kb, 16 * ct), y);
    const int c = 16 * ct + lc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j;
      dgq[j] += y[j] * (float)qg[t * p.sq[2] + c];
      y[j] *= gam[t];
    }
    st_tile(b.dq1 + tokbase, D, 16 * tt, 16 * ct, y);
  }
  float* tp = b.tokp + si * TOKP;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float s = row16_sum(dgq[j]);
    if (lc == 0) tp[TP_GQ + h * C + 16 * tt + 4 * G + j] = s;
  }
}

template <int D>
struct WyKbLds {
  static constexpr int C = CB_C, TB = C * D * 2, CP = C * C * 2;
  static constexpr int K0 = 0, Q0 = TB, O0 = 2 * TB;
  static constexpr int SH0 = 3 * TB, SL0 = SH0 + 2 * D * D, MH0 = SL0 + 2 * D * D, ML0 = MH0 + CP;
  static constexpr int G0 = ML0 + CP, DA0 = G0 + 5 * C * 4;
  static constexpr int BYTES = DA0 + 8 * 4;
  static_assert(BYTES <= 160 * 1024, "WY backward LDS exceeds the 160 KiB of a CU");
};

template <int D>
__global__ void __launch_bounds__(WYB_THREADS) wy_kb(ChunkArgs p, WyBwd b) {
  using L = WyKbLds<D>;
  using LT = BSwz<D>;
  using LP = BSwz<CB_C>;
  constexpr int C = CB_C, NT = D / 16, NKB = D / 32, NH = NT / 2;
  extern __shared__ __align__(16) char smem[];
  bf16* Kb = reinterpret_cast<bf16*>(smem + L::K0);
  bf16* Qb = reinterpret_cast<bf16*>(smem + L::Q0);
  bf16* Ob = reinterpret_cast<bf16*>(smem + L::O0);
  bf16* Sh = reinterpret_cast<bf16*>(smem + L::SH0);
  bf16* Sl = reinterpret_cast<bf16*>(smem + L::SL0);
  bf16* Mh = reinterpret_cast<bf16*>(smem + L::MH0);
  bf16* Ml = reinterpret_cast<bf16*>(smem + L::ML0);
  float* bet = reinterpret_cast<float*>(smem + L::G0);
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;
  float* dap = reinterpret_cast<float*>(smem + L::DA0);

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D, mat = (int64_t)D * D;

  {
    // Sb's planes, and <Sb, S_i> from the same pieces of both
    TokRows<D, WYB_THREADS> tk, tq, to;
    SplitRows<D, D, WYB_THREADS> sb, sx;
    tk.load(p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], p.sk[2]);
    tq.load(p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2], p.sq[2]);
    to.load(b.dO + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2], p.so[2]);
    sb.load(b.Sb + si * mat, D);
    sx.load(b.S_all + si * mat, D);
    tk.store(Kb);
    tq.store(Qb);
    to.store(Ob);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < sb.PER; ++q) acc += dot4(sx.x[q][0], sb.x[q][0]) + dot4(sx.x[q][1], sb.x[q][1]);
    sb.store(Sh, Sl);
    acc = wave_sum(acc);
    if (l == 0) dap[w] = acc;
  }
  for (int e = threadIdx.x; e < 2 * L::CP / 16; e += WYB_THREADS) reinterpret_cast<f32x4*>(Mh)[e] = zero4();
  if (w == 0) wy_gates(p.beta, p.g, bh * p.T + t0 + l, bet, gam, bg, kd, lgam);
  __syncthreads();
  // ---- M's causal tiles (split planes, rows t) and dM = lower_incl(dO X^T) (to the workspace)
  for (int job = w; job < 20; job += WYB_THREADS / 64) {
    int tt, st;
    causal_tile(job % 10, tt, st);
    if (job < 10) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        acc = mfma(row8<LT>(Kb, 16 * st + lc, 32 * kb), row8<LT>(Qb, 16 * tt + lc, 32 * kb), acc);
      const int t = 16 * tt + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = 16 * st + 4 * G + j;
        acc[j] = s <= t ? acc[j] * expf(lgam[t] - lgam[s]) : 0.f;
      }
      bf16x4 h, o;
      split4(acc, h, o);
      *reinterpret_cast<bf16x4*>(Mh + LP::off(t, 16 * st + 4 * G)) = h;
      *reinterpret_cast<bf16x4*>(Ml + LP::off(t, 16 * st + 4 * G)) = o;
    } else {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        acc = mma<1, 2>(Op<1>{{row8<LT>(Ob, 16 * tt + lc, 32 * kb)}}, gl_row_op(b.X + tokbase, D, 16 * st, 32 * kb),
                        acc);
      const int s = 16 * st + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (s > 16 * tt + 4 * G + j) acc[j] = 0.f;
      st_tile(b.dM + si * C * C, C, 16 * tt, 16 * st, acc);
    }
  }
  __syncthreads();
  const int tt = w & 3, h = w >> 2;
  // dX = M^T dO + diag(kd) K Sb^T  (M^T[t][s] = M[s][t] = 0 for s < t)
#pragma unroll 1
  for (int q = 0; q < NH; ++q) {
    const int rt = h * NH + q;
    f32x4 m = zero4(), ks = zero4();
    for (int kb = tt >> 1; kb < 2; ++kb)
      m = mma<2, 1>(pcol<LP>(Mh, Ml, 32 * kb, 16 * tt), Op<1>{{col8<LT>(Ob, 32 * kb, 16 * rt)}}, m);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      ks = mma<1, 2>(Op<1>{{row8<LT>(Kb, 16 * tt + lc, 32 * kb)}}, prow<LT>(Sh, Sl, 16 * rt + lc, 32 * kb), ks);
#pragma unroll
    for (int j = 0; j < 4; ++j) m[j] += kd[16 * tt + 4 * G + j] * ks[j];
    st_tile(b.dX + tokbase, D, 16 * tt, 16 * rt, m);
  }
  // dk2 = diag(kd) X Sb; dL/dkd_t = sum_c (X Sb)[t][c] K[t][c]
  Op<2> xo[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) xo[kb] = gl_row_op(b.X + tokbase, D, 16 * tt, 32 * kb);
  float dkd[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
  for (int q = 0; q < NH; ++q) {
    const int ct = h * NH + q;
    f32x4 y = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) y = mma<2, 2>(xo[kb], pcol<LT>(Sh, Sl, 32 * kb, 16 * ct), y);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j;
      dkd[j] += y[j] * (float)Kb[LT::off(t, 16 * ct + lc)];
      y[j] *= kd[t];
    }
    st_tile(b.dk2 + tokbase, D, 16 * tt, 16 * ct, y);
  }
  float* tp = b.tokp + si * TOKP;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float s = row16_sum(dkd[j]);
    if (lc == 0) tp[TP_KD + h * C + 16 * tt + 4 * G + j] = s;
  }
  if (threadIdx.x == 0)
    tp[TP_DA] = ((dap[0] + dap[1]) + (dap[2] + dap[3])) + ((dap[4] + dap[5]) + (dap[6] + dap[7]));
}

template <int D>
struct WyKc1Lds {
  static constexpr int C = CB_C, TB = C * D * 2, CP = C * C * 2;
  static constexpr int SH0 = 0, SL0 = 2 * D * D, TH0 = 4 * D * D, TL0 = TH0 + CP, XH0 = TL0 + CP, XL0 = XH0 + TB;
  static constexpr int G0 = XL0 + TB;
  static constexpr int BYTES = G0 + 5 * C * 4;
  static_assert(BYTES <= 160 * 1024, "WY backward LDS exceeds the 160 KiB of a CU");
};

template <int D>
__global__ void __launch_bounds__(WYB_THREADS) wy_kc1(ChunkArgs p, WyBwd b) {
  using L = WyKc1Lds<D>;
  using LT = BSwz<D>;
  using LP = BSwz<CB_C>;
  constexpr int C = CB_C, NT = D / 16, NKB = D / 32, NH = NT / 2;
  extern __shared__ __align__(16) char smem[];
  bf16* Sh = reinterpret_cast<bf16*>(smem + L::SH0);
  bf16* Sl = reinterpret_cast<bf16*>(smem + L::SL0);
  bf16* Th = reinterpret_cast<bf16*>(smem + L::TH0);
  bf16* Tl = reinterpret_cast<bf16*>(smem + L::TL0);
  bf16* Xh = reinterpret_cast<bf16*>(smem + L::XH0);  // dX planes (rows t)
  bf16* Xl = reinterpret_cast<bf16*>(smem + L::XL0);
  float* bet = reinterpret_cast<float*>(smem + L::G0);
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D;
  const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2];
  const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2];

  {
    SplitRows<D, D, WYB_THREADS> ss;
    SplitRows<C, C, WYB_THREADS> st;
    SplitRows<D, C, WYB_THREADS> sx;
    ss.load(b.S_all + si * (int64_t)D * D, D);
    st.load(b.T + si * C * C, C);
    sx.load(b.dX + tokbase, D);
    ss.store(Sh, Sl);
    st.store(Th, Tl);
    sx.store(Xh, Xl);
  }
  if (w == 0) wy_gates(p.beta, p.g, bh * p.T + t0 + l, bet, gam, bg, kd, lgam);
  __syncthreads();
  const int tt = w & 3, h = w >> 2;
  const int kbt = tt >> 1;  // T[s][t] = 0 for s < t: k-blocks kbt .. 1
  // R^T tiles [r][t] = sum_s dX[s][r] T[s][t], packed: the pair-order operand (k = r, free t) of R S
  Op<2> ro[NKB];
#pragma unroll
  for (int kp = 0; kp < NKB; ++kp) {
    f32x4 a0 = zero4(), a1 = zero4();
    for (int kb = kbt; kb < 2; ++kb) {
      const Op<2> tb = pcol_p<LP>(Th, Tl, 32 * kb, 16 * tt);
      a0 = mma<2, 2>(pcol_p<LT>(Xh, Xl, 32 * kb, 32 * kp), tb, a0);
      a1 = mma<2, 2>(pcol_p<LT>(Xh, Xl, 32 * kb, 32 * kp + 16), tb, a1);
    }
    ro[kp] = pack_tiles<2>(a0, a1);
  }
  float sbg[4] = {0.f, 0.f, 0.f, 0.f}, sb[4] = {0.f, 0.f, 0.f, 0.f};
  bf16* dvg = b.dv + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2];
#pragma unroll 1
  for (int q = 0; q < NH; ++q) {
    const int ct = h * NH + q;
    const int c = 16 * ct + lc;
    // dk2 -= diag(beta gamma) R S;  dL/d(beta gamma)_t through W: -sum_c (R S)[t][c] K[t][c]
    f32x4 rs = zero4();
#pragma unroll
    for (int kp = 0; kp < NKB; ++kp) rs = mma<2, 2>(ro[kp], pcol_p<LT>(Sh, Sl, 32 * kp, 16 * ct), rs);
    f32x4 dk = ld_tile(b.dk2 + tokbase, D, 16 * tt, 16 * ct);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j;
      sbg[j] -= rs[j] * (float)kg[t * p.sk[2] + c];
      dk[j] -= bg[t] * rs[j];
    }
    st_tile(b.dk2 + tokbase, D, 16 * tt, 16 * ct, dk);
    // R = T^T dX: dv = diag(beta) R, dL/dbeta_t through U: sum_r R[t][r] V[t][r]
    f32x4 rr = zero4();
    for (int kb = kbt; kb < 2; ++kb)
      rr = mma<2, 2>(pcol<LP>(Th, Tl, 32 * kb, 16 * tt), pcol<LT>(Xh, Xl, 32 * kb, 16 * ct), rr);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j;
      sb[j] += rr[j] * (float)vg[t * p.sv[2] + c];
      dvg[t * p.sv[2] + c] = (bf16)(bet[t] * rr[j]);
    }
  }
  float* tp = b.tokp + si * TOKP;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float s1 = row16_sum(sbg[j]), s2 = row16_sum(sb[j]);
    if (lc == 0) {
      tp[TP_SBG + h * C + 16 * tt + 4 * G + j] = s1;
      tp[TP_SB + h * C + 16 * tt + 4 * G + j] = s2;
    }
  }
  // dT = dX Z^T, the causal tiles (the strictly upper part of dT does not reach dA)
  for (int job = w; job < 10; job += WYB_THREADS / 64) {
    int at, st;
    causal_tile(job, at, st);
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      acc = mma<2, 2>(prow<LT>(Xh, Xl, 16 * at + lc, 32 * kb), gl_row_op(b.Z + tokbase, D, 16 * st, 32 * kb), acc);
    st_tile(b.dT + si * C * C, C, 16 * at, 16 * st, acc);
  }
}

template <int D>
struct WyKc2Lds {
  static constexpr int C = CB_C, TB = C * D * 2, CP = C * C * 2;
  static constexpr int Q0 = 0, K0 = TB;
  // split planes: T, dT, Y (rows t), H = G_A^T and DG^T (rows s)
  static constexpr int TH0 = 2 * TB, DT0 = TH0 + 2 * CP, Y0 = DT0 + 2 * CP, H0 = Y0 + 2 * CP, DG0 = H0 + 2 * CP;
  static constexpr int G0 = DG0 + 2 * CP;
  // per causal tile: row sums of E and of the A term of dbeta, column sums of E (16 each)
  static constexpr int P0 = G0 + 5 * C * 4;
  static constexpr int BYTES = P0 + 3 * 10 * 16 * 4;
  static_assert(BYTES <= 160 * 1024, "WY backward LDS exceeds the 160 KiB of a CU");
};

template <int D>
__global__ void __launch_bounds__(WYB_THREADS) wy_kc2(ChunkArgs p, WyBwd b) {
  using L = WyKc2Lds<D>;
  using LT = BSwz<D>;
  using LP = BSwz<CB_C>;
  constexpr int C = CB_C, NT = D / 16, NKB = D / 32, NH = NT / 2, CP = L::CP / 2;  // CP: bf16 per plane
  extern __shared__ __align__(16) char smem[];
  bf16* Qb = reinterpret_cast<bf16*>(smem + L::Q0);
  bf16* Kb = reinterpret_cast<bf16*>(smem + L::K0);
  bf16* Th = reinterpret_cast<bf16*>(smem + L::TH0);
  bf16* Tl = Th + CP;
  bf16* Dh = reinterpret_cast<bf16*>(smem + L::DT0);
  bf16* Dl = Dh + CP;
  bf16* Yh = reinterpret_cast<bf16*>(smem + L::Y0);
  bf16* Yl = Yh + CP;
  bf16* Hh = reinterpret_cast<bf16*>(smem + L::H0);
  bf16* Hl = Hh + CP;
  bf16* Gh = reinterpret_cast<bf16*>(smem + L::DG0);
  bf16* Gl = Gh + CP;
  float* bet = reinterpret_cast<float*>(smem + L::G0);
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;
  float* rowP = reinterpret_cast<float*>(smem + L::P0);  // [10][16]
  float* bsP = rowP + 160;                               // [10][16]
  float* colP = bsP + 160;                               // [10][16]

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D;
  {
    // dT's planes with its strictly upper part (not written) as zeros; H and DG^T zeroed
    TokRows<D, WYB_THREADS> tq, tk;
    SplitRows<C, C, WYB_THREADS> st, sd;
    tq.load(p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2], p.sq[2]);
    tk.load(p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], p.sk[2]);
    st.load(b.T + si * C * C, C);
    sd.load(b.dT + si * C * C, C);
    tq.store(Qb);
    tk.store(Kb);
    st.store(Th, Tl);
    sd.lower();
    sd.store(Dh, Dl);
  }
  for (int e = threadIdx.x; e < 4 * L::CP / 16; e += WYB_THREADS) reinterpret_cast<f32x4*>(Hh)[e] = zero4();
  float graw = 0.f;
  if (w == 0) {
    graw = p.g[bh * p.T + t0 + l];
    wy_gates(p.beta, p.g, bh * p.T + t0 + l, bet, gam, bg, kd, lgam);
  }
  __syncthreads();
  // ---- Y = dT T^T as planes of rows t: tiles Y^T[u][t] = sum_s T[u][s] dT[t][s], stored transposed
  for (int tile = w; tile < 16; tile += WYB_THREADS / 64) {
    const int ut = tile >> 2, tt = tile & 3;
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
      acc = mma<2, 2>(prow<LP>(Th, Tl, 16 * ut + lc, 32 * kb), prow<LP>(Dh, Dl, 16 * tt + lc, 32 * kb), acc);
    bf16x4 h, o;
    split4(acc, h, o);
    *reinterpret_cast<bf16x4*>(Yh + LP::off(16 * tt + lc, 16 * ut + 4 * G)) = h;
    *reinterpret_cast<bf16x4*>(Yl + LP::off(16 * tt + lc, 16 * ut + 4 * G)) = o;
  }
  __syncthreads();
  // ---- causal tiles [t][s]: dA = strict_lower(-T^T Y), G_A = dA beta_t Gamma, DG = dM Gamma,
  //      E = dGamma * Gamma = (dA beta_t (K K^T) + dM (Q K^T)) Gamma, the A term of dbeta
  for (int job = w; job < 10; job += WYB_THREADS / 64) {
    int tt, st;
    causal_tile(job, tt, st);
    f32x4 ta = zero4(), kk = zero4(), qk = zero4();
    for (int kb = tt >> 1; kb < 2; ++kb)
      ta = mma<2, 2>(pcol<LP>(Th, Tl, 32 * kb, 16 * tt), pcol<LP>(Yh, Yl, 32 * kb, 16 * st), ta);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const bf16x8 ks = row8<LT>(Kb, 16 * st + lc, 32 * kb);
      kk = mfma(row8<LT>(Kb, 16 * tt + lc, 32 * kb), ks, kk);
      qk = mfma(row8<LT>(Qb, 16 * tt + lc, 32 * kb), ks, qk);
    }
    const int s = 16 * st + lc;
    const f32x4 dmt = ld_tile(b.dM + si * C * C, C, 16 * tt, 16 * st);
    f32x4 ga, dg;
    float rs[4], bs[4], cs = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j;
      const float e = s <= t ? expf(lgam[t] - lgam[s]) : 0.f;
      const float da = s < t ? -ta[j] : 0.f;
      const float dm = s <= t ? dmt[j] : 0.f;
      ga[j] = da * bet[t] * e;
      dg[j] = dm * e;
      bs[j] = da * kk[j] * e;
      const float E = (da * bet[t] * kk[j] + dm * qk[j]) * e;
      rs[j] = E;
      cs += E;
    }
    // H = G_A^T and DG^T as planes of rows s
    bf16x4 h, o;
    split4(ga, h, o);
    *reinterpret_cast<bf16x4*>(Hh + LP::off(s, 16 * tt + 4 * G)) = h;
    *reinterpret_cast<bf16x4*>(Hl + LP::off(s, 16 * tt + 4 * G)) = o;
    split4(dg, h, o);
    *reinterpret_cast<bf16x4*>(Gh + LP::off(s, 16 * tt + 4 * G)) = h;
    *reinterpret_cast<bf16x4*>(Gl + LP::off(s, 16 * tt + 4 * G)) = o;
    cs = group_sum(cs);
    if (G == 0) colP[job * 16 + lc] = cs;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float r1 = row16_sum(rs[j]), r2 = row16_sum(bs[j]);
      if (lc == 0) {
        rowP[job * 16 + 4 * G + j] = r1;
        bsP[job * 16 + 4 * G + j] = r2;
      }
    }
  }
  __syncthreads();
  // ---- dk = dk2 + G_A K + G_A^T K + DG^T Q,  dq = dq1 + DG K
  const int tt = w & 3, h = w >> 2;
  bf16* dqg = b.dq + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2];
  bf16* dkg = b.dk + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2];
#pragma unroll 1
  for (int q = 0; q < NH; ++q) {
    const int ct = h * NH + q;
    f32x4 dk = ld_tile(b.dk2 + tokbase, D, 16 * tt, 16 * ct);
    f32x4 dq = ld_tile(b.dq1 + tokbase, D, 16 * tt, 16 * ct);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const Op<1> kc{{col8<LT>(Kb, 32 * kb, 16 * ct)}};
      dk = mma<2, 1>(pcol<LP>(Hh, Hl, 32 * kb, 16 * tt), kc, dk);                // G_A[t][s] = H[s][t]
      dk = mma<2, 1>(prow<LP>(Hh, Hl, 16 * tt + lc, 32 * kb), kc, dk);           // G_A[s][t] = H[t][s]
      dk = mma<2, 1>(prow<LP>(Gh, Gl, 16 * tt + lc, 32 * kb), Op<1>{{col8<LT>(Qb, 32 * kb, 16 * ct)}}, dk);
      dq = mma<2, 1>(pcol<LP>(Gh, Gl, 32 * kb, 16 * tt), kc, dq);                // DG[t][s] = DG^T[s][t]
    }
    const int c = 16 * ct + lc;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = 16 * tt + 4 * G + j;
      dkg[t * p.sk[2] + c] = (bf16)dk[j];
      dqg[t * p.sq[2] + c] = (bf16)dq[j];
    }
  }
  // ---- gate gradients (wave 0, lane = token)
  if (w == 0) {
    const float* tp = b.tokp + si * TOKP;
    const float sbg = tp[TP_SBG + l] + tp[TP_SBG + C + l];
    const float dgm = (tp[TP_GQ + l] + tp[TP_GQ + C + l]) + bet[l] * sbg;  // dL/dgamma_t
    const float dkdv = tp[TP_KD + l] + tp[TP_KD + C + l];                   // dL/dkd_t
    const float dbu = (tp[TP_SB + l] + tp[TP_SB + C + l]) + gam[l] * sbg;   // dL/dbeta_t from U and W
    const float dgC = tp[TP_DA];                                            // dL/dgamma_C = <Sb, S_i>
    // row and column sums of E over the causal tiles of this token, in a fixed order
    const int tl = l >> 4, lr = l & 15;
    float rowE = 0.f, bsum = 0.f, colE = 0.f;
    for (int st = 0; st <= tl; ++st) {
      const int job = tl * (tl + 1) / 2 + st;
      rowE += rowP[job * 16 + lr];
      bsum += bsP[job * 16 + lr];
    }
    for (int tt2 = tl; tt2 < 4; ++tt2) colE += colP[(tt2 * (tt2 + 1) / 2 + tl) * 16 + lr];
    // dgc_t: gamma_t = exp(gc_t), kd_t = exp(gc_{C-1} - gc_t), the Gamma
    // exponents (row minus column sums), and gamma_{C-1} = a of the scan
    float dgc = dgm * gam[l] - dkdv * kd[l] + rowE - colE;
    const float kdsum = wave_sum(dkdv * kd[l]);
    if (l == C - 1) dgc += kdsum + dgC * gam[l];
    // dlg_u = sum_{t >= u} dgc_t
    const float dlg = wave_sum(dgc) - (wave_incl_scan(dgc) - dgc);
    const int64_t o = bh * p.T + t0 + l;
    b.dg[o] = graw >= LOG_FLOOR ? dlg : 0.f;
    b.dbeta[o] = dbu + bsum;
  }
}

template <int D>
size_t ckpt_floats(int64_t B, int64_t H, int64_t T) {
  const int64_t chunks = B * H * (T / CB_C), mat = (int64_t)D * D, tok = B * H * T * (int64_t)D;
  return (size_t)(3 * chunks * mat + 2 * tok + chunks);
}

struct Ckpt {
  float *UA, *KA, *S_all, *Qt, *Ov, *av;
};
Ckpt ckpt_of(float* ws, int64_t B, int64_t H, int64_t T, int d) {
  const int64_t chunks = B * H * (T / CB_C), mat = (int64_t)d * d, tok = B * H * T * (int64_t)d;
  Ckpt c;
  c.UA = ws;
  c.KA = c.UA + chunks * mat;
  c.S_all = c.KA + chunks * mat;
  c.Qt = c.S_all + chunks * mat;
  c.Ov = c.Qt + tok;
  c.av = c.Ov + tok;
  return c;
}

template <class K>
hipError_t launch_k(K kern, int threads, int bytes, int64_t grid, hipStream_t s, const ChunkArgs& a, const WyBwd& b) {
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(threads), bytes, s, a, b);
  return hipGetLastError();
}

template <int D>
hipError_t launch_wy(const ChunkArgs& a, float* ws, hipStream_t s) {
  const int64_t chunks = a.B * a.H * a.N;
  const Ckpt c = ckpt_of(ws, a.B, a.H, a.T, D);
  auto kp = wy_prep<D>;
  auto ko = wy_out<D>;
  const int lp = WyPrepLds<D>::BYTES, lo = 2 * D * D * 2;
  hipError_t e = hipFuncSetAttribute((const void*)kp, hipFuncAttributeMaxDynamicSharedMemorySize, lp);
  if (e == hipSuccess) e = hipFuncSetAttribute((const void*)ko, hipFuncAttributeMaxDynamicSharedMemorySize, lo);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kp, dim3((unsigned)chunks), dim3(WYP_THREADS), lp, s, a, c.UA, c.KA, c.Qt, c.Ov, c.av);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  ScanArgs sa{};
  sa.U = c.UA;
  sa.K = c.KA;
  sa.a = c.av;
  sa.S_all = c.S_all;
  sa.BH = a.B * a.H;
  sa.N = a.N;
  sa.dh = D;
  sa.rule = 0;
  sa.ns = 0;
  // split-bf16 state products (about 2^-16 relative error each, far below
  // the bf16 output's rounding): the 8-wave delta scan kernel
  sa.precision = GMDN_PREC_TF32;
  sa.stream = s;
  if ((e = scan_fwd_rows_launch(sa)) != hipSuccess) return e;
  hipLaunchKernelGGL(ko, dim3((unsigned)chunks), dim3(WY_THREADS), lo, s, a, (const float*)c.Qt, (const float*)c.Ov,
                     (const float*)c.S_all);
  return hipGetLastError();
}

// backward workspace (floats): gS, Sb (d x d per chunk); T, dM, dT (C x C
// per chunk); X, Z, dX, dq1, dk2 (B H T d each); the per-chunk tokp records
size_t bwd_floats(int64_t B, int64_t H, int64_t T, int d) {
  const int64_t chunks = B * H * (T / CB_C), mat = (int64_t)d * d, tok = B * H * T * (int64_t)d;
  return (size_t)(2 * chunks * mat + 3 * chunks * CB_C * CB_C + 5 * tok + chunks * TOKP);
}

template <int D>
hipError_t launch_wy_bwd(const ChunkArgs& a, float* ckpt, const void* dO, void* dq, void* dk, void* dv, float* dbeta,
                         float* dg, float* ws, hipStream_t s) {
  const int64_t chunks = a.B * a.H * a.N, mat = (int64_t)D * D, tok = a.B * a.H * a.T * (int64_t)D;
  const int64_t cc = (int64_t)CB_C * CB_C;
  const Ckpt c = ckpt_of(ckpt, a.B, a.H, a.T, D);
  WyBwd b{};
  b.UA = c.UA;
  b.KA = c.KA;
  b.S_all = c.S_all;
  b.Qt = c.Qt;
  b.av = c.av;
  b.dO = static_cast<const bf16*>(dO);
  b.gS = ws;
  float* Sb = ws + chunks * mat;
  b.Sb = Sb;
  b.T = Sb + chunks * mat;
  b.dM = b.T + chunks * cc;
  b.dT = b.dM + chunks * cc;
  b.X = b.dT + chunks * cc;
  b.Z = b.X + tok;
  b.dX = b.Z + tok;
  b.dq1 = b.dX + tok;
  b.dk2 = b.dq1 + tok;
  b.tokp = b.dk2 + tok;
  b.dq = static_cast<bf16*>(dq);
  b.dk = static_cast<bf16*>(dk);
  b.dv = static_cast<bf16*>(dv);
  b.dbeta = dbeta;
  b.dg = dg;
  hipError_t e = launch_k(wy_gs<D>, WY_THREADS, 3 * CB_C * D * 2, chunks, s, a, b);
  if (e != hipSuccess) return e;
  // the delta scan's reverse kernel: dU_i = dL/dS_{i+1} (its dK and da are not needed)
  ScanArgs sa{};
  sa.U = c.UA;
  sa.K = c.KA;
  sa.a = c.av;
  sa.S_all = c.S_all;
  sa.gS = b.gS;
  sa.dU = Sb;
  sa.BH = a.B * a.H;
  sa.N = a.N;
  sa.dh = D;
  sa.rule = 0;
  sa.ns = 0;
  sa.precision = GMDN_PREC_TF32;
  sa.stream = s;
  if ((e = scan_bwd_rows_launch(sa, nullptr)) != hipSuccess) return e;
  if ((e = launch_k(wy_ka<D>, WYB_THREADS, WyKaLds<D>::BYTES, chunks, s, a, b)) != hipSuccess) return e;
  if ((e = launch_k(wy_kb<D>, WYB_THREADS, WyKbLds<D>::BYTES, chunks, s, a, b)) != hipSuccess) return e;
  if ((e = launch_k(wy_kc1<D>, WYB_THREADS, WyKc1Lds<D>::BYTES, chunks, s, a, b)) != hipSuccess) return e;
  return launch_k(wy_kc2<D>, WYB_THREADS, WyKc2Lds<D>::BYTES, chunks, s, a, b);
}

}  // namespace

size_t wy_workspace_floats(int64_t B, int64_t H, int64_t T, int d) {
  return d == 128 ? ckpt_floats<128>(B, H, T) : ckpt_floats<64>(B, H, T);
}

hipError_t wy_fwd_launch(const ChunkArgs& a, int d, float* ws, hipStream_t s) {
  if (d == 128) return launch_wy<128>(a, ws, s);
  if (d == 64) return launch_wy<64>(a, ws, s);
  return hipErrorInvalidValue;
}

size_t wy_bwd_workspace_floats(int64_t B, int64_t H, int64_t T, int d) { return bwd_floats(B, H, T, d); }

hipError_t wy_bwd_launch(const ChunkArgs& a, int d, float* ckpt, const void* dO, void* dq, void* dk, void* dv,
                         float* dbeta, float* dg, float* ws, hipStream_t s) {
  if (d == 128) return launch_wy_bwd<128>(a, ckpt, dO, dq, dk, dv, dbeta, dg, ws, s);
  if (d == 64) return launch_wy_bwd<64>(a, ckpt, dO, dq, dk, dv, dbeta, dg, ws, s);
  return hipErrorInvalidValue;
}

}  // namespace gmdn
