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
  for (int e = threadIdx.x; e < C * D / 8; e += WYP_THREADS) {
    const int t = e / (D / 8), c = (e % (D / 8)) * 8;
    *reinterpret_cast<bf16x8*>(Kb + LT::off(t, c)) = *reinterpret_cast<const bf16x8*>(kg + t * p.sk[2] + c);
    *reinterpret_cast<bf16x8*>(Qb + LT::off(t, c)) = *reinterpret_cast<const bf16x8*>(qg + t * p.sq[2] + c);
    *reinterpret_cast<bf16x8*>(Vb + LT::off(t, c)) = *reinterpret_cast<const bf16x8*>(vg + t * p.sv[2] + c);
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
  for (int e = threadIdx.x; e < D * D / 8; e += WY_THREADS) {
    const int r = e / (D / 8), c = (e % (D / 8)) * 8;
    bf16x4 h0, o0, h1, o1;
    split4(*reinterpret_cast<const f32x4*>(S + (int64_t)r * D + c), h0, o0);
    split4(*reinterpret_cast<const f32x4*>(S + (int64_t)r * D + c + 4), h1, o1);
    *reinterpret_cast<bf16x8*>(Sh + LS::off(r, c)) = cat8(h0, h1);
    *reinterpret_cast<bf16x8*>(Sl + LS::off(r, c)) = cat8(o0, o1);
  }
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
struct WyBwd {
  const float *UA, *KA, *S_all, *Qt, *av;  // forward checkpoint
  const bf16* dO;                         // strides so
  float* gS;                              // wy_gs output
  const float* Sb;                        // the reverse scan's dU (= dL/dS_{i+1})
  float *dQp, *dKp;                       // partial dq, dk (B H T d, float32)
  float *Tp, *dTp, *dMp;                  // T, dT, dM per chunk (C x C, float32)
  float* tokp;                            // per chunk: dgamma, dkd, dbeta partials (3 x C) and da
  bf16 *dq, *dk, *dv;
  float *dbeta, *dg;
};

// gS[r][c] = sum_t dO[t][r] Qt[t][c]
template <int D>
__global__ void __launch_bounds__(WY_THREADS) wy_gs(ChunkArgs p, WyBwd b) {
  constexpr int C = CB_C, LDT = D + 4, NT = D / 16;
  extern __shared__ __align__(16) float sm[];
  float* Os = sm;
  float* Qs = sm + C * LDT;
  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id();
  const bf16* og = b.dO + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2];
  const float* qt = b.Qt + (bh * p.T + t0) * (int64_t)D;
  for (int e = threadIdx.x; e < C * D / 8; e += WY_THREADS) {
    const int t = e / (D / 8), c = (e % (D / 8)) * 8;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(og + t * p.so[2] + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) Os[t * LDT + c + j] = (float)x[j];
    *reinterpret_cast<f32x4*>(Qs + t * LDT + c) = *reinterpret_cast<const f32x4*>(qt + (int64_t)t * D + c);
    *reinterpret_cast<f32x4*>(Qs + t * LDT + c + 4) = *reinterpret_cast<const f32x4*>(qt + (int64_t)t * D + c + 4);
  }
  __syncthreads();
  float* gS = b.gS + si * (int64_t)D * D;
  for (int tile = w; tile < NT * NT; tile += 4) {
    const int tr = tile / NT, tc = tile % NT;
    const f32x4 acc = mm16<C>([&](int r, int k) { return Os[k * LDT + 16 * tr + r]; },
                              [&](int k, int c) { return Qs[k * LDT + 16 * tc + c]; }, zero4());
    st_tile(gS, D, 16 * tr, 16 * tc, acc);
  }
}

template <int D>
struct WyBwdLds {
  static constexpr int C = CB_C;
  static constexpr int LDB = D + 8;        // bf16 stride of a token tile row
  static constexpr int LDT = D + 4;        // float stride of a token tile row
  static constexpr int LDC = C + 4;        // float stride of a C x C matrix row
  static constexpr int BT = C * LDB * 2;   // bytes: bf16 token tile
  static constexpr int FT = C * LDT * 4;   // bytes: float token tile
  static constexpr int CC = C * LDC * 4;   // bytes: float C x C matrix
  // wy_tok1: K, V, dO (bf16); F1: Q (bf16) in steps 0-1, then W / X / dW rows;
  // F2: A in steps 1-2, then dX rows; T; M; then small float arrays
  static constexpr int K0 = 0, V0 = BT, O0 = 2 * BT, F1 = 3 * BT, F2 = F1 + FT, T0 = F2 + FT, M0 = T0 + CC;
  static constexpr int R0 = M0 + CC;
  static constexpr int SMALL1 = 5 * C + 3 * 256 + 4;  // gates, tri_inverse scratch, per-wave <Sb, S_i>
  static constexpr int TOK1_BYTES = R0 + SMALL1 * 4;
  // wy_tok2: Q, K (bf16); T, dT, dM, Y = dT T^T, G_A, dM * Gamma; small arrays
  static constexpr int Q2 = 0, K2 = BT, T2 = 2 * BT, DT2 = T2 + CC, DM2 = DT2 + CC, Y2 = DM2 + CC,
                       GA2 = Y2 + CC, DG2 = GA2 + CC, R2 = DG2 + CC;
  static constexpr int SMALL2 = 5 * C + 2 * C + 4 * C;  // gates, rowE, colE
  static constexpr int TOK2_BYTES = R2 + SMALL2 * 4;
  static_assert(TOK1_BYTES <= 160 * 1024 && TOK2_BYTES <= 160 * 1024, "WY backward LDS exceeds 160 KiB");
  static_assert(BT <= FT && CC <= FT, "Q and A fit the slots they borrow");
};

template <int LDB>
GMDN_DEV float bfx(const bf16* X, int r, int c) { return (float)X[r * LDB + c]; }

template <int D>
GMDN_DEV void load_bf16_rows(bf16* dst, const bf16* src, int64_t stride) {
  constexpr int LDB = D + 8;
  for (int e = threadIdx.x; e < CB_C * D / 8; e += WY_THREADS) {
    const int t = e / (D / 8), c = (e % (D / 8)) * 8;
    *reinterpret_cast<bf16x8*>(dst + t * LDB + c) = *reinterpret_cast<const bf16x8*>(src + t * stride + c);
  }
}

template <int D>
__global__ void __launch_bounds__(WY_THREADS) wy_tok1(ChunkArgs p, WyBwd b) {
  using L = WyBwdLds<D>;
  constexpr int C = CB_C, LDB = L::LDB, LDT = L::LDT, LDC = L::LDC, NT = D / 16;
  extern __shared__ __align__(16) char smem[];
  bf16* Ks = reinterpret_cast<bf16*>(smem + L::K0);
  bf16* Vs = reinterpret_cast<bf16*>(smem + L::V0);
  bf16* Os = reinterpret_cast<bf16*>(smem + L::O0);
  bf16* Qs = reinterpret_cast<bf16*>(smem + L::F1);
  float* F1 = reinterpret_cast<float*>(smem + L::F1);
  float* As = reinterpret_cast<float*>(smem + L::F2);
  float* F2 = reinterpret_cast<float*>(smem + L::F2);
  float* Ts = reinterpret_cast<float*>(smem + L::T0);
  float* Ms = reinterpret_cast<float*>(smem + L::M0);
  float* bet = reinterpret_cast<float*>(smem + L::R0);
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;
  float* Xw = lgam + C;      // 3 x 256
  float* pda = Xw + 768;     // per wave: partial <Sb, S_i>

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int r0 = 16 * w;  // this wave's token rows
  const int64_t mat = (int64_t)D * D;
  const float* S = b.S_all + si * mat;
  const float* Sb = b.Sb + si * mat;
  const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2];

  // ---- step 0: tiles, gates, zeroed T
  load_bf16_rows<D>(Qs, qg, p.sq[2]);
  load_bf16_rows<D>(Ks, p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], p.sk[2]);
  load_bf16_rows<D>(Vs, p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2], p.sv[2]);
  load_bf16_rows<D>(Os, b.dO + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2], p.so[2]);
  for (int e = threadIdx.x; e < C * LDC; e += WY_THREADS) Ts[e] = 0.f;
  if (w == 0) wy_gates(p.beta, p.g, bh * p.T + t0 + l, bet, gam, bg, kd, lgam);
  __syncthreads();
  auto kb = [&](int r, int c) { return bfx<LDB>(Ks, r, c); };

  // ---- step 1: rows of A and M
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    f32x4 a = zero4(), m = zero4();
    if (st <= w) {
      const f32x4 kk = mm16<D>([&](int r, int k) { return kb(r0 + r, k); },
                               [&](int k, int c) { return kb(16 * st + c, k); }, zero4());
      const f32x4 qk = mm16<D>([&](int r, int k) { return bfx<LDB>(Qs, r0 + r, k); },
                               [&](int k, int c) { return kb(16 * st + c, k); }, zero4());
      const int s = 16 * st + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = r0 + 4 * G + j;
        const float e = s <= t ? expf(lgam[t] - lgam[s]) : 0.f;
        a[j] = s < t ? bet[t] * kk[j] * e : 0.f;
        m[j] = qk[j] * e;
      }
    }
    st_tile(As, LDC, r0, 16 * st, a);
    st_tile(Ms, LDC, r0, 16 * st, m);
  }
  __syncthreads();
  // ---- step 2: T = (I + A)^-1
  tri_inverse<LDC>(As, Ts, Xw);

  // ---- step 3: W, U and X = U - W S_i^T for this wave's rows (Q is dead: F1 holds W, then X)
  f32x4 X[NT];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    auto trow = [&](int r, int k) { return Ts[(r0 + r) * LDC + k]; };
    const f32x4 wt = mm16<C>(trow, [&](int k, int c) { return bg[k] * kb(k, 16 * tc + c); }, zero4());
    st_tile(F1, LDT, r0, 16 * tc, wt);
    X[tc] = mm16<C>(trow, [&](int k, int c) { return bet[k] * bfx<LDB>(Vs, k, 16 * tc + c); }, zero4());
  }
#pragma unroll
  for (int tc = 0; tc < NT; ++tc)
    X[tc] -= mm16<D>([&](int r, int k) { return F1[(r0 + r) * LDT + k]; },
                     [&](int k, int c) { return S[(int64_t)(16 * tc + c) * D + k]; }, zero4());
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) st_tile(F1, LDT, r0, 16 * tc, X[tc]);
  __syncthreads();  // X complete

  // ---- step 4: dM = lower_incl(dO X^T), dQt~ = dO S_i, dK~ = X Sb; <Sb, S_i>
  auto orow = [&](int r, int k) { return bfx<LDB>(Os, r0 + r, k); };
  f32x4 dM[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    dM[st] = zero4();
    if (st <= w) {
      dM[st] = mm16<D>(orow, [&](int k, int c) { return F1[(16 * st + c) * LDT + k]; }, zero4());
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (16 * st + lc > r0 + 4 * G + j) dM[st][j] = 0.f;
    }
  }
  float dgam[4] = {0.f, 0.f, 0.f, 0.f}, dkd[4] = {0.f, 0.f, 0.f, 0.f};
  float dbet[4] = {0.f, 0.f, 0.f, 0.f}, dbg[4] = {0.f, 0.f, 0.f, 0.f};
  float* dqp = b.dQp + (bh * p.T + t0) * (int64_t)D;
  float* dkp = b.dKp + (bh * p.T + t0) * (int64_t)D;
  f32x4 dK[NT];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    const f32x4 dqt = mm16<D>(orow, [&](int k, int c) { return S[(int64_t)k * D + 16 * tc + c]; }, zero4());
    const f32x4 dkt = mm16<D>([&](int r, int k) { return F1[(r0 + r) * LDT + k]; },
                              [&](int k, int c) { return Sb[(int64_t)k * D + 16 * tc + c]; }, zero4());
    f32x4 dq;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = r0 + 4 * G + j, c = 16 * tc + lc;
      dgam[j] += dqt[j] * (float)qg[(int64_t)t * p.sq[2] + c];
      dkd[j] += dkt[j] * kb(t, c);
      dq[j] = gam[t] * dqt[j];
      dK[tc][j] = kd[t] * dkt[j];
    }
    st_tile(dqp, D, r0, 16 * tc, dq);
  }
  {
    float acc = 0.f;
    for (int e = threadIdx.x; e < D * D / 4; e += WY_THREADS) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(S + 4 * (int64_t)e);
      const f32x4 y = *reinterpret_cast<const f32x4*>(Sb + 4 * (int64_t)e);
      acc += x[0] * y[0] + x[1] * y[1] + x[2] * y[2] + x[3] * y[3];
    }
    acc = wave_sum(acc);
    if (l == 0) pda[w] = acc;
  }

  // ---- step 5: dX = M^T dO + diag(kd) K Sb^T (F2, A is dead), dW = -dX S_i
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    f32x4 dx = mm16<C>([&](int r, int k) { return Ms[k * LDC + r0 + r]; },
                       [&](int k, int c) { return bfx<LDB>(Os, k, 16 * tc + c); }, zero4());
    dx = mm16<D>([&](int r, int k) { return kd[r0 + r] * kb(r0 + r, k); },
                 [&](int k, int c) { return Sb[(int64_t)(16 * tc + c) * D + k]; }, dx);
    st_tile(F2, LDT, r0, 16 * tc, dx);
  }
  f32x4 dW[NT];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc)
    dW[tc] = -mm16<D>([&](int r, int k) { return F2[(r0 + r) * LDT + k]; },
                      [&](int k, int c) { return S[(int64_t)k * D + 16 * tc + c]; }, zero4());
  __syncthreads();  // every wave has read X and written its dX rows
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) st_tile(F1, LDT, r0, 16 * tc, dW[tc]);
  __syncthreads();

  // ---- step 6: dT (to the workspace), dv, and the T^T dW term of dk
  float* dTp = b.dTp + si * C * C;
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    f32x4 dt = mm16<D>([&](int r, int k) { return F2[(r0 + r) * LDT + k]; },
                       [&](int k, int c) { return bet[16 * st + c] * bfx<LDB>(Vs, 16 * st + c, k); }, zero4());
    dt = mm16<D>([&](int r, int k) { return F1[(r0 + r) * LDT + k]; },
                 [&](int k, int c) { return bg[16 * st + c] * kb(16 * st + c, k); }, dt);
    st_tile(dTp, C, r0, 16 * st, dt);
  }
  bf16* dvg = b.dv + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    auto tcol = [&](int r, int k) { return Ts[k * LDC + r0 + r]; };
    const f32x4 dvb = mm16<C>(tcol, [&](int k, int c) { return F2[k * LDT + 16 * tc + c]; }, zero4());
    const f32x4 dkb = mm16<C>(tcol, [&](int k, int c) { return F1[k * LDT + 16 * tc + c]; }, zero4());
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = r0 + 4 * G + j, c = 16 * tc + lc;
      dbet[j] += dvb[j] * bfx<LDB>(Vs, t, c);
      dbg[j] += dkb[j] * kb(t, c);
      dvg[(int64_t)t * p.sv[2] + c] = (bf16)(bet[t] * dvb[j]);
      dK[tc][j] += bg[t] * dkb[j];
    }
    st_tile(dkp, D, r0, 16 * tc, dK[tc]);
  }
  // ---- T, dM and the per-token gate partials to the workspace
  float* Tp = b.Tp + si * C * C;
  float* dMp = b.dMp + si * C * C;
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    st_tile(Tp, C, r0, 16 * st, ld_tile(Ts, LDC, r0, 16 * st));
    st_tile(dMp, C, r0, 16 * st, dM[st]);
  }
  float* tp = b.tokp + si * (3 * C + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = r0 + 4 * G + j;
    const float sg = row16_sum(dgam[j]), sk = row16_sum(dkd[j]), sb = row16_sum(dbet[j]), sbg = row16_sum(dbg[j]);
    if (lc == 0) {
      tp[t] = sg + bet[t] * sbg;          // dL/dgamma_t (Q~ = diag(gamma) Q, and beta gamma)
      tp[C + t] = sk;                     // dL/dkd_t
      tp[2 * C + t] = sb + gam[t] * sbg;  // dL/dbeta_t from U and W
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) tp[3 * C] = (pda[0] + pda[1]) + (pda[2] + pda[3]);  // dL/dgamma_C = <Sb, S_i>
}

template <int D>
__global__ void __launch_bounds__(WY_THREADS) wy_tok2(ChunkArgs p, WyBwd b) {
  using L = WyBwdLds<D>;
  constexpr int C = CB_C, LDB = L::LDB, LDC = L::LDC, NT = D / 16;
  extern __shared__ __align__(16) char smem[];
  bf16* Qs = reinterpret_cast<bf16*>(smem + L::Q2);
  bf16* Ks = reinterpret_cast<bf16*>(smem + L::K2);
  float* Ts = reinterpret_cast<float*>(smem + L::T2);
  float* dTs = reinterpret_cast<float*>(smem + L::DT2);
  float* dMs = reinterpret_cast<float*>(smem + L::DM2);
  float* Ys = reinterpret_cast<float*>(smem + L::Y2);
  float* GAs = reinterpret_cast<float*>(smem + L::GA2);
  float* DGs = reinterpret_cast<float*>(smem + L::DG2);
  float* bet = reinterpret_cast<float*>(smem + L::R2);
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;
  float* rowE = lgam + C;   // per token: sum_s dGamma[t,s] Gamma[t,s] + the A term of dbeta (2 x C)
  float* colE = rowE + 2 * C;  // per wave: column sums of dGamma * Gamma (4 x C)

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C, si = bh * p.N + i;
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int r0 = 16 * w;
  load_bf16_rows<D>(Qs, p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2], p.sq[2]);
  load_bf16_rows<D>(Ks, p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], p.sk[2]);
  const float* Tp = b.Tp + si * C * C;
  const float* dTp = b.dTp + si * C * C;
  const float* dMp = b.dMp + si * C * C;
  for (int e = threadIdx.x; e < C * C / 4; e += WY_THREADS) {
    const int r = e / (C / 4), c = (e % (C / 4)) * 4;
    *reinterpret_cast<f32x4*>(Ts + r * LDC + c) = *reinterpret_cast<const f32x4*>(Tp + r * C + c);
    *reinterpret_cast<f32x4*>(dTs + r * LDC + c) = *reinterpret_cast<const f32x4*>(dTp + r * C + c);
    *reinterpret_cast<f32x4*>(dMs + r * LDC + c) = *reinterpret_cast<const f32x4*>(dMp + r * C + c);
  }
  float graw = 0.f;
  if (w == 0) {
    graw = p.g[bh * p.T + t0 + l];
    wy_gates(p.beta, p.g, bh * p.T + t0 + l, bet, gam, bg, kd, lgam);
  }
  __syncthreads();
  auto kb = [&](int r, int c) { return bfx<LDB>(Ks, r, c); };

  // ---- Y = dT T^T (rows of this wave)
#pragma unroll
  for (int st = 0; st < 4; ++st)
    st_tile(Ys, LDC, r0, 16 * st,
            mm16<C>([&](int r, int k) { return dTs[(r0 + r) * LDC + k]; },
                    [&](int k, int c) { return Ts[(16 * st + c) * LDC + k]; }, zero4()));
  __syncthreads();

  // ---- dA = strict_lower(-T^T Y); the A and M terms: G_A = dA beta_t Gamma, dM Gamma,
  // dbeta_t += sum_s dA R Gamma, E = dGamma * Gamma = (dA beta_t R + dM Rq) Gamma
  float rsum[4] = {0.f, 0.f, 0.f, 0.f}, bsum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    f32x4 ga = zero4(), dg = zero4();
    float csum = 0.f;
    if (st <= w) {
      const f32x4 dA = mm16<C>([&](int r, int k) { return Ts[k * LDC + r0 + r]; },
                               [&](int k, int c) { return Ys[k * LDC + 16 * st + c]; }, zero4());
      const f32x4 kk = mm16<D>([&](int r, int k) { return kb(r0 + r, k); },
                               [&](int k, int c) { return kb(16 * st + c, k); }, zero4());
      const f32x4 qk = mm16<D>([&](int r, int k) { return bfx<LDB>(Qs, r0 + r, k); },
                               [&](int k, int c) { return kb(16 * st + c, k); }, zero4());
      const int s = 16 * st + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = r0 + 4 * G + j;
        const float e = s <= t ? expf(lgam[t] - lgam[s]) : 0.f;
        const float da = s < t ? -dA[j] : 0.f;
        const float dm = s <= t ? dMs[t * LDC + s] : 0.f;
        ga[j] = da * bet[t] * e;
        dg[j] = dm * e;
        bsum[j] += da * kk[j] * e;
        const float E = (da * bet[t] * kk[j] + dm * qk[j]) * e;
        rsum[j] += E;
        csum += E;
      }
    }
    st_tile(GAs, LDC, r0, 16 * st, ga);
    st_tile(DGs, LDC, r0, 16 * st, dg);
    csum = group_sum(csum);
    if (G == 0) colE[w * C + 16 * st + lc] = csum;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float rs = row16_sum(rsum[j]), bs = row16_sum(bsum[j]);
    if (lc == 0) {
      rowE[r0 + 4 * G + j] = rs;
      rowE[C + r0 + 4 * G + j] = bs;
    }
  }
  __syncthreads();

  // ---- dk = partial + G_A K + G_A^T K + (dM Gamma)^T Q,  dq = partial + (dM Gamma) K
  const float* dqp = b.dQp + (bh * p.T + t0) * (int64_t)D;
  const float* dkp = b.dKp + (bh * p.T + t0) * (int64_t)D;
  bf16* dqg = b.dq + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2];
  bf16* dkg = b.dk + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    auto kcol = [&](int k, int c) { return kb(k, 16 * tc + c); };
    f32x4 dk = ld_tile(dkp, D, r0, 16 * tc);
    dk = mm16<C>([&](int r, int k) { return GAs[(r0 + r) * LDC + k]; }, kcol, dk);
    dk = mm16<C>([&](int r, int k) { return GAs[k * LDC + r0 + r]; }, kcol, dk);
    dk = mm16<C>([&](int r, int k) { return DGs[k * LDC + r0 + r]; },
                 [&](int k, int c) { return bfx<LDB>(Qs, k, 16 * tc + c); }, dk);
    f32x4 dq = ld_tile(dqp, D, r0, 16 * tc);
    dq = mm16<C>([&](int r, int k) { return DGs[(r0 + r) * LDC + k]; }, kcol, dq);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = r0 + 4 * G + j;
      const int c = 16 * tc + lc;
      dkg[t * p.sk[2] + c] = (bf16)dk[j];
      dqg[t * p.sq[2] + c] = (bf16)dq[j];
    }
  }

  // ---- gate gradients (wave 0, lane = token)
  if (w == 0) {
    const float* tp = b.tokp + si * (3 * C + 4);
    const float dgm = tp[l], dkdv = tp[C + l], dbu = tp[2 * C + l], dgC = tp[3 * C];
    // dgc_t: gamma_t = exp(gc_t), kd_t = exp(gc_{C-1} - gc_t), the Gamma
    // exponents (row minus column sums), and gamma_{C-1} = a of the scan
    float dgc = dgm * gam[l] - dkdv * kd[l] + rowE[l] - ((colE[l] + colE[C + l]) + (colE[2 * C + l] + colE[3 * C + l]));
    const float kdsum = wave_sum(dkdv * kd[l]);
    if (l == C - 1) dgc += kdsum + dgC * gam[l];
    // dlg_u = sum_{t >= u} dgc_t
    const float dlg = wave_sum(dgc) - (wave_incl_scan(dgc) - dgc);
    const int64_t o = bh * p.T + t0 + l;
    b.dg[o] = graw >= LOG_FLOOR ? dlg : 0.f;
    b.dbeta[o] = dbu + rowE[C + l];
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
hipError_t launch_k(K kern, int bytes, int64_t grid, hipStream_t s, const ChunkArgs& a, const WyBwd& b) {
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(WY_THREADS), bytes, s, a, b);
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

// backward workspace (floats): gS, Sb (d x d per chunk), partial dq, dk
// (B H T d), T, dT, dM (C x C per chunk), per-chunk gate partials (3 C + 4)
size_t bwd_floats(int64_t B, int64_t H, int64_t T, int d) {
  const int64_t chunks = B * H * (T / CB_C), mat = (int64_t)d * d, tok = B * H * T * (int64_t)d;
  return (size_t)(2 * chunks * mat + 2 * tok + 3 * chunks * CB_C * CB_C + chunks * (3 * CB_C + 4));
}

template <int D>
hipError_t launch_wy_bwd(const ChunkArgs& a, float* ckpt, const void* dO, void* dq, void* dk, void* dv, float* dbeta,
                         float* dg, float* ws, hipStream_t s) {
  using L = WyBwdLds<D>;
  const int64_t chunks = a.B * a.H * a.N, mat = (int64_t)D * D, tok = a.B * a.H * a.T * (int64_t)D;
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
  b.dQp = Sb + chunks * mat;
  b.dKp = b.dQp + tok;
  b.Tp = b.dKp + tok;
  b.dTp = b.Tp + chunks * CB_C * CB_C;
  b.dMp = b.dTp + chunks * CB_C * CB_C;
  b.tokp = b.dMp + chunks * CB_C * CB_C;
  b.dq = static_cast<bf16*>(dq);
  b.dk = static_cast<bf16*>(dk);
  b.dv = static_cast<bf16*>(dv);
  b.dbeta = dbeta;
  b.dg = dg;
  hipError_t e = launch_k(wy_gs<D>, 2 * CB_C * (D + 4) * 4, chunks, s, a, b);
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
  if ((e = launch_k(wy_tok1<D>, L::TOK1_BYTES, chunks, s, a, b)) != hipSuccess) return e;
  return launch_k(wy_tok2<D>, L::TOK2_BYTES, chunks, s, a, b);
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
