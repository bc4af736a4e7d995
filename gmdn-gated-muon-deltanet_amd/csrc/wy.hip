// Exact WY/UT mode: the token-exact gated delta rule
//     S_t = alpha_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T,   o_t = S_t q_t
// chunked with the WY/UT transform (the reference trains the chunk-frozen
// E-form instead and leaves this mode out, train_ablation.py:12-18).
//
// Per (b, h) and chunk of C = 64 tokens, with gamma_t the decay product from
// the chunk start (log-gates clamped at log 1e-6), Gamma[t, s] = gamma_t / gamma_s:
//     A = strict_lower(diag(beta) (K K^T * Gamma)),   T = (I + A)^-1
//     X = U - W S^T with U = T diag(beta) V, W = T diag(beta gamma) K
//     o = diag(gamma) Q S^T + M X,   M = lower_incl(Q K^T * Gamma)
//     S' = gamma_C S + X^T diag(gamma_C / gamma) K
// The state recurrence is affine, S' = a S + U_A - S K_A, which is the
// drop-in delta scan's (fast_scan.py:82) with
//     a = gamma_C,  U_A = (diag(beta) V)^T P,  K_A = (diag(beta gamma) K)^T P,
//     P = T^T diag(gamma_C / gamma) K,
// and the output is o = Qt S^T + Ov with
//     Qt = diag(gamma) Q - (M T diag(beta gamma)) K,  Ov = (M T diag(beta)) V.
//
// wy_prep (one workgroup of 4 waves per (b, h, chunk)) forms a, U_A, K_A, Qt
// and Ov with exact float32 MFMA (v_mfma_f32_16x16x4_f32) on float32 tiles
// in LDS; T by blocked forward substitution (the four 16 x 16 diagonal
// blocks by one wave each, the off-diagonal blocks in three levels).  The
// delta scan kernels then carry S, and wy_out forms o = Qt S_i^T + Ov.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"
#include "scan_a.h"

namespace gmdn {
namespace {

constexpr int WY_THREADS = 256;

template <int D>
struct WyLds {
  static constexpr int LDT = D + 4;   // float stride of a token tile row
  static constexpr int LDC = CB_C + 4;  // float stride of a C x C matrix row
  static constexpr int TILE = CB_C * LDT;   // floats
  static constexpr int CC = CB_C * LDC;     // floats
  static constexpr int K0 = 0, V0 = TILE, Q0 = 2 * TILE;   // Q's slot later holds P
  static constexpr int T0 = 3 * TILE, A0 = T0 + CC;          // A's slot later holds M, then M T
  static constexpr int X0 = A0 + CC;                         // 3 waves x 16 x 16 scratch
  static constexpr int S0 = X0 + 3 * 256;  // beta, gamma, beta gamma, gamma_C / gamma, log gamma
  static constexpr int FLOATS = S0 + 5 * CB_C;
  static_assert(FLOATS * 4 <= 160 * 1024, "WY prep LDS exceeds the 160 KiB of a CU");
};

// acc += sum_k A(m, k) B(k, n) over a 16 x 16 tile, k in steps of 4 (exact fp32
// MFMA); a(i, k) / b(k, i) give the lane's operand element for row / column i.
template <int K, class FA, class FB>
GMDN_DEV f32x4 mm16(FA a, FB b, f32x4 acc) {
  const int l = lane_id(), i = l & 15, G = l >> 4;
#pragma unroll 4
  for (int k = 0; k < K; k += 4) acc = mfma_f32(a(i, k + G), b(k + G, i), acc);
  return acc;
}

// D-layout tile -> row-major float matrix at (r0, c0)
GMDN_DEV void st_tile(float* X, int ld, int r0, int c0, const f32x4& t) {
  const int l = lane_id(), c = l & 15, G = l >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) X[(r0 + 4 * G + j) * ld + c0 + c] = t[j];
}

template <int D>
__global__ void __launch_bounds__(WY_THREADS)
wy_prep(ChunkArgs p, float* __restrict__ UA, float* __restrict__ KA, float* __restrict__ Qt,
        float* __restrict__ Ov, float* __restrict__ aout) {
  using L = WyLds<D>;
  constexpr int C = CB_C, LDT = L::LDT, LDC = L::LDC, NT = D / 16;
  extern __shared__ __align__(16) float sm[];
  float* Ks = sm + L::K0;
  float* Vs = sm + L::V0;
  float* Qs = sm + L::Q0;
  float* Ts = sm + L::T0;
  float* As = sm + L::A0;
  float* bet = sm + L::S0;
  float* gam = bet + C;
  float* bg = gam + C;
  float* kd = bg + C;
  float* lgam = kd + C;  // prefix sums of the clamped log-gates

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C;
  const int w = wave_id(), l = lane_id();

  // ---- tiles as float32, gates, zeroed T
  const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2];
  const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2];
  const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2];
  for (int e = threadIdx.x; e < C * D / 8; e += WY_THREADS) {
    const int t = e / (D / 8), c = (e % (D / 8)) * 8;
    const bf16x8 kq = *reinterpret_cast<const bf16x8*>(kg + t * p.sk[2] + c);
    const bf16x8 vq = *reinterpret_cast<const bf16x8*>(vg + t * p.sv[2] + c);
    const bf16x8 qq = *reinterpret_cast<const bf16x8*>(qg + t * p.sq[2] + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      Ks[t * LDT + c + j] = (float)kq[j];
      Vs[t * LDT + c + j] = (float)vq[j];
      Qs[t * LDT + c + j] = (float)qq[j];
    }
  }
  for (int e = threadIdx.x; e < C * LDC; e += WY_THREADS) Ts[e] = 0.f;
  if (w == 0) {
    const float bt = p.beta[bh * p.T + t0 + l];
    const float lg = fmaxf(p.g[bh * p.T + t0 + l], LOG_FLOOR);
    // inclusive prefix sum of the log-gates over the chunk
    float gc = lg;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(gc, o, 64);
      if (l >= o) gc += y;
    }
    const float gC = __shfl(gc, 63, 64);
    const float g_ = expf(gc);
    bet[l] = bt;
    gam[l] = g_;
    bg[l] = bt * g_;
    kd[l] = expf(gC - gc);
    lgam[l] = gc;
    if (l == 63) aout[bh * p.N + i] = g_;
  }
  __syncthreads();

  // ---- A = strict_lower(diag(beta) (K K^T * Gamma)): causal tiles by wave.
  // Gamma[t, s] = exp(log gamma_t - log gamma_s) on the causal entries only:
  // the ratio gamma_t / gamma_s of two underflowed products would be 0 / 0.
  const float* gm = gam;
  for (int tile = w; tile < 16; tile += 4) {
    const int tt = tile >> 2, st = tile & 3;
    f32x4 acc = zero4();
    if (st <= tt) {
      acc = mm16<D>([&](int ii, int k) { return Ks[(16 * tt + ii) * LDT + k]; },
                    [&](int k, int ii) { return Ks[(16 * st + ii) * LDT + k]; }, acc);
      const int c = l & 15, G = l >> 4, s = 16 * st + c;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tt + 4 * G + j;
        acc[j] = s < t ? bet[t] * acc[j] * expf(lgam[t] - lgam[s]) : 0.f;
      }
    }
    st_tile(As, LDC, 16 * tt, 16 * st, acc);
  }
  __syncthreads();

  // ---- T = (I + A)^-1: diagonal 16 x 16 blocks by forward substitution
  // (wave w, lane j < 16 holds column j of block w)
  if (l < 16) {
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
  // off-diagonal blocks T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj, level d = i - j;
  // wave w takes the block with j = w; lane (r = l / 4, c = 4 (l % 4) ..)
  float* Xw = sm + L::X0 + 256 * (w < 3 ? w : 0);
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

  // ---- M = lower_incl(Q K^T * Gamma) into A's slot, then M T in place
  for (int tile = w; tile < 16; tile += 4) {
    const int tt = tile >> 2, st = tile & 3;
    f32x4 acc = zero4();
    if (st <= tt) {
      acc = mm16<D>([&](int ii, int k) { return Qs[(16 * tt + ii) * LDT + k]; },
                    [&](int k, int ii) { return Ks[(16 * st + ii) * LDT + k]; }, acc);
      const int c = l & 15, G = l >> 4, s = 16 * st + c;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tt + 4 * G + j;
        acc[j] = s <= t ? acc[j] * expf(lgam[t] - lgam[s]) : 0.f;
      }
    }
    st_tile(As, LDC, 16 * tt, 16 * st, acc);
  }
  __syncthreads();
  {
    f32x4 mt[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int tile = w + 4 * q, tt = tile >> 2, st = tile & 3;
      mt[q] = zero4();
      if (st <= tt)
        mt[q] = mm16<CB_C>([&](int ii, int k) { return As[(16 * tt + ii) * LDC + k]; },
                           [&](int k, int ii) { return Ts[k * LDC + 16 * st + ii]; }, mt[q]);
    }
    __syncthreads();  // every wave has read M
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int tile = w + 4 * q, tt = tile >> 2, st = tile & 3;
      st_tile(As, LDC, 16 * tt, 16 * st, mt[q]);
    }
  }
  __syncthreads();

  // ---- Qt = diag(gamma) Q - (M T diag(beta gamma)) K and Ov = (M T diag(beta)) V
  //      (float32, (B, H, T, d) contiguous); lane (c, G) of tile (tt, tc)
  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D;
  for (int tile = w; tile < 4 * NT; tile += 4) {
    const int tt = tile / NT, tc = tile % NT;
    f32x4 qa = mm16<CB_C>([&](int ii, int k) { return As[(16 * tt + ii) * LDC + k] * bg[k]; },
                          [&](int k, int ii) { return Ks[k * LDT + 16 * tc + ii]; }, zero4());
    f32x4 oa = mm16<CB_C>([&](int ii, int k) { return As[(16 * tt + ii) * LDC + k] * bet[k]; },
                          [&](int k, int ii) { return Vs[k * LDT + 16 * tc + ii]; }, zero4());
    const int c = l & 15, G = l >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j, col = 16 * tc + c;
      Qt[tokbase + (int64_t)t * D + col] = gm[t] * Qs[t * LDT + col] - qa[j];
      Ov[tokbase + (int64_t)t * D + col] = oa[j];
    }
  }
  __syncthreads();  // Q's slot is free: P = T^T diag(gamma_C / gamma) K
  float* Ps = Qs;
  for (int tile = w; tile < 4 * NT; tile += 4) {
    const int st = tile / NT, tc = tile % NT;
    const f32x4 pa = mm16<CB_C>([&](int ii, int k) { return Ts[k * LDC + 16 * st + ii] * kd[k]; },
                                [&](int k, int ii) { return Ks[k * LDT + 16 * tc + ii]; }, zero4());
    st_tile(Ps, LDT, 16 * st, 16 * tc, pa);
  }
  __syncthreads();
  // ---- U_A = (diag(beta) V)^T P, K_A = (diag(beta gamma) K)^T P  (d x d, float32)
  const int64_t mbase = (bh * p.N + i) * (int64_t)D * D;
  for (int tile = w; tile < NT * NT; tile += 4) {
    const int tr = tile / NT, tc = tile % NT;
    const f32x4 ua = mm16<CB_C>([&](int ii, int k) { return Vs[k * LDT + 16 * tr + ii] * bet[k]; },
                                [&](int k, int ii) { return Ps[k * LDT + 16 * tc + ii]; }, zero4());
    const f32x4 ka = mm16<CB_C>([&](int ii, int k) { return Ks[k * LDT + 16 * tr + ii] * bg[k]; },
                                [&](int k, int ii) { return Ps[k * LDT + 16 * tc + ii]; }, zero4());
    const int c = l & 15, G = l >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t o = mbase + (int64_t)(16 * tr + 4 * G + j) * D + 16 * tc + c;
      UA[o] = ua[j];
      KA[o] = ka[j];
    }
  }
}

// o = Qt S_i^T + Ov for one (b, h, chunk): Qt rows and S_i staged in LDS as float32
template <int D>
__global__ void __launch_bounds__(WY_THREADS)
wy_out(ChunkArgs p, const float* __restrict__ Qt, const float* __restrict__ Ov, const float* __restrict__ Sst) {
  constexpr int C = CB_C, LDT = D + 4, NT = D / 16;
  extern __shared__ __align__(16) float sm[];
  float* Qs = sm;             // C x D
  float* Ss = sm + C * LDT;   // D x D
  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H, t0 = (int64_t)i * C;
  const int w = wave_id(), l = lane_id();
  const int64_t tokbase = (bh * p.T + t0) * (int64_t)D;
  const float* S = Sst + (bh * p.N + i) * (int64_t)D * D;
  for (int e = threadIdx.x; e < C * D / 4; e += WY_THREADS) {
    const int t = e / (D / 4), c = (e % (D / 4)) * 4;
    *reinterpret_cast<f32x4*>(Qs + t * LDT + c) = *reinterpret_cast<const f32x4*>(Qt + tokbase + (int64_t)t * D + c);
  }
  for (int e = threadIdx.x; e < D * D / 4; e += WY_THREADS) {
    const int r = e / (D / 4), c = (e % (D / 4)) * 4;
    *reinterpret_cast<f32x4*>(Ss + r * LDT + c) = *reinterpret_cast<const f32x4*>(S + (int64_t)r * D + c);
  }
  __syncthreads();
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2];
  for (int tile = w; tile < 4 * NT; tile += 4) {
    const int tt = tile / NT, tr = tile % NT;
    // tile [t][r] = sum_c Qt[t][c] S[r][c]
    const f32x4 acc = mm16<D>([&](int ii, int k) { return Qs[(16 * tt + ii) * LDT + k]; },
                              [&](int k, int ii) { return Ss[(16 * tr + ii) * LDT + k]; }, zero4());
    const int c = l & 15, G = l >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = 16 * tt + 4 * G + j, r = 16 * tr + c;
      og[t * p.so[2] + r] = (bf16)(acc[j] + Ov[tokbase + (int64_t)t * D + r]);
    }
  }
}

template <int D>
hipError_t launch_wy(const ChunkArgs& a, float* ws, hipStream_t s) {
  const int64_t chunks = a.B * a.H * a.N, mat = (int64_t)D * D, tok = a.B * a.H * a.T * (int64_t)D;
  float* UA = ws;
  float* KA = UA + chunks * mat;
  float* S_all = KA + chunks * mat;
  float* Qt = S_all + chunks * mat;
  float* Ov = Qt + tok;
  float* av = Ov + tok;
  auto kp = wy_prep<D>;
  auto ko = wy_out<D>;
  const int lp = WyLds<D>::FLOATS * 4, lo = (CB_C + D) * (D + 4) * 4;
  hipError_t e = hipFuncSetAttribute((const void*)kp, hipFuncAttributeMaxDynamicSharedMemorySize, lp);
  if (e == hipSuccess) e = hipFuncSetAttribute((const void*)ko, hipFuncAttributeMaxDynamicSharedMemorySize, lo);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kp, dim3((unsigned)chunks), dim3(WY_THREADS), lp, s, a, UA, KA, Qt, Ov, av);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  ScanArgs sa{};
  sa.U = UA;
  sa.K = KA;
  sa.a = av;
  sa.S_all = S_all;
  sa.BH = a.B * a.H;
  sa.N = a.N;
  sa.dh = D;
  sa.rule = 0;
  sa.ns = 0;
  sa.precision = GMDN_PREC_IEEE;  // exact float32 state products
  sa.stream = s;
  if ((e = scan_fwd_rows_launch(sa)) != hipSuccess) return e;
  hipLaunchKernelGGL(ko, dim3((unsigned)chunks), dim3(WY_THREADS), lo, s, a, (const float*)Qt, (const float*)Ov,
                     (const float*)S_all);
  return hipGetLastError();
}

}  // namespace

size_t wy_workspace_floats(int64_t B, int64_t H, int64_t T, int d) {
  const int64_t chunks = B * H * (T / CB_C), mat = (int64_t)d * d, tok = B * H * T * (int64_t)d;
  return (size_t)(3 * chunks * mat + 2 * tok + chunks);
}

hipError_t wy_fwd_launch(const ChunkArgs& a, int d, float* ws, hipStream_t s) {
  if (d == 128) return launch_wy<128>(a, ws, s);
  if (d == 64) return launch_wy<64>(a, ws, s);
  return hipErrorInvalidValue;
}

}  // namespace gmdn
