// Level B on float32 token streams (desc->dtype == GMDN_DTYPE_F32): the
// reference's matrix form of the mixer core (train_ablation.py:142-187) with
// exact float32 products everywhere, as the reference computes it when
// autocast is off (its CPU path, train_ablation.py:424, 465).  Per (b, h) and
// chunk i of C = 64 tokens:
//
//   A  = tril(Q K^T) diag(beta)                 (diagonal included, :161-163)
//   Kw = K^T diag(w) K,  Uv = V^T diag(w) K     (:164-165; w: delta beta,
//                                                muon prod_{s>t} mu_s, adam 1)
//   Qt = Q - A K,  Ov = A V                     (:166-167)
//   a, b, m, n: the chunk scalars               (:169-175)
//   S_all = fast_state_scan(Uv, Kw, a, b, m, n) (:178-182)
//   o  = Qt S_i^T + Ov                          (:184-186)
//
// Forward: f32_prep (chunk-parallel: Kw, Uv, a, b, m, n), the drop-in scan's
// kernels in 'ieee' (exact float32 MFMA; any rule), f32_out (chunk-parallel:
// o).  Backward: f32_gs (gS_i = dL/dS_i = dO^T Qt), the drop-in scan's
// backward in 'ieee' (dUv_i, dKw_i, da, db, dm, dn), f32_tok (token and gate
// gradients):
//
//   dQt = dO S_i,  E = V - K S_i^T,  dA = tril(dO E^T)
//   dQ  = dQt + (dA diag(beta)) K
//   dK  = -A^T dQt + (dA diag(beta))^T Q + diag(w) (V dUv + K (dKw + dKw^T))
//   dV  = A^T dO + diag(w) K dUv^T
//   dw_t = k_t . (V dUv)_t + k_t^T dKw k_t
//   dbeta_s = sum_t dA[t,s] (q_t . k_s) + db / C  (+ dw_s for delta)
//   dg_t = da a [g_t >= log 1e-6],  dgmu_t = (dm m + sum_{s<t} dw_s w_s [muon]) [gmu_t >= log 1e-6],
//   dgnu_t = dn n [gnu_t >= log 1e-6]
//
// Every kernel runs one workgroup of four waves per (b, h, chunk) on
// float32 tiles staged in LDS (row stride d + 4 floats); wave w owns token
// rows 16 w .. 16 w + 15 wherever a product is local to token rows.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"
#include "f32mm.h"
#include "scan_a.h"

namespace gmdn {
namespace {

constexpr int F_THREADS = 256;
constexpr int F_WAVES = 4;
static_assert(CB_C == 16 * F_WAVES, "one 16-token tile per wave");

struct F32Args {
  const float *q, *k, *v, *dO;
  const float *beta, *g, *gmu, *gnu;
  float* o;
  int64_t B, H, T;
  int N;
  int64_t sq[3], sk[3], sv[3], so[3];
  const float* S;                 // S_i planes (B, H, N, d, d)
  float *Kw, *Uv, *abmn;          // f32_prep outputs
  float* gS;                      // f32_gs output
  const float *dKw, *dUv, *dsc;   // the drop-in backward's dK, dU and [da | db | dm | dn]
  float *dq, *dk, *dv, *dbeta, *dg, *dgmu, *dgnu;
};

template <int D>
struct F32Lds {
  static constexpr int C = CB_C;
  static constexpr int LD = D + 4;       // float stride of a token tile row
  static constexpr int LDC = C + 2;      // float stride of a C x C matrix row
  static constexpr int TILE = C * LD;    // floats of a token tile
  static constexpr int CC = C * LDC;     // floats of a C x C matrix
  static constexpr int SMAT = D * LD;    // floats of a d x d plane
  // f32_out: K and V tiles, later S_i
  static constexpr int KV = 2 * TILE > SMAT ? 2 * TILE : SMAT;
  // f32_tok: V tile, later E, then A and dA diag(beta)
  static constexpr int VSLOT = TILE > 2 * CC ? TILE : 2 * CC;
  static constexpr int PREP_BYTES = (2 * TILE + C) * 4;
  static constexpr int OUT_BYTES = (TILE + KV + CC + C) * 4;
  static constexpr int GS_BYTES = (3 * TILE + CC + C) * 4;
  static constexpr int TOK_BYTES = (3 * TILE + VSLOT + (3 + F_WAVES) * C) * 4;
  static_assert(OUT_BYTES <= 160 * 1024 && GS_BYTES <= 160 * 1024 && TOK_BYTES <= 160 * 1024,
                "float32 chunk LDS exceeds the 160 KiB of a CU");
};

// Chunk rows of a float32 token stream into an LDS tile (row stride D + 4).
template <int D>
GMDN_DEV void load_rows(float* dst, const float* src, int64_t stride) {
  constexpr int LD = D + 4, V4 = D / 4;
  for (int e = threadIdx.x; e < CB_C * V4; e += F_THREADS) {
    const int t = e / V4, c = (e % V4) * 4;
    *reinterpret_cast<f32x4*>(dst + t * LD + c) = *reinterpret_cast<const f32x4*>(src + t * stride + c);
  }
}

// A = tril(Q K^T) diag(beta) into As (row stride LDC); rb = beta of the chunk.
template <int D>
GMDN_DEV void causal_a(float* As, const float* Qs, const float* Ks, const float* rb, int w) {
  using L = F32Lds<D>;
  constexpr int LD = L::LD;
  const int l = lane_id(), lc = l & 15, G = l >> 4;
  for (int tile = w; tile < 16; tile += F_WAVES) {
    const int tt = tile >> 2, st = tile & 3;
    f32x4 acc = zero4();
    if (st <= tt) {
      acc = mm16<D>([&](int r, int k) { return Qs[(16 * tt + r) * LD + k]; },
                    [&](int k, int c) { return Ks[(16 * st + c) * LD + k]; }, acc);
      const int s = 16 * st + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = s <= 16 * tt + 4 * G + j ? acc[j] * rb[s] : 0.f;
    }
    st_tile(As, L::LDC, 16 * tt, 16 * st, acc);
  }
}

// Qt = Q - A K in place of Q (every product reads A and K only).
template <int D>
GMDN_DEV void qt_in_place(float* Qs, const float* As, const float* Ks, int w) {
  using L = F32Lds<D>;
  constexpr int LD = L::LD, NT = D / 16;
  for (int tile = w; tile < 4 * NT; tile += F_WAVES) {
    const int tt = tile / NT, tc = tile % NT;
    const f32x4 ak = mm16<CB_C>([&](int r, int k) { return As[(16 * tt + r) * L::LDC + k]; },
                                [&](int k, int c) { return Ks[k * LD + 16 * tc + c]; }, zero4());
    st_tile(Qs, LD, 16 * tt, 16 * tc, ld_tile(Qs, LD, 16 * tt, 16 * tc) - ak);
  }
}

struct ChunkIdx {
  int64_t bh, bb, hh, t0, si;
  int i;
  GMDN_DEV explicit ChunkIdx(const F32Args& p) {
    bh = blockIdx.x / p.N;
    i = (int)(blockIdx.x % p.N);
    bb = bh / p.H;
    hh = bh % p.H;
    t0 = (int64_t)i * CB_C;
    si = bh * p.N + i;
  }
};

// ------------------------------------------------------------------ forward
template <int D, int RULE>
__global__ void __launch_bounds__(F_THREADS) f32_prep(F32Args p) {
  using L = F32Lds<D>;
  constexpr int C = CB_C, LD = L::LD, NT = D / 16;
  extern __shared__ __align__(16) float sm[];
  float* Ks = sm;
  float* Vs = sm + L::TILE;
  float* rw = sm + 2 * L::TILE;
  const ChunkIdx x(p);
  const int w = wave_id(), l = lane_id();
  load_rows<D>(Ks, p.k + x.bb * p.sk[0] + x.hh * p.sk[1] + x.t0 * p.sk[2], p.sk[2]);
  load_rows<D>(Vs, p.v + x.bb * p.sv[0] + x.hh * p.sv[1] + x.t0 * p.sv[2], p.sv[2]);
  if (w == 0) {
    const int64_t e = x.bh * p.T + x.t0 + l;
    const float bt = p.beta[e];
    const float lg = fmaxf(p.g[e], LOG_FLOOR);
    const float lm = RULE >= 1 ? fmaxf(p.gmu[e], LOG_FLOOR) : 0.f;
    const float a = expf(wave_sum(lg));
    const float b = wave_sum(bt) * (1.f / C);
    const float msum = wave_sum(lm);
    const float n = RULE == 2 ? expf(wave_sum(fmaxf(p.gnu[e], LOG_FLOOR))) : 1.f;
    float wt = bt;                                            // delta: w = beta
    if constexpr (RULE == 1) wt = expf(msum - wave_incl_scan(lm));  // muon: exp(sum_{s > t} log mu_s)
    if constexpr (RULE == 2) wt = 1.f;                        // adam: w = 1
    rw[l] = wt;
    if (l == 0) {
      const int64_t BHN = p.B * p.H * p.N;
      p.abmn[x.si] = a;
      p.abmn[BHN + x.si] = b;
      p.abmn[2 * BHN + x.si] = RULE >= 1 ? expf(msum) : 1.f;
      p.abmn[3 * BHN + x.si] = n;
    }
  }
  __syncthreads();
  float* Kw = p.Kw + x.si * (int64_t)D * D;
  float* Uv = p.Uv + x.si * (int64_t)D * D;
  for (int tile = w; tile < NT * NT; tile += F_WAVES) {
    const int ta = tile / NT, tb = tile % NT;
    const f32x4 kw = mm16<C>([&](int r, int k) { return rw[k] * Ks[k * LD + 16 * ta + r]; },
                             [&](int k, int c) { return Ks[k * LD + 16 * tb + c]; }, zero4());
    const f32x4 uv = mm16<C>([&](int r, int k) { return rw[k] * Vs[k * LD + 16 * ta + r]; },
                             [&](int k, int c) { return Ks[k * LD + 16 * tb + c]; }, zero4());
    st_tile(Kw, D, 16 * ta, 16 * tb, kw);
    st_tile(Uv, D, 16 * ta, 16 * tb, uv);
  }
}

template <int D>
__global__ void __launch_bounds__(F_THREADS) f32_out(F32Args p) {
  using L = F32Lds<D>;
  constexpr int C = CB_C, LD = L::LD, NT = D / 16, NO = 4 * NT / F_WAVES;
  extern __shared__ __align__(16) float sm[];
  float* Qs = sm;
  float* Ks = sm + L::TILE;
  float* Vs = Ks + L::TILE;
  float* Ss = Ks;  // S_i once A K and A V are formed
  float* As = sm + L::TILE + L::KV;
  float* rb = As + L::CC;
  const ChunkIdx x(p);
  const int w = wave_id(), l = lane_id();
  load_rows<D>(Qs, p.q + x.bb * p.sq[0] + x.hh * p.sq[1] + x.t0 * p.sq[2], p.sq[2]);
  load_rows<D>(Ks, p.k + x.bb * p.sk[0] + x.hh * p.sk[1] + x.t0 * p.sk[2], p.sk[2]);
  load_rows<D>(Vs, p.v + x.bb * p.sv[0] + x.hh * p.sv[1] + x.t0 * p.sv[2], p.sv[2]);
  if (w == 0) rb[l] = p.beta[x.bh * p.T + x.t0 + l];
  __syncthreads();
  causal_a<D>(As, Qs, Ks, rb, w);
  __syncthreads();
  // Ov = A V into registers, Qt = Q - A K in place of Q
  f32x4 O[NO];
#pragma unroll
  for (int q = 0; q < NO; ++q) {
    const int tile = w + F_WAVES * q, tt = tile / NT, tc = tile % NT;
    auto arow = [&](int r, int k) { return As[(16 * tt + r) * L::LDC + k]; };
    O[q] = mm16<C>(arow, [&](int k, int c) { return Vs[k * LD + 16 * tc + c]; }, zero4());
    const f32x4 ak = mm16<C>(arow, [&](int k, int c) { return Ks[k * LD + 16 * tc + c]; }, zero4());
    st_tile(Qs, LD, 16 * tt, 16 * tc, ld_tile(Qs, LD, 16 * tt, 16 * tc) - ak);
  }
  __syncthreads();  // K and V are read: their slot takes S_i
  {
    const float* S = p.S + x.si * (int64_t)D * D;
    for (int e = threadIdx.x; e < D * D / 4; e += F_THREADS) {
      const int r = e / (D / 4), c = (e % (D / 4)) * 4;
      *reinterpret_cast<f32x4*>(Ss + r * LD + c) = *reinterpret_cast<const f32x4*>(S + (int64_t)r * D + c);
    }
  }
  __syncthreads();
  float* og = p.o + x.bb * p.so[0] + x.hh * p.so[1] + x.t0 * p.so[2];
  const int lc = l & 15, G = l >> 4;
#pragma unroll
  for (int q = 0; q < NO; ++q) {
    const int tile = w + F_WAVES * q, tt = tile / NT, tr = tile % NT;
    // o[t][r] = sum_c Qt[t][c] S[r][c] + Ov[t][r]
    const f32x4 acc = mm16<D>([&](int r, int k) { return Qs[(16 * tt + r) * LD + k]; },
                              [&](int k, int c) { return Ss[(16 * tr + c) * LD + k]; }, O[q]);
#pragma unroll
    for (int j = 0; j < 4; ++j) og[(int64_t)(16 * tt + 4 * G + j) * p.so[2] + 16 * tr + lc] = acc[j];
  }
}

// ----------------------------------------------------------------- backward
template <int D>
__global__ void __launch_bounds__(F_THREADS) f32_gs(F32Args p) {
  using L = F32Lds<D>;
  constexpr int C = CB_C, LD = L::LD, NT = D / 16;
  extern __shared__ __align__(16) float sm[];
  float* Qs = sm;
  float* Ks = sm + L::TILE;
  float* Os = sm + 2 * L::TILE;
  float* As = sm + 3 * L::TILE;
  float* rb = As + L::CC;
  const ChunkIdx x(p);
  const int w = wave_id(), l = lane_id();
  load_rows<D>(Qs, p.q + x.bb * p.sq[0] + x.hh * p.sq[1] + x.t0 * p.sq[2], p.sq[2]);
  load_rows<D>(Ks, p.k + x.bb * p.sk[0] + x.hh * p.sk[1] + x.t0 * p.sk[2], p.sk[2]);
  load_rows<D>(Os, p.dO + x.bb * p.so[0] + x.hh * p.so[1] + x.t0 * p.so[2], p.so[2]);
  if (w == 0) rb[l] = p.beta[x.bh * p.T + x.t0 + l];
  __syncthreads();
  causal_a<D>(As, Qs, Ks, rb, w);
  __syncthreads();
  qt_in_place<D>(Qs, As, Ks, w);
  __syncthreads();
  // gS[r][c] = sum_t dO[t][r] Qt[t][c]
  float* gS = p.gS + x.si * (int64_t)D * D;
  for (int tile = w; tile < NT * NT; tile += F_WAVES) {
    const int tr = tile / NT, tc = tile % NT;
    const f32x4 acc = mm16<C>([&](int r, int k) { return Os[k * LD + 16 * tr + r]; },
                              [&](int k, int c) { return Qs[k * LD + 16 * tc + c]; }, zero4());
    st_tile(gS, D, 16 * tr, 16 * tc, acc);
  }
}

template <int D, int RULE>
__global__ void __launch_bounds__(F_THREADS) f32_tok(F32Args p) {
  using L = F32Lds<D>;
  constexpr int C = CB_C, LD = L::LD, LDC = L::LDC, NT = D / 16, NTT = C / 16;
  extern __shared__ __align__(16) float sm[];
  float* Qs = sm;
  float* Os = sm + L::TILE;        // dO
  float* Ks = sm + 2 * L::TILE;    // K, later dQt
  float* Vs = sm + 3 * L::TILE;    // V, later E, then A and dA diag(beta)
  float* As = Vs;
  float* Abs = Vs + L::CC;
  float* red = Vs + L::VSLOT;
  float* rb = red;                 // beta
  float* rw = red + C;             // token weights w
  float* rdw = red + 2 * C;        // dL/dw
  float* pdb = red + 3 * C;        // [wave][s]: sum over the wave's t of dA[t,s] (q_t . k_s)
  const ChunkIdx x(p);
  const int w = wave_id(), l = lane_id(), lc = l & 15, G = l >> 4;
  const int tt = w;  // this wave's token tile
  load_rows<D>(Qs, p.q + x.bb * p.sq[0] + x.hh * p.sq[1] + x.t0 * p.sq[2], p.sq[2]);
  load_rows<D>(Os, p.dO + x.bb * p.so[0] + x.hh * p.so[1] + x.t0 * p.so[2], p.so[2]);
  load_rows<D>(Ks, p.k + x.bb * p.sk[0] + x.hh * p.sk[1] + x.t0 * p.sk[2], p.sk[2]);
  load_rows<D>(Vs, p.v + x.bb * p.sv[0] + x.hh * p.sv[1] + x.t0 * p.sv[2], p.sv[2]);
  float gbeta = 0.f, gg = 0.f, gm = 0.f, gn = 0.f;
  if (w == 0) {
    const int64_t e = x.bh * p.T + x.t0 + l;
    gbeta = p.beta[e];
    gg = p.g[e];
    if constexpr (RULE >= 1) gm = p.gmu[e];
    if constexpr (RULE == 2) gn = p.gnu[e];
    float wt = gbeta;
    if constexpr (RULE == 1) {
      const float lm = fmaxf(gm, LOG_FLOOR);
      wt = expf(wave_sum(lm) - wave_incl_scan(lm));
    }
    if constexpr (RULE == 2) wt = 1.f;
    rb[l] = gbeta;
    rw[l] = wt;
  }
  __syncthreads();
  const int64_t mat = (int64_t)D * D;
  const float* S = p.S + x.si * mat;
  const float* dUv = p.dUv + x.si * mat;
  const float* dKw = p.dKw + x.si * mat;
  auto own = [&](const float* X) { return [=](int r, int k) { return X[(16 * tt + r) * LD + k]; }; };

  // ---- phase A, rows of tile tt: Z = V dUv (dK's w-term so far), E = V - K S^T, dQt = dO S,
  // the raw Q K^T tiles; dw accumulates k_t . (V dUv)_t
  f32x4 Z[NT], E[NT], dqt[NT], qk[NTT];
  float dwj[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    Z[tc] = mm16<D>(own(Vs), [&](int k, int c) { return dUv[k * D + 16 * tc + c]; }, zero4());
    const f32x4 ks = mm16<D>(own(Ks), [&](int k, int c) { return S[(16 * tc + c) * D + k]; }, zero4());
    dqt[tc] = mm16<D>(own(Os), [&](int k, int c) { return S[k * D + 16 * tc + c]; }, zero4());
    const f32x4 kt = ld_tile(Ks, LD, 16 * tt, 16 * tc);
    E[tc] = ld_tile(Vs, LD, 16 * tt, 16 * tc) - ks;
#pragma unroll
    for (int j = 0; j < 4; ++j) dwj[j] += Z[tc][j] * kt[j];
  }
#pragma unroll
  for (int st = 0; st < NTT; ++st)
    qk[st] = st <= tt ? mm16<D>(own(Qs), [&](int k, int c) { return Ks[(16 * st + c) * LD + k]; }, zero4())
                      : zero4();
  __syncthreads();  // every wave has read its V rows: E takes their place
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) st_tile(Vs, LD, 16 * tt, 16 * tc, E[tc]);
  __syncthreads();

  // ---- dA = tril(dO E^T) for rows of tile tt; dbeta's (q_t . k_s) term
  f32x4 dA[NTT];
#pragma unroll
  for (int st = 0; st < NTT; ++st) {
    dA[st] = zero4();
    float pb = 0.f;
    if (st <= tt) {
      dA[st] = mm16<D>(own(Os), [&](int k, int c) { return Vs[(16 * st + c) * LD + k]; }, zero4());
      const int s = 16 * st + lc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (s > 16 * tt + 4 * G + j) dA[st][j] = 0.f;
        pb += dA[st][j] * qk[st][j];
      }
    }
    pb = group_sum(pb);
    if (G == 0) pdb[tt * C + 16 * st + lc] = pb;
  }
  __syncthreads();  // E is read: A and dA diag(beta) take its place
#pragma unroll
  for (int st = 0; st < NTT; ++st) {
    const float bs = rb[16 * st + lc];
    f32x4 a = zero4(), ab = zero4();
    if (st <= tt) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a[j] = 16 * st + lc <= 16 * tt + 4 * G + j ? qk[st][j] * bs : 0.f;
        ab[j] = dA[st][j] * bs;
      }
    }
    st_tile(As, LDC, 16 * tt, 16 * st, a);
    st_tile(Abs, LDC, 16 * tt, 16 * st, ab);
  }
  __syncthreads();

  // ---- dQ = dQt + (dA diag(beta)) K; Z += K (dKw + dKw^T); Y3 = K dUv^T
  float* dqg = p.dq + x.bb * p.sq[0] + x.hh * p.sq[1] + x.t0 * p.sq[2];
  f32x4 Y3[NT];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    const f32x4 dq = mm16<C>([&](int r, int k) { return Abs[(16 * tt + r) * LDC + k]; },
                             [&](int k, int c) { return Ks[k * LD + 16 * tc + c]; }, dqt[tc]);
#pragma unroll
    for (int j = 0; j < 4; ++j) dqg[(int64_t)(16 * tt + 4 * G + j) * p.sq[2] + 16 * tc + lc] = dq[j];
    const f32x4 y2 = mm16<D>(own(Ks), [&](int k, int c) { return dKw[k * D + 16 * tc + c] + dKw[(16 * tc + c) * D + k]; },
                             zero4());
    const f32x4 kt = ld_tile(Ks, LD, 16 * tt, 16 * tc);
#pragma unroll
    for (int j = 0; j < 4; ++j) dwj[j] += 0.5f * y2[j] * kt[j];  // k^T dKw k = k^T (dKw + dKw^T) k / 2
    Z[tc] += y2;
    Y3[tc] = mm16<D>(own(Ks), [&](int k, int c) { return dUv[(16 * tc + c) * D + k]; }, zero4());
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float s = row16_sum(dwj[j]);
    if (lc == 0) rdw[16 * tt + 4 * G + j] = s;
  }
  __syncthreads();  // K is read: dQt takes its place
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) st_tile(Ks, LD, 16 * tt, 16 * tc, dqt[tc]);
  __syncthreads();

  // ---- phase B, rows s of tile tt: dK = -A^T dQt + (dA diag(beta))^T Q + diag(w) Z,
  // dV = A^T dO + diag(w) Y3
  float* dkg = p.dk + x.bb * p.sk[0] + x.hh * p.sk[1] + x.t0 * p.sk[2];
  float* dvg = p.dv + x.bb * p.sv[0] + x.hh * p.sv[1] + x.t0 * p.sv[2];
  float wr[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) wr[j] = rw[16 * tt + 4 * G + j];
#pragma unroll
  for (int tc = 0; tc < NT; ++tc) {
    f32x4 dk, dv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      dk[j] = wr[j] * Z[tc][j];
      dv[j] = wr[j] * Y3[tc][j];
    }
    dk = mm16<C>([&](int r, int k) { return Abs[k * LDC + 16 * tt + r]; },
                 [&](int k, int c) { return Qs[k * LD + 16 * tc + c]; }, dk);
    dk = mm16<C>([&](int r, int k) { return -As[k * LDC + 16 * tt + r]; },
                 [&](int k, int c) { return Ks[k * LD + 16 * tc + c]; }, dk);
    dv = mm16<C>([&](int r, int k) { return As[k * LDC + 16 * tt + r]; },
                 [&](int k, int c) { return Os[k * LD + 16 * tc + c]; }, dv);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t t = 16 * tt + 4 * G + j;
      dkg[t * p.sk[2] + 16 * tc + lc] = dk[j];
      dvg[t * p.sv[2] + 16 * tc + lc] = dv[j];
    }
  }

  // ---- gate gradients (lanes = tokens)
  if (w == 0) {
    const int64_t o = x.bh * p.T + x.t0 + l;
    const int64_t BHN = p.B * p.H * p.N;
    const float da = p.dsc[x.si], db = p.dsc[BHN + x.si];
    float dbeta = db * (1.f / C);  // b = mean(beta)
#pragma unroll
    for (int q = 0; q < F_WAVES; ++q) dbeta += pdb[q * C + l];
    if constexpr (RULE == 0) dbeta += rdw[l];  // w = beta
    p.dbeta[o] = dbeta;
    const float a = expf(wave_sum(fmaxf(gg, LOG_FLOOR)));
    p.dg[o] = gg >= LOG_FLOOR ? da * a : 0.f;
    if constexpr (RULE >= 1) {
      const float dm = p.dsc[2 * BHN + x.si];
      const float m = expf(wave_sum(fmaxf(gm, LOG_FLOOR)));
      float dl = dm * m;
      if constexpr (RULE == 1) {
        // w_s = exp(sum_{u > s} log mu_u): d w_s / d log mu_t = w_s for s < t
        const float y = rdw[l] * rw[l];
        dl += wave_incl_scan(y) - y;
      }
      p.dgmu[o] = gm >= LOG_FLOOR ? dl : 0.f;
    }
    if constexpr (RULE == 2) {
      const float dn = p.dsc[3 * BHN + x.si];
      const float n = expf(wave_sum(fmaxf(gn, LOG_FLOOR)));
      p.dgnu[o] = gn >= LOG_FLOOR ? dn * n : 0.f;
    }
  }
}

F32Args f32_args(const ChunkArgs& a) {
  F32Args f{};
  f.q = reinterpret_cast<const float*>(a.q);
  f.k = reinterpret_cast<const float*>(a.k);
  f.v = reinterpret_cast<const float*>(a.v);
  f.beta = a.beta;
  f.g = a.g;
  f.gmu = a.gmu;
  f.gnu = a.gnu;
  f.B = a.B;
  f.H = a.H;
  f.T = a.T;
  f.N = a.N;
  for (int i = 0; i < 3; ++i) {
    f.sq[i] = a.sq[i];
    f.sk[i] = a.sk[i];
    f.sv[i] = a.sv[i];
    f.so[i] = a.so[i];
  }
  return f;
}

template <class K>
hipError_t launch(K kern, int bytes, int64_t grid, const F32Args& f, hipStream_t s) {
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(F_THREADS), bytes, s, f);
  return hipGetLastError();
}

int planes_of(int rule) { return 1 + (rule >= 1) + (rule == 2); }  // S [, M] [, V]

template <int D>
hipError_t fwd_d(const ChunkArgs& a, int rule, int ns, float* states, hipStream_t s) {
  using L = F32Lds<D>;
  F32Args f = f32_args(a);
  f.o = reinterpret_cast<float*>(a.o);
  const int64_t BH = a.B * a.H, BHN = BH * a.N, mat = (int64_t)D * D, grid = BHN;
  const int P = planes_of(rule);
  float* S = states;
  f.Kw = states + P * BHN * mat;
  f.Uv = f.Kw + BHN * mat;
  f.abmn = f.Uv + BHN * mat;
  f.S = S;
  hipError_t e = rule == 0   ? launch(f32_prep<D, 0>, L::PREP_BYTES, grid, f, s)
                 : rule == 1 ? launch(f32_prep<D, 1>, L::PREP_BYTES, grid, f, s)
                             : launch(f32_prep<D, 2>, L::PREP_BYTES, grid, f, s);
  if (e != hipSuccess) return e;
  ScanArgs sa{};
  sa.U = f.Uv;
  sa.K = f.Kw;
  sa.a = f.abmn;
  sa.b = f.abmn + BHN;
  sa.m = f.abmn + 2 * BHN;
  sa.n = f.abmn + 3 * BHN;
  sa.S_all = S;
  sa.M_all = rule >= 1 ? S + BHN * mat : nullptr;
  sa.V_all = rule == 2 ? S + 2 * BHN * mat : nullptr;
  sa.BH = BH;
  sa.N = a.N;
  sa.dh = D;
  sa.rule = rule;
  sa.ns = ns;
  sa.precision = GMDN_PREC_IEEE;
  sa.stream = s;
  e = rule == 1 ? scan_fwd_muon_launch(sa) : scan_fwd_rows_launch(sa);
  if (e != hipSuccess) return e;
  return launch(f32_out<D>, L::OUT_BYTES, grid, f, s);
}

template <int D>
hipError_t bwd_d(const ChunkArgs& a, int rule, int ns, const float* states, float* ws, size_t ws_floats,
                 hipStream_t s) {
  using L = F32Lds<D>;
  F32Args f = f32_args(a);
  f.dO = reinterpret_cast<const float*>(a.o);
  const int64_t BH = a.B * a.H, BHN = BH * a.N, mat = (int64_t)D * D, grid = BHN;
  const int P = planes_of(rule);
  const float* S = states;
  const float* Kw = states + P * BHN * mat;
  const float* Uv = Kw + BHN * mat;
  const float* abmn = Uv + BHN * mat;
  f.S = S;
  f.gS = ws;
  float* dU = ws + BHN * mat;
  float* dK = ws + 2 * BHN * mat;
  float* dsc = ws + 3 * BHN * mat;
  float* part = dsc + 4 * BHN;
  const int64_t part_floats = (int64_t)ws_floats - (3 * BHN * mat + 4 * BHN);
  hipError_t e = launch(f32_gs<D>, L::GS_BYTES, grid, f, s);
  if (e != hipSuccess) return e;
  ScanArgs sa{};
  sa.U = Uv;
  sa.K = Kw;
  sa.a = abmn;
  sa.b = abmn + BHN;
  sa.m = abmn + 2 * BHN;
  sa.n = abmn + 3 * BHN;
  sa.S_all = const_cast<float*>(S);
  sa.M_all = rule >= 1 ? const_cast<float*>(S) + BHN * mat : nullptr;
  sa.V_all = rule == 2 ? const_cast<float*>(S) + 2 * BHN * mat : nullptr;
  sa.gS = f.gS;
  sa.dU = dU;
  sa.dK = dK;
  sa.da = dsc;
  sa.db = dsc + BHN;
  sa.dm = dsc + 2 * BHN;
  sa.dn = dsc + 3 * BHN;
  sa.BH = BH;
  sa.N = a.N;
  sa.dh = D;
  sa.rule = rule;
  sa.ns = ns;
  sa.precision = GMDN_PREC_IEEE;
  sa.stream = s;
  e = rule == 1 ? scan_bwd_muon_launch(sa, part, part_floats) : scan_bwd_rows_launch(sa, part);
  if (e != hipSuccess) return e;
  if ((e = scan_bwd_dk_launch(sa, part)) != hipSuccess) return e;
  f.dKw = dK;
  f.dUv = dU;
  f.dsc = dsc;
  f.dq = reinterpret_cast<float*>(a.dq);
  f.dk = reinterpret_cast<float*>(a.dk);
  f.dv = reinterpret_cast<float*>(a.dv);
  f.dbeta = a.dbeta;
  f.dg = a.dg;
  f.dgmu = a.dgmu;
  f.dgnu = a.dgnu;
  return rule == 0   ? launch(f32_tok<D, 0>, L::TOK_BYTES, grid, f, s)
         : rule == 1 ? launch(f32_tok<D, 1>, L::TOK_BYTES, grid, f, s)
                     : launch(f32_tok<D, 2>, L::TOK_BYTES, grid, f, s);
}

}  // namespace

size_t chunk_f32_states_floats(int64_t BH, int64_t N, int d, int rule) {
  // S [, M] [, V] of every chunk, Kw, Uv, then a, b, m, n
  return (size_t)((planes_of(rule) + 2) * BH * N * (int64_t)d * d + 4 * BH * N);
}

size_t chunk_f32_bwd_ws_floats(int64_t BH, int64_t N, int d, int rule, int ns) {
  // gS, dU, dK, the four scalar gradients, then the drop-in backward's workspace
  const int64_t BHN = BH * N, mat = (int64_t)d * d;
  int64_t scan = 0;
  if (rule == 2) scan = BHN * (d / 16) * 4;
  if (rule == 1) scan = BH * muon_bwd_ws_floats(d, ns);
  return (size_t)(3 * BHN * mat + 4 * BHN + scan);
}

hipError_t chunk_fwd_f32_launch(const ChunkArgs& a, int d, int rule, int ns, float* states, hipStream_t s) {
  switch (d) {
    case 32: return fwd_d<32>(a, rule, ns, states, s);
    case 64: return fwd_d<64>(a, rule, ns, states, s);
    case 128: return fwd_d<128>(a, rule, ns, states, s);
  }
  return hipErrorInvalidValue;
}

hipError_t chunk_bwd_f32_launch(const ChunkArgs& a, int d, int rule, int ns, const float* states, float* ws,
                                size_t ws_floats, hipStream_t s) {
  switch (d) {
    case 32: return bwd_d<32>(a, rule, ns, states, ws, ws_floats, s);
    case 64: return bwd_d<64>(a, rule, ns, states, ws, ws_floats, s);
    case 128: return bwd_d<128>(a, rule, ns, states, ws, ws_floats, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace gmdn
