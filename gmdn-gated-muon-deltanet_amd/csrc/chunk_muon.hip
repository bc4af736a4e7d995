// Level B, muon rule: the mixer core (reference train_ablation.py:142-187
// with the scan of fast_scan.py:86-88) for rule 1, in two kernels.
//
// chunk_fwd_muon: one workgroup of D/16 waves per (b, h) carries S and the
// momentum M of its head through the chunks (wave w keeps rows 16w.. of both
// as D-layout tiles of the transposes, as the drop-in muon scan does).  Per
// chunk only the k and v tiles and the gate rows stream in; the chunk's
// update is formed in the E-form
//     N = K S^T - V  (= -E),   G = E^T diag(w) K,   w_t = prod_{s > t} mu_s,
// without materialising the reference's Kw = K^T diag(w) K and
// Uv = V^T diag(w) K (train_ablation.py:164-165); then
//     M <- m M + G,  S <- a S + b msign_ns(M)
// with the Newton-Schulz steps of the shared split-bf16 engine (ns.h).  The
// pre-update S_i and M_i of every chunk are written (float32, (B, H, N, d, d))
// for the output kernel and the backward.
//
// chunk_out: chunk-parallel, one workgroup per (b, h, chunk):
//     o = Q S_i^T + A E,   A = tril(Q K^T) diag(beta),   E = V - K S_i^T
// (== (Q - A K) S_i^T + A V, train_ablation.py:166-167, :186).
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"
#include "ns.h"

namespace gmdn {

template <int D>
struct MuonFwdLds {
  static constexpr uint32_t TILE = CB_C * D * 2;           // one k or v chunk (bytes)
  static constexpr uint32_t XM = 0;                        // Newton-Schulz X planes
  static constexpr uint32_t PM = NSSplit<D>::BYTES;        // Newton-Schulz P planes
  static constexpr uint32_t K0 = 2 * NSSplit<D>::BYTES;    // k tile of the chunk
  static constexpr uint32_t V0 = K0 + TILE;                // v tile of the chunk
  static constexpr uint32_t BYTES = V0 + TILE;
  // inside the X planes, free from a chunk's last Newton-Schulz step to the
  // next chunk's first publish: per-wave token weights, block-sum partials
  static constexpr uint32_t W0 = 0;                        // [waves][64] float
  static constexpr uint32_t RED0 = (D / 16) * CB_C * 4;    // [waves] float
  static_assert(RED0 + 64 <= NSSplit<D>::BYTES, "scratch fits the X planes");
  static_assert(BYTES <= 160 * 1024, "muon forward LDS exceeds the 160 KiB of a CU");
};

// Inclusive prefix sum over the 64 lanes.
GMDN_DEV float wave_prefix_sum(float x) {
  const int l = lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float y = __shfl_up(x, o, 64);
    if (l >= o) x += y;
  }
  return x;
}

template <int D>
__global__ void __launch_bounds__(D * 4) chunk_fwd_muon(ChunkArgs p, float* __restrict__ S_out,
                                                       float* __restrict__ M_out, int ns) {
  using LQ = BSwz<D>;
  using L = MuonFwdLds<D>;
  using NSX = NSSplit<D>;
  constexpr int NT = D / 16, NKB = D / 32, NW = D / 16, NTHR = D * 4;
  extern __shared__ __align__(16) char smem[];
  const lds_ptr base = lds_base(smem);
  const bf16* Ks = reinterpret_cast<const bf16*>(smem + L::K0);
  const bf16* Vs = reinterpret_cast<const bf16*>(smem + L::V0);
  float* const wsl = reinterpret_cast<float*>(smem + L::W0) + wave_id() * CB_C;  // this wave's w[64]
  float* const red = reinterpret_cast<float*>(smem + L::RED0);

  const int64_t bh = blockIdx.x;
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const int w = wave_id(), l = lane_id(), G = l >> 4, lc = l & 15;
  const int r0 = 16 * w;
  const int64_t mat = (int64_t)D * D;
  const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
  const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1];
  const float* betag = p.beta + bh * p.T;
  const float* gg = p.g + bh * p.T;
  const float* mug = p.gmu + bh * p.T;
  const uint32_t lds0 = lds_addr(smem);

  DmaPlan<LQ, CB_C, NTHR> dk, dv;
  dk.init(w, p.sk[2]);
  dv.init(w, p.sv[2]);
  auto issue_tiles = [&](int i) {
    const int64_t t0 = (int64_t)i * CB_C;
    dk.issue(kg + t0 * p.sk[2], lds0 + L::K0, w);
    dv.issue(vg + t0 * p.sv[2], lds0 + L::V0, w);
  };

  const NSX nsx;
  f32x4 S[NT], M[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) S[t] = M[t] = zero4();

  // gate rows of a chunk, lane l <-> token l
  float gb = 0.f, ga = 0.f, gm = 0.f;
  auto load_gates = [&](int i) {
    const int64_t e = (int64_t)i * CB_C + l;
    gb = betag[e];
    ga = gg[e];
    gm = mug[e];
  };
  if (p.N > 0) {
    issue_tiles(0);
    load_gates(0);
  }

  for (int i = 0; i < p.N; ++i) {
    const int64_t si = bh * p.N + i;
    // everything issued during the previous chunk has had its Newton-Schulz
    // steps to land: chunk i's tiles and gate rows, the previous checkpoint
    wait_vmem();
    // ---- chunk scalars and token weights (every wave, redundantly; lane <-> token)
    const float lg = fmaxf(ga, LOG_FLOOR), lm = fmaxf(gm, LOG_FLOOR);
    const float a = expf(wave_sum(lg));
    const float b = wave_sum(gb) * (1.f / CB_C);
    const float msum = wave_sum(lm);
    const float m = expf(msum);
    // w_t = exp(sum_{s > t} log mu_s) (train_ablation.py:154-156)
    wsl[l] = expf(msum - wave_prefix_sum(lm));
    __syncthreads();  // every wave's tile copies visible; the weights written
    if (i + 1 < p.N) load_gates(i + 1);
    // ---- the pre-update state and momentum of chunk i
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t o = si * mat + (int64_t)(r0 + lc) * D + 16 * t + 4 * G;
      *reinterpret_cast<f32x4*>(S_out + o) = S[t];
      if (M_out) *reinterpret_cast<f32x4*>(M_out + o) = M[t];
    }
    // ---- N = K S^T - V = -E for all 64 tokens, the wave's 16 rows (lane <-> row)
    Op<2> Sop[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sop[kb] = pack_tiles<2>(S[2 * kb], S[2 * kb + 1]);
    f32x4 Nt[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) Nt[tt] = -b_dtile<LQ>(Vs, 16 * tt, r0);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) Nt[tt] = mma<1, 2>(Op<1>{{b_row<LQ>(Ks, 16 * tt, 32 * kb)}}, Sop[kb], Nt[tt]);
    // ---- G^T tiles = sum_t K[t][c] (w_t E[t][r]): B operand -w N over tokens
    Op<2> WN[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(wsl + 32 * kt + 4 * G);
      const f32x4 w1 = *reinterpret_cast<const f32x4*>(wsl + 32 * kt + 16 + 4 * G);
      WN[kt] = pack_tiles<2>(-(w0 * Nt[2 * kt]), -(w1 * Nt[2 * kt + 1]));
    }
    float sq = 0.f;
#pragma unroll
    for (int tc = 0; tc < NT; ++tc) {
      f32x4 g = zero4();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) g = mma<1, 2>(Op<1>{{b_col<LQ>(Ks, 32 * kt, 16 * tc)}}, WN[kt], g);
      M[tc] = m * M[tc] + g;
      sq += M[tc][0] * M[tc][0] + M[tc][1] * M[tc][1] + M[tc][2] * M[tc][2] + M[tc][3] * M[tc][3];
    }
    // the block sum's first barrier retires every wave's reads of the tiles:
    // the next chunk's copies go in behind it and land during the steps
    const float nrm = sqrtf(block_sum<NW>(sq, red));
    if (i + 1 < p.N) issue_tiles(i + 1);
    const float scale = 1.f / (nrm + 1e-7f);
    f32x4 X[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) X[t] = M[t] * scale;
    for (int s = 0; s < ns; ++s) nsx.step(X, base + L::XM, base + L::PM);
    if (ns == 0) __syncthreads();  // the scratch in the X planes is rewritten next chunk
#pragma unroll
    for (int t = 0; t < NT; ++t) S[t] = a * S[t] + b * X[t];
  }
}

// ------------------------------------------------------------------ output
template <int D>
struct OutLds {
  static constexpr uint32_t TILE = CB_C * D * 2;
  static constexpr uint32_t Q0 = 0, K0 = TILE, V0 = 2 * TILE;
  static constexpr uint32_t AP = CB_C * CB_C * 2;             // one -A plane
  static constexpr uint32_t A0 = 3 * TILE;                    // -A hi plane, then lo
  static constexpr uint32_t B0 = A0 + 2 * AP;                 // beta of the chunk
  static constexpr uint32_t BYTES = B0 + CB_C * 4;
};

template <int D>
__global__ void __launch_bounds__(D * 4) chunk_out(ChunkArgs p, const float* __restrict__ Sst) {
  using LQ = BSwz<D>;
  using LA = BSwz<CB_C>;
  using L = OutLds<D>;
  constexpr int NKB = D / 32, NW = D / 16, NTHR = D * 4;
  extern __shared__ __align__(16) char smem[];
  const bf16* Qs = reinterpret_cast<const bf16*>(smem + L::Q0);
  const bf16* Ks = reinterpret_cast<const bf16*>(smem + L::K0);
  const bf16* Vs = reinterpret_cast<const bf16*>(smem + L::V0);
  bf16* Ahi = reinterpret_cast<bf16*>(smem + L::A0);
  bf16* Alo = reinterpret_cast<bf16*>(smem + L::A0 + L::AP);
  float* bet = reinterpret_cast<float*>(smem + L::B0);

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const int w = wave_id(), l = lane_id(), G = l >> 4, lc = l & 15;
  const int r0 = 16 * w;
  const int64_t t0 = (int64_t)i * CB_C;
  {
    DmaPlan<LQ, CB_C, NTHR> pq, pk, pv;
    pq.init(w, p.sq[2]);
    pk.init(w, p.sk[2]);
    pv.init(w, p.sv[2]);
    const uint32_t lds0 = lds_addr(smem);
    pq.issue(p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2], lds0 + L::Q0, w);
    pk.issue(p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], lds0 + L::K0, w);
    pv.issue(p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2], lds0 + L::V0, w);
  }
  float bv = 0.f;
  if (threadIdx.x < CB_C) bv = p.beta[bh * p.T + t0 + threadIdx.x];
  // rows r0 + lc of S_i as split operands, columns in pair order
  const float* srow = Sst + (bh * p.N + i) * (int64_t)D * D + (int64_t)(r0 + lc) * D;
  Op<2> Sop[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(srow + 32 * kb + 4 * G);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(srow + 32 * kb + 16 + 4 * G);
    Sop[kb] = pack_tiles<2>(x0, x1);
  }
  wait_vmem();
  if (threadIdx.x < CB_C) bet[threadIdx.x] = bv;
  __syncthreads();

  // -A^T tiles: tile k = 4 tt + st (t = 16 tt + .., s = 16 st + ..) by wave k % NW;
  // lane (t, G) holds (K Q^T)[s = 16 st + 4G + j][t]; above the diagonal: zeros
#pragma unroll
  for (int kk = 0; kk < 16 / NW; ++kk) {
    const int k = w + NW * kk, tt = k >> 2, st = k & 3;
    bf16x4 hi4, lo4;
    if (tt < st) {
      hi4 = lo4 = bf16x4{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
    } else {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        acc = mfma(b_row<LQ>(Ks, 16 * st, 32 * kb), b_row<LQ>(Qs, 16 * tt, 32 * kb), acc);
      const f32x4 bs = *reinterpret_cast<const f32x4*>(bet + 16 * st + 4 * G);
      f32x4 val;
#pragma unroll
      for (int j = 0; j < 4; ++j) val[j] = (st < tt || 4 * G + j <= lc) ? -acc[j] * bs[j] : 0.f;
      split4(val, hi4, lo4);
    }
    const int ao = LA::off(16 * tt + lc, 16 * st + 4 * G);
    *reinterpret_cast<bf16x4*>(Ahi + ao) = hi4;
    *reinterpret_cast<bf16x4*>(Alo + ao) = lo4;
  }
  // N = K S^T - V = -E (lane <-> state row r0 + lc)
  f32x4 Nt[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) Nt[tt] = -b_dtile<LQ>(Vs, 16 * tt, r0);
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) Nt[tt] = mma<1, 2>(Op<1>{{b_row<LQ>(Ks, 16 * tt, 32 * kb)}}, Sop[kb], Nt[tt]);
  Op<2> Nop[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) Nop[ks] = pack_tiles<2>(Nt[2 * ks], Nt[2 * ks + 1]);
  __syncthreads();  // -A published
  // o^T tiles (rows r, lane <-> token): S Q^T + (-E)^T (-A)^T
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2] + r0 + 4 * G;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    f32x4 O = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) O = mma<2, 1>(Sop[kb], Op<1>{{b_row<LQ>(Qs, 16 * tt, 32 * kb)}}, O);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (32 * ks > 16 * tt + 15) continue;
      const Op<2> Ar{{b_row<LA>(Ahi, 16 * tt, 32 * ks), b_row<LA>(Alo, 16 * tt, 32 * ks)}};
      O = mma<2, 2>(Nop[ks], Ar, O);
    }
    // lane (t, G): o[16 tt + t][r0 + 4G .. +3]
    *reinterpret_cast<bf16x4*>(og + (16 * tt + lc) * p.so[2]) =
        to_bf16x4(O);
  }
}

template <int D>
static hipError_t launch_muon(const ChunkArgs& a, float* S_out, float* M_out, int ns, hipStream_t s) {
  auto kf = chunk_fwd_muon<D>;
  auto ko = chunk_out<D>;
  const int lf = MuonFwdLds<D>::BYTES, lo = OutLds<D>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize, lf);
  if (e == hipSuccess) e = hipFuncSetAttribute((const void*)ko, hipFuncAttributeMaxDynamicSharedMemorySize, lo);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kf, dim3((unsigned)(a.B * a.H)), dim3(D * 4), lf, s, a, S_out, M_out, ns);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ko, dim3((unsigned)(a.B * a.H * a.N)), dim3(D * 4), lo, s, a, (const float*)S_out);
  return hipGetLastError();
}

hipError_t chunk_out_launch(const ChunkArgs& a, int d, const float* S_all, hipStream_t s) {
  if (d == 128 || d == 64) {
    auto ko = d == 128 ? chunk_out<128> : chunk_out<64>;
    const int lo = d == 128 ? OutLds<128>::BYTES : OutLds<64>::BYTES;
    hipError_t e = hipFuncSetAttribute((const void*)ko, hipFuncAttributeMaxDynamicSharedMemorySize, lo);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(ko, dim3((unsigned)(a.B * a.H * a.N)), dim3(d * 4), lo, s, a, S_all);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

hipError_t chunk_fwd_muon_launch(const ChunkArgs& a, int d, float* S_out, float* M_out, int ns, hipStream_t s) {
  if (d == 128) return launch_muon<128>(a, S_out, M_out, ns, s);
  if (d == 64) return launch_muon<64>(a, S_out, M_out, ns, s);
  return hipErrorInvalidValue;
}

}  // namespace gmdn
