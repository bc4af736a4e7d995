// Level B: the fused mixer core, phases 1-3 of the reference mixer
// (train_ablation.py:142-187) in one kernel per direction.
//
// E-form (substituting train_ablation.py:164-167 into :186 and
// fast_scan.py:82), per (b, h) and chunk i with state S_i (d_v x d_k, fp32):
//   A   = tril(Q K^T) diag(beta)            (diagonal kept, :161-163)
//   E   = V - K S_i^T                        (per-token errors vs frozen S_i)
//   o   = Q S_i^T + A E                      (== (Q - A K) S_i^T + A V)
//   G   = E^T diag(w) K                      (== Uv - S_i Kw)
//   delta: S_{i+1} = a S_i + G
//   adam : M <- m M + (1-m) G ; V <- n V + (1-n) G^2 ;
//          S_{i+1} = a S_i + b M / (sqrt(V) + eps)
// with a = exp(sum max(g, log 1e-6)), b = mean beta, m, n likewise
// (train_ablation.py:150-158, :169-175).  Only q, k, v, beta and the
// log-gates stream from HBM; o streams out; S stays in registers.
//
// The delta rule's forward runs chunk_fwd_rows (csrc/chunk_fwd_rows.hip),
// adam's at d = 64 chunk_fwd_adam16 (csrc/chunk_fwd_adam.hip); the kernel
// below serves adam at d = 128.
// Work split (forward).  A workgroup of 4 waves owns 32 rows of S for the
// whole sequence; wave (rt, h) owns row tile rt (16 rows) and column half h
// of S, the token half h of E and of o, and the column half h of G.  Two LDS
// exchanges per chunk hand each wave its partner's half of the packed
// S^T and E operands.  All products with a computed (fp32) factor use split
// bf16 operands (hi + lo, three MFMAs; two when the other factor is an exact
// bf16 input): plain bf16 rounding of S, E or A costs ~1e-2 of RMS, which
// together with the bf16 output rounding exceeds 2e-2 of RMS at B=4, H=16,
// T=4096, d=128.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

#include <type_traits>

namespace gmdn {

// Roles.  The forward runs 8 waves per workgroup, two per SIMD: four state
// waves carry the recurrence (E, then G and the state update) and four
// output waves everything that hangs off it (the A tiles, o = Q S^T + A E,
// the o stores, the chunk's gate scalars and all LDS-DMA traffic), so the
// serial chain of each chunk holds only the recurrence's own products.
// Per chunk i:
//   state : [X_i] S_i^T operands, -E (token half h) -> XE   [Y_i]  G, update, S_{i+1} halves -> XS  [X_{i+1}]
//   output: [X_i] DMA chunk i+2, gate scalars, S_i^T operands,
//                 -A tiles -> A planes                     [Y_i]  o_i = Q S^T + A E, staged through
//                                                                 the chunk's (now dead) V slot, stored  [X_{i+1}]
constexpr int FW_WAVES = 8;
constexpr int FW_THREADS = 64 * FW_WAVES;

// LDS carve-up of the forward kernel (bytes)
// Chunk tiles (Q, K, the workgroup's 32 columns of V, and the gate chunk)
// live in a ring of RING LDS buffers filled by LDS-DMA RING - 1 chunks
// ahead, so HBM latency is covered by that many chunks of work.  The chunk
// loop is unrolled over the ring, so every LDS read address is a per-lane
// base register (computed once) plus an immediate offset.
template <int D>
struct FwdLds {
  static constexpr int NKBH = D / 64;            // k-blocks in a column half
  static constexpr int TILE = CB_C * D * 2;      // one Q or K chunk (bytes)
  static constexpr int VT = CB_C * 32 * 2;       // the workgroup's V columns
  static constexpr int GT = 4 * CB_C * 4;        // beta, g, gmu, gnu
  static constexpr int Q0 = 0;
  static constexpr int K0 = Q0 + RING * TILE;
  static constexpr int V0 = K0 + RING * TILE;
  static constexpr int G0 = V0 + RING * VT;
  static constexpr int A0 = G0 + RING * GT;        // -A hi plane, then lo plane
  static constexpr int AP = CB_C * CB_C * 2;
  static constexpr int XSP = 32 * D * 2;          // S exchange: [32 rows][D] bf16, hi plane then lo
  static constexpr int XS0 = A0 + 2 * AP;
  static constexpr int XEP = 32 * CB_C * 2;        // E exchange: [32 rows][64 tokens] bf16 planes
  static constexpr int XE0 = XS0 + 2 * XSP;        // N hi, N lo, -wN hi, -wN lo
  static constexpr int SC0 = XE0 + 4 * XEP;        // chunk scalars a, b, m, n per stage
  static constexpr int BYTES = SC0 + RING * 16;
  static_assert(BYTES <= 160 * 1024, "forward LDS exceeds the 160 KiB of a CU");
  // LDS-DMA instructions one output wave issues per chunk (Q, K, V; the
  // first output wave also the gates)
  static constexpr int DMA_OPS = 2 * (CB_C * D / 8) / CB_THREADS + (CB_C * 32 / 8) / CB_THREADS;
};

template <int D, int RULE>
__global__ void __launch_bounds__(FW_THREADS) chunk_fwd(ChunkArgs p) {
  using LQ = BSwz<D>;
  using LV = BSwz<32>;
  using LA = BSwz<CB_C>;
  using L = FwdLds<D>;
  constexpr int NKB = D / 32;   // k-blocks over the state's columns
  constexpr int NTH = D / 32;   // column tiles in a half
  constexpr int NKBH = L::NKBH;
  constexpr int ROWB = D * 2;   // bytes per Q/K row
  extern __shared__ __align__(16) char smem[];
  bf16* const Ahi = reinterpret_cast<bf16*>(smem + L::A0);
  bf16* const Alo = reinterpret_cast<bf16*>(smem + L::A0 + L::AP);

  int64_t bh;
  int blk;
  map_block(p.B * p.H, D / 32, bh, blk);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool state_wave = w < CB_WAVES;
  const int sw = w & (CB_WAVES - 1);  // index within the role
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int rt = sw >> 1, h = sw & 1;
  const int r0 = 32 * blk + 16 * rt;  // first state row of this wave
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
  const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
  const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + 32 * blk;
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + r0 + lc;
  // gate chunk: 16 lanes x 16 bytes each; lanes 0-15 beta, 16-31 g,
  // 32-47 gmu, 48-63 gnu (beta again where the rule has no such gate)
  const float* gsrc = (G == 0 ? p.beta : G == 1 ? p.g : G == 2 ? (RULE == 2 ? p.gmu : p.beta)
                                                               : (RULE == 2 ? p.gnu : p.beta)) +
                      bh * p.T + 4 * lc;

  // ---- per-lane LDS byte offsets (stage, row-tile and k offsets are immediates)
  // Every MFMA operand is read in natural k order: lane (m, G) takes
  // X[m][k0 + 8G .. k0 + 8G + 7] in one 16-byte read, or (column operands)
  // X[k0 + 8G .. k0 + 8G + 7][c] in two transposing reads.  The exchanges
  // between waves are row-major matrices in LDS, so no operand needs a
  // register shuffle.
  using LX = BSwz<CB_C>;  // E exchange planes (64 token columns)
  uint32_t rowb[NKB];     // row lc of a 16-row tile, columns 32 kb + 8G
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) rowb[kb] = swz_off<LQ>(lc, 32 * kb + 8 * G);
  // transposing reads of K columns 16 ct + i for this wave's column tiles:
  // rows 8G + lc/4 (first read) and 8G + 4 + lc/4 (second)
  uint32_t kc0[NTH], kc1[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) {
    kc0[t] = swz_off<LQ>(8 * G + (lc >> 2), 16 * (h * NTH + t) + 4 * (lc & 3));
    kc1[t] = swz_off<LQ>(8 * G + 4 + (lc >> 2), 16 * (h * NTH + t) + 4 * (lc & 3));
  }
  // transposing reads of V (rows 32h + 16u + 4G + lc/4, columns 16 rt + 4 (lc & 3))
  // (the row part 32h + 16u is added as an immediate: whole multiples of 4
  // rows leave the swizzle term unchanged; the column part 16 rt is not
  // additive under the XOR and stays in the base)
  const uint32_t voff = swz_off<LV>(4 * G + (lc >> 2), 16 * rt + 4 * (lc & 3));
  // row reads of -A (rows 32h + 16u + lc, columns 32 kbs + 8G)
  uint32_t aoff[2];
#pragma unroll
  for (int kbs = 0; kbs < 2; ++kbs) aoff[kbs] = swz_off<LA>(32 * h + lc, 32 * kbs + 8 * G);
  // S exchange: this state wave writes row 16 rt + lc, columns 16 (h NTH + t) + 4G
  uint32_t xsw[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) xsw[t] = swz_off<LQ>(16 * rt + lc, 16 * (h * NTH + t) + 4 * G);
  // E exchange: row 16 rt + lc; written at tokens 32h + 16u + 4G, read at 32 kbs + 8G
  uint32_t xew[2], xer[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    xew[u] = swz_off<LX>(16 * rt + lc, 32 * h + 16 * u + 4 * G);
    xer[u] = swz_off<LX>(16 * rt + lc, 32 * u + 8 * G);
  }
  // LDS pointers, one set per region, so that the stage, row-tile and k
  // offsets added inside the loop stay within the 16-bit immediate
  const uint32_t lds0 = lds_addr(smem);
  const lds_ptr L0 = lds_base(smem);
  lds_cptr qrow[NKB], krow[NKB], xsr[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    qrow[kb] = L0 + (rowb[kb] + L::Q0);
    krow[kb] = L0 + (rowb[kb] + L::K0);
    xsr[kb] = L0 + (rowb[kb] + L::XS0);
  }
  lds_cptr kcol0[NTH], kcol1[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) {
    kcol0[t] = L0 + (kc0[t] + L::K0);
    kcol1[t] = L0 + (kc1[t] + L::K0);
  }
  const lds_cptr vaddr = L0 + (voff + L::V0);
  lds_cptr ap[2];
#pragma unroll
  for (int kbs = 0; kbs < 2; ++kbs) ap[kbs] = L0 + (aoff[kbs] + L::A0);

  // the strictly-upper tiles of -A are never written: zero them once
  for (int e = threadIdx.x; e < CB_C * CB_C; e += FW_THREADS) {
    const int r = e / CB_C, c = e % CB_C;
    if ((c >> 4) > (r >> 4)) {
      Ahi[LA::off(r, c)] = (bf16)0.f;
      Alo[LA::off(r, c)] = (bf16)0.f;
    }
  }

  // LDS-DMA: issued by the output waves only (index sw among them)
  DmaPlan<LQ, CB_C, CB_THREADS> dq, dk;
  DmaPlan<LV, CB_C, CB_THREADS> dv;
  dq.init(sw, p.sq[2]);
  dk.init(sw, p.sk[2]);
  dv.init(sw, p.sv[2]);
  auto issue_loads = [&](int i, int stg) {
    const int64_t t0 = (int64_t)i * CB_C;
    dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + stg * L::TILE, sw);
    dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + stg * L::TILE, sw);
    dv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + stg * L::VT, sw);
    if (sw == 0) lds_dma16(gsrc + t0, smem + L::G0 + stg * L::GT);
  };

  // state waves: S (and adam's M, V) for row r0 + lc, columns of half h
  f32x4 S[NTH], Mm[NTH], Vv[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) S[t] = Mm[t] = Vv[t] = zero4();
  f32x4 O[2] = {zero4(), zero4()};  // output waves: o tiles of the chunk
  // split a D-layout tile into hi / lo bf16 and store both 8-byte pieces
  auto put_split = [&](uint32_t off, uint32_t plane, const f32x4& x) {
    bf16x4 hi, lo;
    split4(x, hi, lo);
    lds_st<bf16x4>(L0 + off, hi);
    lds_st<bf16x4>(L0 + (off + plane), lo);
  };
  // S_{i+1}^T half of this state wave -> the S exchange (row-major, split)
  auto publish_S = [&]() {
#pragma unroll
    for (int t = 0; t < NTH; ++t) put_split(xsw[t] + L::XS0, L::XSP, S[t]);
  };
  // split operand at a base pointer: hi plane, lo plane `plane` bytes later
  auto read_op = [&](lds_cptr addr, uint32_t plane) {
    Op<2> x;
    x.v[0] = lds_ld<bf16x8>(addr);
    x.v[1] = lds_ld<bf16x8>(addr + plane);
    return x;
  };
  // chunk scalars a = exp(sum max(g, log 1e-6)), and for adam b = mean(beta),
  // m, n: reduced by one output wave into the stage's scalar slot
  float* const scal = reinterpret_cast<float*>(smem + L::SC0);
  auto chunk_scalars = [&](int stg) {
    const float* gg = reinterpret_cast<const float*>(smem + L::G0 + stg * L::GT);
    const float a = expf(wave_sum(fmaxf(gg[CB_C + l], LOG_FLOOR)));
    float bs = 0.f, ms = 0.f, ns = 0.f;
    if constexpr (RULE == 2) {
      bs = wave_sum(gg[l]) * (1.f / CB_C);
      ms = expf(wave_sum(fmaxf(gg[2 * CB_C + l], LOG_FLOOR)));
      ns = expf(wave_sum(fmaxf(gg[3 * CB_C + l], LOG_FLOOR)));
    }
    if (l == 0) *reinterpret_cast<f32x4*>(scal + 4 * stg) = f32x4{a, bs, ms, ns};
  };

  if (state_wave) {
    publish_S();
  } else {
    for (int j = 0; j < RING - 1 && j < p.N; ++j) issue_loads(j, j);
    wait_vmem();
  }
  __syncthreads();  // X_0

  // one tile of -A^T = -(K Q^T) diag(beta), restricted to s <= t
  auto a_tile = [&](auto stg_tag, auto st_tag, auto tt_tag) {
    constexpr int STG = decltype(stg_tag)::value;
    constexpr uint32_t SQK = STG * L::TILE;
    const float* gates = reinterpret_cast<const float*>(smem + L::G0 + STG * L::GT);
    constexpr int st = decltype(st_tag)::value, tt = decltype(tt_tag)::value;
    bf16x8 ka[NKB], qa[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      ka[kb] = lds_ld<bf16x8>(krow[kb] + SQK + st * 16 * ROWB);
      qa[kb] = lds_ld<bf16x8>(qrow[kb] + SQK + tt * 16 * ROWB);
    }
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc = mfma(ka[kb], qa[kb], acc);
    // lane (t, G) holds (Q K^T)[t][s] for s = 16 st + 4G + j
    const f32x4 bs = *reinterpret_cast<const f32x4*>(gates + 16 * st + 4 * G);
    f32x4 val;
#pragma unroll
    for (int j = 0; j < 4; ++j) val[j] = (st < tt || 4 * G + j <= lc) ? -acc[j] * bs[j] : 0.f;
    bf16x4 hi4, lo4;
    split4(val, hi4, lo4);
    const int ao = LA::off(16 * tt + lc, 16 * st + 4 * G);
    *reinterpret_cast<bf16x4*>(Ahi + ao) = hi4;
    *reinterpret_cast<bf16x4*>(Alo + ao) = lo4;
  };

  // One chunk of each role; STG = i % RING is a compile-time constant.  The
  // roles run separate loops (so that the register allocator never holds
  // one role's loop state in the other's) with the same barrier sequence.
  auto state_chunk = [&](auto stg_tag, int i) {
    constexpr int STG = decltype(stg_tag)::value;
    constexpr uint32_t SQK = STG * L::TILE;  // stage offsets within the regions
    constexpr uint32_t VC = STG * L::VT;
    const float* gates = reinterpret_cast<const float*>(smem + L::G0 + STG * L::GT);
    const bool ahead = i + RING - 1 < p.N;
    using std::integral_constant;
    using I0 = integral_constant<int, 0>;
    using I1 = integral_constant<int, 1>;
    using I2 = integral_constant<int, 2>;
    using I3 = integral_constant<int, 3>;
    Op<2> Sop[NKB];  // S_i^T operands of every k-block (rows of this row tile)
    // ================= state, before Y_i: -E for this wave's tokens
    if constexpr (RULE == 2) {
      if (p.states) {  // adam's moments for the backward (S_i itself: the output waves)
        const int64_t plane = p.B * p.H * p.N * (int64_t)D * D;
        float* sp = p.states + ((bh * p.N + i) * D + r0 + lc) * (int64_t)D + 4 * G;
#pragma unroll
        for (int t = 0; t < NTH; ++t) {
          *reinterpret_cast<f32x4*>(sp + plane + 16 * (h * NTH + t)) = Mm[t];
          *reinterpret_cast<f32x4*>(sp + 2 * plane + 16 * (h * NTH + t)) = Vv[t];
        }
      }
    }
    auto segE = [&](auto rt_tag, auto h_tag) {
      constexpr int RT = decltype(rt_tag)::value, H = decltype(h_tag)::value;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Sop[kb] = read_op(xsr[kb] + RT * 16 * ROWB, L::XSP);
      // N = K S^T - V = -E for this wave's tokens 32H .. 32H+31 (two chains)
      f32x4 Nt[2];
      bf16x8 Kr[2][NKB];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const bf16x4 vb = lds_tr16(vaddr + (VC + (32 * H + 16 * u) * 64));
        Nt[u] = f32x4{-(float)vb[0], -(float)vb[1], -(float)vb[2], -(float)vb[3]};
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) Kr[u][kb] = lds_ld<bf16x8>(krow[kb] + SQK + (2 * H + u) * 16 * ROWB);
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) Nt[u] = mma<1, 2>(Op<1>{{Kr[u][kb]}}, Sop[kb], Nt[u]);
      // publish the E operands: N (for A E) and -w N (for G), w per token row
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const f32x4 bt = *reinterpret_cast<const f32x4*>(gates + 32 * H + 16 * u + 4 * G);
        const f32x4 wt = RULE == 0 ? -bt : f32x4{-1.f, -1.f, -1.f, -1.f};
        put_split(xew[u] + L::XE0, L::XEP, Nt[u]);
        put_split(xew[u] + L::XE0 + 2 * L::XEP, L::XEP, Nt[u] * wt);
      }
    };
    switch (sw) {
      case 0: segE(I0{}, I0{}); a_tile(stg_tag, I0{}, I0{}); break;
      case 1: segE(I0{}, I1{}); a_tile(stg_tag, I1{}, I1{}); break;
      case 2: segE(I1{}, I0{}); a_tile(stg_tag, I2{}, I2{}); break;
      default: segE(I1{}, I1{}); a_tile(stg_tag, I3{}, I3{}); break;
    }
    __syncthreads();  // Y_i: E halves and -A published
    // ================= state, after Y_i: G^T for this wave's column half, update
    Op<2> WE[2];
#pragma unroll
    for (int kbs = 0; kbs < 2; ++kbs) WE[kbs] = read_op(L0 + (xer[kbs] + L::XE0 + 2 * L::XEP), L::XEP);
    bf16x8 Kcol[NTH][2];
#pragma unroll
    for (int t = 0; t < NTH; ++t)
#pragma unroll
      for (int kbs = 0; kbs < 2; ++kbs) {
        Kcol[t][kbs] = cat8(lds_tr16(kcol0[t] + SQK + kbs * 32 * ROWB), lds_tr16(kcol1[t] + SQK + kbs * 32 * ROWB));
      }
    const f32x4 sc = *reinterpret_cast<const f32x4*>(scal + 4 * STG);
    const float a = sc[0], bsc = sc[1], msc = sc[2], nsc = sc[3];
    f32x4 acc[NTH];
#pragma unroll
    for (int t = 0; t < NTH; ++t) acc[t] = RULE == 0 ? a * S[t] : zero4();
#pragma unroll
    for (int kbs = 0; kbs < 2; ++kbs)
#pragma unroll
      for (int t = 0; t < NTH; ++t) acc[t] = mma<1, 2>(Op<1>{{Kcol[t][kbs]}}, WE[kbs], acc[t]);
#pragma unroll
    for (int t = 0; t < NTH; ++t) {
      if constexpr (RULE == 0) {
        S[t] = acc[t];
      } else {
        Mm[t] = msc * Mm[t] + (1.f - msc) * acc[t];
        Vv[t] = nsc * Vv[t] + (1.f - nsc) * acc[t] * acc[t];
#pragma unroll
        for (int j = 0; j < 4; ++j) S[t][j] = a * S[t][j] + bsc * Mm[t][j] * hw_rcp(hw_sqrt(Vv[t][j]) + p.eps);
      }
    }
    publish_S();  // S_{i+1}^T half, read after X_{i+1}
    __syncthreads();  // X_{i+1}: next chunk's tiles landed, S_{i+1} halves published
  };
  auto output_chunk = [&](auto stg_tag, int i) {
    constexpr int STG = decltype(stg_tag)::value;
    constexpr uint32_t SQK = STG * L::TILE;  // stage offsets within the regions
    constexpr uint32_t VC = STG * L::VT;
    const float* gates = reinterpret_cast<const float*>(smem + L::G0 + STG * L::GT);
    const bool ahead = i + RING - 1 < p.N;
    using std::integral_constant;
    using I0 = integral_constant<int, 0>;
    using I1 = integral_constant<int, 1>;
    using I2 = integral_constant<int, 2>;
    using I3 = integral_constant<int, 3>;
    Op<2> Sop[NKB];  // S_i^T operands of every k-block (rows of this row tile)
    // ================= output, before Y_i: DMA, gate scalars, S^T operands, -A tiles, Q S^T
    if (ahead) issue_loads(i + RING - 1, (STG + RING - 1) % RING);
    if (sw == 3) chunk_scalars(STG);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sop[kb] = read_op(xsr[kb] + rt * 16 * ROWB, L::XSP);
    // causal tiles (st, tt) of -A: the diagonal ones go to the state waves,
    // the rest to the output waves: {01 02}, {03 12}, {13}, {23}
    switch (sw) {
      case 0: a_tile(stg_tag, I0{}, I1{}); a_tile(stg_tag, I0{}, I2{}); break;
      case 1: a_tile(stg_tag, I0{}, I3{}); a_tile(stg_tag, I1{}, I2{}); break;
      case 2: a_tile(stg_tag, I1{}, I3{}); break;
      default: a_tile(stg_tag, I2{}, I3{}); break;
    }
    // o = Q S^T + (-A)(-E) for this wave's tokens; Q S^T needs no E: before Y_i
    auto qs = [&](auto h_tag) {
      constexpr int H = decltype(h_tag)::value;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        O[u] = zero4();
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
          O[u] = mma<2, 1>(Sop[kb], Op<1>{{lds_ld<bf16x8>(qrow[kb] + SQK + (2 * H + u) * 16 * ROWB)}}, O[u]);
      }
    };
    if (h == 0)
      qs(I0{});
    else
      qs(I1{});
    __syncthreads();  // Y_i: E halves and -A published
    // ================= output, after Y_i: the (-A)(-E) term
    Op<2> EN[2];
#pragma unroll
    for (int kbs = 0; kbs < 2; ++kbs) EN[kbs] = read_op(L0 + (xer[kbs] + L::XE0), L::XEP);
    auto ae = [&](auto h_tag) {
      constexpr int H = decltype(h_tag)::value;
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int kbs = 0; kbs <= H; ++kbs)
          O[u] = mma<2, 2>(EN[kbs], read_op(ap[kbs] + u * 16 * CB_C * 2, L::AP), O[u]);
    };
    if (h == 0)
      ae(I0{});
    else
      ae(I1{});
    // o for tokens 32h .. 32h+31, columns r0 .. r0+15: staged through this
    // wave's 1 KiB of the chunk's V slot (read only before Y_i, refilled
    // only after X_{i+1}) and stored as one 16-byte piece per lane.  Both
    // products above have their operands swapped, so O[u] is the transposed
    // tile: lane (t, G) holds token 16u + t, columns r0 + 4G .. r0 + 4G + 3.
    {
      bf16* stage = reinterpret_cast<bf16*>(smem + L::V0 + STG * L::VT) + sw * 512;
#pragma unroll
      for (int u = 0; u < 2; ++u)
        *reinterpret_cast<bf16x4*>(stage + (16 * u + lc) * 16 + 4 * G) =
            to_bf16x4(O[u]);
      const int tok = l >> 1, half = l & 1;  // lanes: 32 tokens x 2 pieces of 8 columns
      const bf16x8 piece = *reinterpret_cast<const bf16x8*>(stage + tok * 16 + 8 * half);
      *reinterpret_cast<bf16x8*>(og - lc + ((int64_t)i * CB_C + 32 * h + tok) * p.so[2] + 8 * half) = piece;
    }
    // the checkpoint of S_i for the backward, from the split operands this
    // wave holds (rows r0 .. r0+15, k-blocks of column half h), so that the
    // state waves never wait on vector memory.  The delta rule keeps the even
    // chunks only (plane i / 2): its backward rebuilds S_{i+1} on chip.
    constexpr int CK = NKB;  // 16-byte pieces per lane
    const bool ck = p.states && (RULE != 0 || (i & 1) == 0);
    if (ck) {
      const int64_t plane = RULE == 0 ? bh * ((p.N + 1) / 2) + i / 2 : bh * p.N + i;
      float* sp = p.states + (plane * D + r0 + lc) * (int64_t)D + 8 * G;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        if ((2 * kb >= NKB) != (h == 1)) continue;
        *reinterpret_cast<bf16x8*>(sp + 32 * kb) =
            __builtin_shufflevector(Sop[kb].v[0], Sop[kb].v[1], 0, 1, 2, 3, 8, 9, 10, 11);
        *reinterpret_cast<bf16x8*>(sp + 32 * kb + 4) =
            __builtin_shufflevector(Sop[kb].v[0], Sop[kb].v[1], 4, 5, 6, 7, 12, 13, 14, 15);
      }
    }
    // chunk i+1's tiles must have landed; the operations issued after them
    // (the loads for chunk i+RING-1, this chunk's o store and checkpoint
    // pieces) may stay in flight.  Vector memory operations complete in issue
    // order for this count: vmcnt <= (operations issued since) suffices.
    if (ahead) {
      if (ck) {
        if (sw == 0)
          wait_vmem_le<L::DMA_OPS + CK + 2>();
        else
          wait_vmem_le<L::DMA_OPS + CK + 1>();
      } else {
        if (sw == 0)
          wait_vmem_le<L::DMA_OPS + 2>();
        else
          wait_vmem_le<L::DMA_OPS + 1>();
      }
    } else {
      wait_vmem();
    }
    __syncthreads();  // X_{i+1}: next chunk's tiles landed, S_{i+1} halves published
  };
  auto run = [&](auto&& chunk) {
    for (int i = 0; i < p.N; i += RING) {
      chunk(std::integral_constant<int, 0>{}, i);
      if (i + 1 < p.N) chunk(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < p.N) chunk(std::integral_constant<int, 2>{}, i + 2);
    }
  };
  if (state_wave)
    run(state_chunk);
  else
    run(output_chunk);
}

template <int D, int RULE>
static hipError_t launch_fwd(const ChunkArgs& a, hipStream_t stream) {
  auto kern = chunk_fwd<D, RULE>;
  const int lds = FwdLds<D>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (D / 32);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(FW_THREADS), lds, stream, a);
  return hipGetLastError();
}

hipError_t chunk_fwd_launch(const ChunkArgs& a, int d, int rule, hipStream_t s) {
  // row-owned state waves: the delta rule, and adam at d = 64 (at d = 128
  // adam's three state tiles per row block exceed that kernel's registers)
  if (rule == 2 && d == 64) return chunk_fwd_adam16_launch(a, d, s);
  if (rule == 0) return chunk_fwd_rows_launch(a, d, rule, s);
  return launch_fwd<128, 2>(a, s);
}

}  // namespace gmdn

using namespace gmdn;

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_desc(const gmdn_chunk_desc* d) {
  if (!d) return GMDN_ERR_ARG;
  if (d->B < 0 || d->H < 0 || d->T < 0) return GMDN_ERR_ARG;
  if (d->rule < 0 || d->rule > 2 || d->ns < 0 || d->ns > 8) return GMDN_ERR_ARG;
  if (d->dtype != GMDN_DTYPE_BF16 && d->dtype != GMDN_DTYPE_F32) return GMDN_ERR_UNSUPPORTED;
  // bf16 streams: d = 64, 128; float32 streams (the matrix form): also 32
  const bool d_ok = d->d == 64 || d->d == 128 || (d->dtype == GMDN_DTYPE_F32 && d->d == 32);
  if (d->C != CB_C || !d_ok) return GMDN_ERR_UNSUPPORTED;
  if (d->T % CB_C != 0) return GMDN_ERR_ARG;
  if (d->B * d->H > ((int64_t)1 << 31) || d->T / CB_C > ((int64_t)1 << 30)) return GMDN_ERR_ARG;
  // DMA tiles need 16-byte aligned rows: token strides in multiples of 8 elements
  for (int i = 0; i < 3; ++i)
    if ((d->sq[i] & 7) || (d->sk[i] & 7) || (d->sv[i] & 7)) return GMDN_ERR_UNSUPPORTED;
  return GMDN_OK;
}

ChunkArgs make_args(const gmdn_chunk_desc* d, const void* q, const void* k, const void* v,
                    const float* beta, const float* g, const float* gmu, const float* gnu, void* o,
                    void* states) {
  ChunkArgs a{};
  a.q = (const bf16*)q;
  a.k = (const bf16*)k;
  a.v = (const bf16*)v;
  a.beta = beta;
  a.g = g;
  a.gmu = gmu;
  a.gnu = gnu;
  a.o = (bf16*)o;
  a.states = (float*)states;
  a.B = d->B;
  a.H = d->H;
  a.T = d->T;
  a.N = (int)(d->T / CB_C);
  a.eps = d->eps;
  for (int i = 0; i < 3; ++i) {
    a.sq[i] = d->sq[i];
    a.sk[i] = d->sk[i];
    a.sv[i] = d->sv[i];
    a.so[i] = d->so[i];
  }
  return a;
}

// d x d planes of Gb in the backward's workspace
size_t gb_planes(const gmdn_chunk_desc* desc) {
  const int64_t N = desc->T / CB_C;
  return (size_t)(desc->B * desc->H * (desc->rule == 0 ? N / 2 : N));
}

// the delta rule's and adam's (d = 64) backward workspace without the carry:
// Gb planes and the per-(chunk, row block) partial sums
size_t chunk_bwd_min_ws_bytes(const gmdn_chunk_desc* desc) {
  const size_t chunks = (size_t)(desc->B * desc->H * (desc->T / CB_C));
  return gb_planes(desc) * desc->d * desc->d * sizeof(float) + chunks * (desc->d / 16) * 4 * sizeof(float);
}

// adam at d = 64: Sb, Mb, Vb between the reverse scan's segments
size_t ascan_carry_bytes(const gmdn_chunk_desc* desc) {
  return desc->rule == 2 && desc->d == 64 ? (size_t)(desc->B * desc->H) * desc->d * desc->d * 3 * sizeof(float) : 0;
}

}  // namespace

extern "C" {

size_t gmdn_chunk_states_bytes(const gmdn_chunk_desc* desc) {
  if (check_desc(desc) != GMDN_OK) return 0;
  // delta: S_i of the even chunks (the backward rebuilds the odd ones);
  // muon: S_i and its momentum M_i, adam: S_i and the moments M_i, V_i, of
  // every chunk
  const int64_t N = desc->T / CB_C;
  if (desc->dtype == GMDN_DTYPE_F32)
    return chunk_f32_states_floats(desc->B * desc->H, N, desc->d, desc->rule) * sizeof(float);
  const size_t sq = (size_t)desc->d * desc->d * sizeof(float);
  if (desc->rule == 0) return (size_t)(desc->B * desc->H * ((N + 1) / 2)) * sq;
  // adam at d = 128 trains through the exact float32 scan: S, M, V, Kw, Uv
  // planes of every chunk and the chunk scalars
  if (desc->rule == 2 && desc->d == 128) return chunk_adam_mat_states_floats(desc->B * desc->H, N, desc->d) * 4;
  const size_t planes = desc->rule == 2 ? 3 : 2;
  return planes * (size_t)(desc->B * desc->H * N) * sq;
}

int gmdn_chunk_fwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v,
                   const float* beta, const float* g, const float* gmu, const float* gnu, void* o,
                   void* states, void* stream) {
  int rc = check_desc(desc);
  if (rc != GMDN_OK) return rc;
  if (desc->B * desc->H * desc->T == 0) return GMDN_OK;
  if (!q || !k || !v || !beta || !g || !o) return GMDN_ERR_ARG;
  if (desc->rule >= 1 && !gmu) return GMDN_ERR_ARG;
  if (desc->rule == 2 && !gnu) return GMDN_ERR_ARG;
  // tiles and gate chunks are fetched with 16-byte LDS-DMA loads
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(beta) || !aligned16(g) ||
      (gmu && !aligned16(gmu)) || (gnu && !aligned16(gnu)))
    return GMDN_ERR_UNSUPPORTED;
  // o is written in 16-byte pieces along d
  if (!aligned16(o) || (desc->so[0] & 7) || (desc->so[1] & 7) || (desc->so[2] & 7)) return GMDN_ERR_UNSUPPORTED;
  const ChunkArgs a = make_args(desc, q, k, v, beta, g, gmu, gnu, o, states);
  hipStream_t s = (hipStream_t)stream;
  if (desc->dtype == GMDN_DTYPE_F32) {
    // float32 streams: the matrix form around the drop-in scan, whose chunk
    // states the output kernel reads -- `states` is required for inference too
    if (!states || !aligned16(states)) return GMDN_ERR_ARG;
    if (desc->rule == 2 && desc->eps != 1e-6f) return GMDN_ERR_UNSUPPORTED;  // the drop-in adam's epsilon
    return chunk_fwd_f32_launch(a, desc->d, desc->rule, desc->ns, static_cast<float*>(states), s) == hipSuccess
               ? GMDN_OK
               : GMDN_ERR_LAUNCH;
  }
  if (desc->rule == 1) {
    // muon: the output kernel reads the chunk states from `states`, which is
    // therefore required for inference too
    if (!states || !aligned16(states)) return GMDN_ERR_ARG;
    if (desc->ns > 8) return GMDN_ERR_ARG;
    float* S_out = static_cast<float*>(states);
    float* M_out = S_out + a.B * a.H * a.N * (int64_t)desc->d * desc->d;
    return chunk_fwd_muon_launch(a, desc->d, S_out, M_out, desc->ns, s) == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
  }
  if (desc->rule == 2 && desc->d == 128 && states) {
    // training: the drop-in adam scan in exact float32 between chunk-parallel
    // kernels (its epsilon is the reference's 1e-6, fast_scan.py:94)
    if (!aligned16(states)) return GMDN_ERR_ARG;
    if (desc->eps != 1e-6f) return GMDN_ERR_UNSUPPORTED;
    return chunk_fwd_adam_mat_launch(a, desc->d, static_cast<float*>(states), s) == hipSuccess ? GMDN_OK
                                                                                               : GMDN_ERR_LAUNCH;
  }
  return chunk_fwd_launch(a, desc->d, desc->rule, s) == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

size_t gmdn_wy_fwd_workspace_bytes(const gmdn_chunk_desc* desc) {
  if (check_desc(desc) != GMDN_OK) return 0;
  return wy_workspace_floats(desc->B, desc->H, desc->T, desc->d) * sizeof(float);
}

int gmdn_wy_fwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v, const float* beta,
                const float* g, void* o, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_desc(desc);
  if (rc != GMDN_OK) return rc;
  if (desc->dtype != GMDN_DTYPE_BF16) return GMDN_ERR_UNSUPPORTED;  // bf16 token streams only
  if (desc->B * desc->H * desc->T == 0) return GMDN_OK;
  if (!q || !k || !v || !beta || !g || !o) return GMDN_ERR_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return GMDN_ERR_UNSUPPORTED;
  if ((desc->so[0] & 7) || (desc->so[1] & 7) || (desc->so[2] & 7)) return GMDN_ERR_UNSUPPORTED;
  if (!workspace || !aligned16(workspace) || workspace_bytes < gmdn_wy_fwd_workspace_bytes(desc))
    return GMDN_ERR_WORKSPACE;
  const ChunkArgs a = make_args(desc, q, k, v, beta, g, nullptr, nullptr, o, nullptr);
  return wy_fwd_launch(a, desc->d, static_cast<float*>(workspace), (hipStream_t)stream) == hipSuccess
             ? GMDN_OK
             : GMDN_ERR_LAUNCH;
}

size_t gmdn_wy_bwd_workspace_bytes(const gmdn_chunk_desc* desc) {
  if (check_desc(desc) != GMDN_OK || desc->dtype != GMDN_DTYPE_BF16) return 0;
  return wy_bwd_workspace_floats(desc->B, desc->H, desc->T, desc->d) * sizeof(float);
}

int gmdn_wy_bwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v, const float* beta,
                const float* g, const void* ckpt, const void* dO, void* dq, void* dk, void* dv, float* dbeta,
                float* dg, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_desc(desc);
  if (rc != GMDN_OK) return rc;
  if (desc->dtype != GMDN_DTYPE_BF16) return GMDN_ERR_UNSUPPORTED;
  if (desc->B * desc->H * desc->T == 0) return GMDN_OK;
  if (!q || !k || !v || !beta || !g || !ckpt || !dO || !dq || !dk || !dv || !dbeta || !dg) return GMDN_ERR_ARG;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dO) || !aligned16(ckpt))
    return GMDN_ERR_UNSUPPORTED;
  if ((desc->so[0] & 7) || (desc->so[1] & 7) || (desc->so[2] & 7)) return GMDN_ERR_UNSUPPORTED;
  if (!workspace || !aligned16(workspace) || workspace_bytes < gmdn_wy_bwd_workspace_bytes(desc))
    return GMDN_ERR_WORKSPACE;
  const ChunkArgs a = make_args(desc, q, k, v, beta, g, nullptr, nullptr, nullptr, nullptr);
  return wy_bwd_launch(a, desc->d, const_cast<float*>(static_cast<const float*>(ckpt)), dO, dq, dk, dv, dbeta, dg,
                       static_cast<float*>(workspace), (hipStream_t)stream) == hipSuccess
             ? GMDN_OK
             : GMDN_ERR_LAUNCH;
}

size_t gmdn_chunk_bwd_workspace_bytes(const gmdn_chunk_desc* desc) {
  if (check_desc(desc) != GMDN_OK) return 0;
  if (desc->dtype == GMDN_DTYPE_F32)
    return chunk_f32_bwd_ws_floats(desc->B * desc->H, desc->T / CB_C, desc->d, desc->rule, desc->ns) *
           sizeof(float);
  // muon: Kw, Uv, gS and dU per chunk, the chunk scalars and their
  // gradients, and the drop-in muon backward's workspace
  if (desc->rule == 1)
    return chunk_bwd_muon_ws_floats(desc->B * desc->H, desc->T / CB_C, desc->d, desc->ns) * sizeof(float);
  if (desc->rule == 2 && desc->d == 128)
    return chunk_bwd_adam_mat_ws_floats(desc->B * desc->H, desc->T / CB_C, desc->d) * sizeof(float);
  // Gb_i, the cotangent of a chunk's state update (fp32 d x d per chunk; the
  // delta rule keeps the odd chunks' only), then per (chunk, row block)
  // partial sums of the chunk scalars' gradients; adam: then the carry of
  // the reverse scan's segments
  return chunk_bwd_min_ws_bytes(desc) + ascan_carry_bytes(desc);
}

int gmdn_chunk_bwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v,
                   const float* beta, const float* g, const float* gmu, const float* gnu,
                   const void* states, const void* dO, void* dq, void* dk, void* dv, float* dbeta,
                   float* dg, float* dgmu, float* dgnu, void* workspace, size_t workspace_bytes,
                   void* stream) {
  int rc = check_desc(desc);
  if (rc != GMDN_OK) return rc;
  if (desc->B * desc->H * desc->T == 0) return GMDN_OK;
  if (!q || !k || !v || !beta || !g || !states || !dO || !dq || !dk || !dv || !dbeta || !dg)
    return GMDN_ERR_ARG;
  if (desc->rule >= 1 && (!gmu || !dgmu)) return GMDN_ERR_ARG;
  if (desc->rule == 2 && (!gnu || !dgnu)) return GMDN_ERR_ARG;
  if (desc->rule == 1 && desc->precision != GMDN_PREC_TF32 && desc->precision != GMDN_PREC_IEEE)
    return GMDN_ERR_ARG;
  // adam at d = 128 runs its scan in exact float32 (the split-bf16 state
  // products exceed the gradient tolerance there): the reference's epsilon
  if (desc->rule == 2 && (desc->d == 128 || desc->dtype == GMDN_DTYPE_F32) && desc->eps != 1e-6f)
    return GMDN_ERR_UNSUPPORTED;
  if (desc->B * desc->H * (desc->T / CB_C) >= ((int64_t)1 << 31)) return GMDN_ERR_ARG;  // one workgroup per chunk
  const bool bf16_rows = desc->dtype != GMDN_DTYPE_F32 && !(desc->rule == 2 && desc->d == 128);
  const size_t min_ws = desc->rule == 1 && desc->dtype != GMDN_DTYPE_F32 && desc->precision == GMDN_PREC_TF32
                            ? chunk_bwd_muon_min_ws_floats(desc->B * desc->H, desc->T / CB_C, desc->d, desc->ns) *
                                  sizeof(float)
                        : desc->rule != 1 && bf16_rows ? chunk_bwd_min_ws_bytes(desc)
                                                       : gmdn_chunk_bwd_workspace_bytes(desc);
  if (!workspace || workspace_bytes < min_ws) return GMDN_ERR_WORKSPACE;
  // dO tiles arrive by 16-byte LDS-DMA loads and dq, dk, dv leave in 16-byte
  // row pieces: every stream needs 16-byte aligned rows
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dO) || !aligned16(dq) ||
      !aligned16(dk) || !aligned16(dv) || !aligned16(beta) || !aligned16(g) || !aligned16(states) ||
      !aligned16(workspace) || (gmu && !aligned16(gmu)) || (gnu && !aligned16(gnu)))
    return GMDN_ERR_UNSUPPORTED;
  if ((desc->so[0] & 7) || (desc->so[1] & 7) || (desc->so[2] & 7)) return GMDN_ERR_UNSUPPORTED;
  ChunkArgs a = make_args(desc, q, k, v, beta, g, gmu, gnu, const_cast<void*>(dO),
                          const_cast<void*>(states));
  a.gb = (float*)workspace;
  a.part = a.gb + (int64_t)gb_planes(desc) * desc->d * desc->d;
  a.dq = (bf16*)dq;
  a.dk = (bf16*)dk;
  a.dv = (bf16*)dv;
  a.dbeta = dbeta;
  a.dg = dg;
  a.dgmu = dgmu;
  a.dgnu = dgnu;
  if (desc->dtype == GMDN_DTYPE_F32)
    return chunk_bwd_f32_launch(a, desc->d, desc->rule, desc->ns, static_cast<const float*>(states),
                                (float*)workspace, workspace_bytes / sizeof(float), (hipStream_t)stream) == hipSuccess
               ? GMDN_OK
               : GMDN_ERR_LAUNCH;
  if (desc->rule == 2 && desc->d == 128)
    return chunk_bwd_adam_mat_launch(a, desc->d, (float*)workspace, (hipStream_t)stream) == hipSuccess
               ? GMDN_OK
               : GMDN_ERR_LAUNCH;
  if (desc->rule == 1)
    return chunk_bwd_muon_launch(a, desc->d, desc->ns, desc->precision, (float*)workspace,
                                 workspace_bytes / sizeof(float), (hipStream_t)stream) == hipSuccess
               ? GMDN_OK
               : GMDN_ERR_LAUNCH;
  // adam: the reverse scan in segments beside the token gradients when the
  // workspace holds the carry (its default size), in one pass otherwise
  const size_t base = chunk_bwd_min_ws_bytes(desc), carry = ascan_carry_bytes(desc);
  float* ascan_carry = carry && workspace_bytes >= base + carry ? (float*)((char*)workspace + base) : nullptr;
  return chunk_bwd_launch(a, desc->d, desc->rule, ascan_carry, (hipStream_t)stream) == hipSuccess ? GMDN_OK
                                                                                                 : GMDN_ERR_LAUNCH;
}

}  // extern "C"
