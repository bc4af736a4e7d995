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

// LDS carve-up of the forward kernel (bytes)
// Chunk tiles (Q, K, the workgroup's 32 columns of V, and the gate chunk)
// live in a ring of FWD_STAGES LDS buffers filled by LDS-DMA FWD_STAGES - 1
// chunks ahead, so HBM latency is covered by that many chunks of work.  The
// chunk loop is unrolled over the ring, so every LDS read address is a
// per-lane base register (computed once) plus an immediate offset.
constexpr int FWD_STAGES = RING;

template <int D>
struct FwdLds {
  static constexpr int NKBH = D / 64;            // k-blocks in a column half
  static constexpr int TILE = CB_C * D * 2;      // one Q or K chunk (bytes)
  static constexpr int VT = CB_C * 32 * 2;       // the workgroup's V columns
  static constexpr int GT = 4 * CB_C * 4;        // beta, g, gmu, gnu
  static constexpr int Q0 = 0;
  static constexpr int K0 = Q0 + FWD_STAGES * TILE;
  static constexpr int V0 = K0 + FWD_STAGES * TILE;
  static constexpr int G0 = V0 + FWD_STAGES * VT;
  static constexpr int A0 = G0 + FWD_STAGES * GT;  // -A hi plane, then lo plane
  static constexpr int AP = CB_C * CB_C * 2;
  static constexpr int XS0 = A0 + 2 * AP;          // S^T operand exchange
  static constexpr int XE0 = XS0 + CB_WAVES * NKBH * 2 * 1024;  // E operand exchange
  static constexpr int BYTES = XE0 + CB_WAVES * 2 * 2 * 1024;
  static_assert(BYTES <= 160 * 1024, "forward LDS exceeds the 160 KiB of a CU");
  // LDS-DMA instructions one wave issues per chunk (Q, K, V; wave 0 also the gates)
  static constexpr int DMA_OPS = 2 * (CB_C * D / 8) / CB_THREADS + (CB_C * 32 / 8) / CB_THREADS;
};

template <int D, int RULE>
__global__ void __launch_bounds__(CB_THREADS) chunk_fwd(ChunkArgs p) {
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
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int rt = w >> 1, h = w & 1;
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
  // row reads of Q / K: lane (r, G) reads row r of a 16-row tile at columns
  // k0 + 4G (half 0) and k0 + 16 + 4G (half 1), k0 = 32 kb
  uint32_t rowoff[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) rowoff[kb][hf] = swz_off<LQ>(lc, 32 * kb + 16 * hf + 4 * G);
  // transposing reads of K columns 16 ct .. for this wave's column tiles
  uint32_t coloff[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) coloff[t] = swz_off<LQ>(4 * G + (lc >> 2), 16 * (h * NTH + t) + 4 * (lc & 3));
  // transposing reads of V (rows 32h + 16u + 4G + lc/4, columns 16 rt + 4 (lc & 3))
  // (the row part 32h + 16u is added as an immediate in segment 1: whole
  // multiples of 4 rows leave the swizzle term unchanged; the column part
  // 16 rt is not additive under the XOR and stays in the base)
  const uint32_t voff = swz_off<LV>(4 * G + (lc >> 2), 16 * rt + 4 * (lc & 3));
  // row reads of -A (rows 16 tt + lc, tt = 2h + u; columns 32 kbs + 16 hf + 4G)
  uint32_t aoff[2][2];
#pragma unroll
  for (int kbs = 0; kbs < 2; ++kbs)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) aoff[kbs][hf] = swz_off<LA>(32 * h + lc, 32 * kbs + 16 * hf + 4 * G);
  const uint32_t xoff = 16 * l;  // exchange slots: one 16-byte piece per lane
  // LDS pointers, one set per region, so that the stage, row-tile and k
  // offsets added inside the loop stay within the 16-bit immediate
  const uint32_t lds0 = lds_addr(smem);
  const lds_ptr L0 = lds_base(smem);
  lds_cptr qrow[NKB][2], krowa[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      qrow[kb][hf] = L0 + (rowoff[kb][hf] + L::Q0);
      krowa[kb][hf] = L0 + (rowoff[kb][hf] + L::K0);
    }
  lds_cptr colp[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) colp[t] = L0 + (coloff[t] + L::K0);
  const lds_cptr vaddr = L0 + (voff + L::V0);
  lds_cptr ap[2][2];
#pragma unroll
  for (int kbs = 0; kbs < 2; ++kbs)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) ap[kbs][hf] = L0 + (aoff[kbs][hf] + L::A0);
  const lds_ptr xsaddr = L0 + (xoff + L::XS0);
  const lds_ptr xeaddr = L0 + (xoff + L::XE0);

  // the strictly-upper tiles of -A are never written: zero them once
  for (int e = threadIdx.x; e < CB_C * CB_C; e += CB_THREADS) {
    const int r = e / CB_C, c = e % CB_C;
    if ((c >> 4) > (r >> 4)) {
      Ahi[LA::off(r, c)] = (bf16)0.f;
      Alo[LA::off(r, c)] = (bf16)0.f;
    }
  }

  DmaPlan<LQ, CB_C, CB_THREADS> dq, dk;
  DmaPlan<LV, CB_C, CB_THREADS> dv;
  dq.init(w, p.sq[2]);
  dk.init(w, p.sk[2]);
  dv.init(w, p.sv[2]);
  auto issue_loads = [&](int i, int stg) {
    const int64_t t0 = (int64_t)i * CB_C;
    dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + stg * L::TILE, w);
    dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + stg * L::TILE, w);
    dv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + stg * L::VT, w);
    if (w == 0) lds_dma16(gsrc + t0, smem + L::G0 + stg * L::GT);
  };

  f32x4 S[NTH], Mm[NTH], Vv[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) S[t] = Mm[t] = Vv[t] = zero4();
  // o of a chunk is stored at the start of the next one, so that the wait for
  // the next chunk's tiles (vmcnt counts stores too on gfx9) does not also
  // wait for this chunk's stores to be acknowledged.
  f32x4 O[2] = {zero4(), zero4()};
  auto store_o = [&](int i) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bf16* op = og + ((int64_t)i * CB_C + 16 * (2 * h + u) + 4 * G) * p.so[2];
#pragma unroll
      for (int j = 0; j < 4; ++j) op[j * p.so[2]] = (bf16)O[u][j];
    }
  };
  // exchange slot (16 bytes per lane) of wave ww, piece k
  auto xs_addr = [&](int ww, int k) { return xsaddr + ((ww * NKBH + k) * 2) * 1024; };
  auto xe_addr = [&](int ww, int k) { return xeaddr + ((ww * 2 + k) * 2) * 1024; };
  auto publish_S = [&]() {
#pragma unroll
    for (int kbl = 0; kbl < NKBH; ++kbl) {
      const Op<2> x = pack_tiles<2>(S[2 * kbl], S[2 * kbl + 1]);
      lds_st<bf16x8>(xs_addr(w, kbl), x.v[0]);
      lds_st<bf16x8>(xs_addr(w, kbl) + 1024, x.v[1]);
    }
  };
  auto read_op = [&](lds_cptr addr) {
    Op<2> x;
    x.v[0] = lds_ld<bf16x8>(addr);
    x.v[1] = lds_ld<bf16x8>(addr + 1024);
    return x;
  };
  float a = 0.f, bsc = 0.f, msc = 0.f, nsc = 0.f;
  auto chunk_scalars = [&](int stg) {
    const float* gg = reinterpret_cast<const float*>(smem + L::G0 + stg * L::GT);
    a = expf(wave_sum(fmaxf(gg[CB_C + l], LOG_FLOOR)));
    if constexpr (RULE == 2) {
      bsc = wave_sum(gg[l]) * (1.f / CB_C);
      msc = expf(wave_sum(fmaxf(gg[2 * CB_C + l], LOG_FLOOR)));
      nsc = expf(wave_sum(fmaxf(gg[3 * CB_C + l], LOG_FLOOR)));
    }
  };

  for (int j = 0; j < FWD_STAGES - 1 && j < p.N; ++j) issue_loads(j, j);
  publish_S();
  wait_vmem();
  __syncthreads();  // X_0
  if (p.N > 0) chunk_scalars(0);

  // One chunk; STG = i % FWD_STAGES is a compile-time constant.
  auto chunk = [&](auto stg_tag, int i) {
    constexpr int STG = decltype(stg_tag)::value;
    constexpr uint32_t SQK = STG * L::TILE;  // stage offsets within the regions
    constexpr uint32_t VC = STG * L::VT;
    const float* gates = reinterpret_cast<const float*>(smem + L::G0 + STG * L::GT);
    if (i > 0) store_o(i - 1);
    const bool ahead = i + FWD_STAGES - 1 < p.N;
    if (ahead) issue_loads(i + FWD_STAGES - 1, (STG + FWD_STAGES - 1) % FWD_STAGES);
    if (p.states) {  // pre-update state (and adam's moments) for the backward
      const int64_t plane = p.B * p.H * p.N * (int64_t)D * D;
      float* sp = p.states + ((bh * p.N + i) * D + r0 + lc) * (int64_t)D + 4 * G;
#pragma unroll
      for (int t = 0; t < NTH; ++t) {
        *reinterpret_cast<f32x4*>(sp + 16 * (h * NTH + t)) = S[t];
        if constexpr (RULE == 2) {
          *reinterpret_cast<f32x4*>(sp + plane + 16 * (h * NTH + t)) = Mm[t];
          *reinterpret_cast<f32x4*>(sp + 2 * plane + 16 * (h * NTH + t)) = Vv[t];
        }
      }
    }
    // k-block kb of row tile `rowtile` (a compile-time offset from the base set)
    auto rows = [&](const lds_cptr (&base)[NKB][2], int rowtile, int kb) {
      return cat8(lds_ld<bf16x4>(base[kb][0] + SQK + rowtile * 16 * ROWB),
                  lds_ld<bf16x4>(base[kb][1] + SQK + rowtile * 16 * ROWB));
    };
    // ================= segment 1 (specialised per wave: RT, H compile-time)
    auto segment1 = [&](auto rt_tag, auto h_tag, auto tiles) {
      constexpr int RT = decltype(rt_tag)::value, H = decltype(h_tag)::value;
      // S_i^T operand of every k-block, from the slot of the wave owning it
      // (row tile rt, column half kb / NKBH)
      Op<2> Sop[NKB];
  #pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Sop[kb] = read_op(xs_addr(2 * RT + kb / NKBH, kb % NKBH));
      // N = K S^T - V = -E for this wave's tokens 32h .. 32h+31 (two chains)
      f32x4 Nt[2];
      {
        bf16x8 Kr[2][NKB];
  #pragma unroll
        for (int u = 0; u < 2; ++u) {
          const bf16x4 vb = lds_tr16(vaddr + (VC + (32 * H + 16 * u) * 64));
          Nt[u] = f32x4{-(float)vb[0], -(float)vb[1], -(float)vb[2], -(float)vb[3]};
  #pragma unroll
          for (int kb = 0; kb < NKB; ++kb) Kr[u][kb] = rows(krowa, 2 * H + u, kb);
        }
  #pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
  #pragma unroll
          for (int u = 0; u < 2; ++u) Nt[u] = mma<1, 2>(Op<1>{{Kr[u][kb]}}, Sop[kb], Nt[u]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // o = Q S^T for this wave's tokens (two chains)
      {
        bf16x8 Qr[2][NKB];
  #pragma unroll
        for (int u = 0; u < 2; ++u)
  #pragma unroll
          for (int kb = 0; kb < NKB; ++kb) Qr[u][kb] = rows(qrow, 2 * H + u, kb);
        O[0] = O[1] = zero4();
  #pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
  #pragma unroll
          for (int u = 0; u < 2; ++u) O[u] = mma<1, 2>(Op<1>{{Qr[u][kb]}}, Sop[kb], O[u]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // publish the E operands: N (for A E) and -w N (for G), w per token row
      {
        const f32x4 b0 = *reinterpret_cast<const f32x4*>(gates + 32 * H + 4 * G);
        const f32x4 b1 = *reinterpret_cast<const f32x4*>(gates + 32 * H + 16 + 4 * G);
        const f32x4 w0 = RULE == 0 ? -b0 : f32x4{-1.f, -1.f, -1.f, -1.f};
        const f32x4 w1 = RULE == 0 ? -b1 : f32x4{-1.f, -1.f, -1.f, -1.f};
        const Op<2> en = pack_tiles<2>(Nt[0], Nt[1]);
        const Op<2> we = pack_tiles<2>(Nt[0] * w0, Nt[1] * w1);
        lds_st<bf16x8>(xe_addr(2 * RT + H, 0), en.v[0]);
        lds_st<bf16x8>(xe_addr(2 * RT + H, 0) + 1024, en.v[1]);
        lds_st<bf16x8>(xe_addr(2 * RT + H, 1), we.v[0]);
        lds_st<bf16x8>(xe_addr(2 * RT + H, 1) + 1024, we.v[1]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // this wave's tiles of -A^T = -(K Q^T) diag(beta), restricted to s <= t.
      // Tile idx = w + 4k of the causal list; the switch makes st, tt constant.
      auto a_tile = [&](auto st_tag, auto tt_tag) {
        constexpr int st = decltype(st_tag)::value, tt = decltype(tt_tag)::value;
        bf16x8 ka[NKB], qa[NKB];
  #pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          ka[kb] = rows(krowa, st, kb);
          qa[kb] = rows(qrow, tt, kb);
        }
        f32x4 acc = zero4();
  #pragma unroll
        for (int kb = 0; kb < NKB; ++kb) acc = mfma(ka[kb], qa[kb], acc);
        // lane (t, G) holds (Q K^T)[t][s] for s = 16 st + 4G + j
        const f32x4 bs = *reinterpret_cast<const f32x4*>(gates + 16 * st + 4 * G);
        bf16x4 hi4, lo4;
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float val = (st < tt || 4 * G + j <= lc) ? -acc[j] * bs[j] : 0.f;
          bf16 hv, lv;
          split2(val, hv, lv);
          hi4[j] = hv;
          lo4[j] = lv;
        }
        const int ao = LA::off(16 * tt + lc, 16 * st + 4 * G);
        *reinterpret_cast<bf16x4*>(Ahi + ao) = hi4;
        *reinterpret_cast<bf16x4*>(Alo + ao) = lo4;
        __builtin_amdgcn_sched_barrier(0);
      };
      tiles(a_tile);
    };
    using std::integral_constant;
    using I0 = integral_constant<int, 0>;
    using I1 = integral_constant<int, 1>;
    using I2 = integral_constant<int, 2>;
    using I3 = integral_constant<int, 3>;
    // causal tiles (st, tt) of -A per wave: w0 {00 12 23}, w1 {01 22 33}, w2 {11 03}, w3 {02 13}
    switch (w) {
      case 0:
        segment1(I0{}, I0{}, [&](auto&& f) { f(I0{}, I0{}); f(I1{}, I2{}); f(I2{}, I3{}); });
        break;
      case 1:
        segment1(I0{}, I1{}, [&](auto&& f) { f(I0{}, I1{}); f(I2{}, I2{}); f(I3{}, I3{}); });
        break;
      case 2:
        segment1(I1{}, I0{}, [&](auto&& f) { f(I1{}, I1{}); f(I0{}, I3{}); });
        break;
      default:
        segment1(I1{}, I1{}, [&](auto&& f) { f(I0{}, I2{}); f(I1{}, I3{}); });
        break;
    }
    __syncthreads();  // Y_i: E halves and -A published
    // ================= segment 2
    // E operands of both token halves (slots of waves (rt, 0) and (rt, 1))
    Op<2> EN[2], WE[2];
#pragma unroll
    for (int hs = 0; hs < 2; ++hs) {
      EN[hs] = read_op(xe_addr(2 * rt + hs, 0));
      WE[hs] = read_op(xe_addr(2 * rt + hs, 1));
    }
    // G^T for this wave's column half (NTH chains) and the state update
    {
      bf16x8 Kcol[NTH][2];
#pragma unroll
      for (int t = 0; t < NTH; ++t)
#pragma unroll
        for (int kbs = 0; kbs < 2; ++kbs) {
          Kcol[t][kbs] = cat8(lds_tr16(colp[t] + SQK + kbs * 32 * ROWB),
                              lds_tr16(colp[t] + SQK + kbs * 32 * ROWB + 16 * ROWB));
        }
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
          for (int j = 0; j < 4; ++j) S[t][j] = a * S[t][j] + bsc * Mm[t][j] / (sqrtf(Vv[t][j]) + p.eps);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    publish_S();  // S_{i+1}^T half, read after X_{i+1}
    __builtin_amdgcn_sched_barrier(0);
    // o += (-A)(-E) over the causal token blocks kbs <= h
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int kbs = 0; kbs < 2; ++kbs) {
        if (kbs > h) continue;
        auto arow = [&](uint32_t plane) {
          return cat8(lds_ld<bf16x4>(ap[kbs][0] + (plane + u * 16 * CB_C * 2)),
                      lds_ld<bf16x4>(ap[kbs][1] + (plane + u * 16 * CB_C * 2)));
        };
        O[u] = mma<2, 2>(Op<2>{{arow(0), arow(L::AP)}}, EN[kbs], O[u]);
      }
    }
    // chunk i+1's tiles must have landed; the loads issued after them (for
    // chunk i+FWD_STAGES-1) may stay in flight.  Vector loads complete in
    // issue order, so vmcnt <= (loads issued since) suffices; stores only
    // make the count more conservative.
    if (ahead) {
      if (w == 0)
        wait_vmem_le<L::DMA_OPS + 1>();
      else
        wait_vmem_le<L::DMA_OPS>();
    } else {
      wait_vmem();
    }
    __syncthreads();  // X_{i+1}: next chunk's tiles landed, S_{i+1} halves published
    if (i + 1 < p.N) chunk_scalars((STG + 1) % FWD_STAGES);
  };

  for (int i = 0; i < p.N; i += FWD_STAGES) {
    chunk(std::integral_constant<int, 0>{}, i);
    if (i + 1 < p.N) chunk(std::integral_constant<int, 1>{}, i + 1);
    if (i + 2 < p.N) chunk(std::integral_constant<int, 2>{}, i + 2);
  }
  if (p.N > 0) store_o(p.N - 1);
}

template <int D, int RULE>
static hipError_t launch_fwd(const ChunkArgs& a, hipStream_t stream) {
  auto kern = chunk_fwd<D, RULE>;
  const int lds = FwdLds<D>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (D / 32);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(CB_THREADS), lds, stream, a);
  return hipGetLastError();
}

hipError_t chunk_fwd_launch(const ChunkArgs& a, int d, int rule, hipStream_t s) {
  if (d == 128) return rule == 0 ? launch_fwd<128, 0>(a, s) : launch_fwd<128, 2>(a, s);
  return rule == 0 ? launch_fwd<64, 0>(a, s) : launch_fwd<64, 2>(a, s);
}

}  // namespace gmdn

using namespace gmdn;

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_desc(const gmdn_chunk_desc* d) {
  if (!d) return GMDN_ERR_ARG;
  if (d->B < 0 || d->H < 0 || d->T < 0) return GMDN_ERR_ARG;
  if (d->rule < 0 || d->rule > 2 || d->ns < 0 || d->ns > 8) return GMDN_ERR_ARG;
  if (d->C != CB_C || (d->d != 64 && d->d != 128)) return GMDN_ERR_UNSUPPORTED;
  if (d->dtype != GMDN_DTYPE_BF16) return GMDN_ERR_UNSUPPORTED;
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

}  // namespace

extern "C" {

size_t gmdn_chunk_states_bytes(const gmdn_chunk_desc* desc) {
  if (check_desc(desc) != GMDN_OK) return 0;
  // S_i for every rule; adam adds its moments M_i and V_i
  const size_t planes = desc->rule == 2 ? 3 : 1;
  return planes * (size_t)(desc->B * desc->H * (desc->T / CB_C)) * desc->d * desc->d * sizeof(float);
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
  if (desc->rule == 1) return GMDN_ERR_UNSUPPORTED;
  const ChunkArgs a = make_args(desc, q, k, v, beta, g, gmu, gnu, o, states);
  hipStream_t s = (hipStream_t)stream;
  return chunk_fwd_launch(a, desc->d, desc->rule, s) == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

size_t gmdn_chunk_bwd_workspace_bytes(const gmdn_chunk_desc* desc) {
  if (check_desc(desc) != GMDN_OK) return 0;
  // Gb_i, the cotangent of every chunk's state update (fp32 d x d per chunk),
  // then per (chunk, row block) partial sums of the chunk scalars' gradients
  const size_t chunks = (size_t)(desc->B * desc->H * (desc->T / CB_C));
  return chunks * desc->d * desc->d * sizeof(float) + chunks * (desc->d / 32) * 4 * sizeof(float);
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
  if (desc->rule == 1) return GMDN_ERR_UNSUPPORTED;
  // adam at d = 128: the sign-like update M / (sqrt(V) + eps) amplifies the
  // rounding of the split-bf16 state products beyond the gradient tolerance
  if (desc->rule == 2 && desc->d != 64) return GMDN_ERR_UNSUPPORTED;
  if (desc->B * desc->H * (desc->T / CB_C) >= ((int64_t)1 << 31)) return GMDN_ERR_ARG;  // one workgroup per chunk
  if (!workspace || workspace_bytes < gmdn_chunk_bwd_workspace_bytes(desc)) return GMDN_ERR_WORKSPACE;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dO) || !aligned16(dv) ||
      !aligned16(beta) || !aligned16(g) || !aligned16(states) || !aligned16(workspace))
    return GMDN_ERR_UNSUPPORTED;
  ChunkArgs a = make_args(desc, q, k, v, beta, g, gmu, gnu, const_cast<void*>(dO),
                          const_cast<void*>(states));
  a.gb = (float*)workspace;
  a.part = a.gb + a.B * a.H * a.N * (int64_t)desc->d * desc->d;
  a.dq = (bf16*)dq;
  a.dk = (bf16*)dk;
  a.dv = (bf16*)dv;
  a.dbeta = dbeta;
  a.dg = dg;
  a.dgmu = dgmu;
  a.dgnu = dgnu;
  return chunk_bwd_launch(a, desc->d, desc->rule, (hipStream_t)stream) == hipSuccess ? GMDN_OK
                                                                                     : GMDN_ERR_LAUNCH;
}

}  // extern "C"
