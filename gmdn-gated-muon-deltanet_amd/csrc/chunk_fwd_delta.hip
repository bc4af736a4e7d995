// Level B forward of the delta rule: state rows owned by single waves.
//
// Same mathematics as chunk_fwd<D, 0> (reference train_ablation.py:142-187
// with fast_scan.py:72-95, E-form): per (b, h) and chunk i with state S_i,
//   E = V - K S_i^T,   S_{i+1} = a S_i + E^T diag(beta) K,
//   o = Q S_i^T + tril(Q K^T) diag(beta) E = Q S_i^T + tril(Q K^T) (beta E).
//
// Work split.  A workgroup of four waves, one per SIMD, owns 32 rows of S for
// the whole sequence (B H D / 32 workgroups, the D/32 of one (b, h) on one XCD).
//  * State waves 0, 1 each own 16 whole rows.  The chunk's recurrence stays in
//    the wave's registers: E is formed as D-layout tiles (token rows, state-row
//    columns), and two such tiles stacked along the tokens are the pair-order
//    operand of the next product, so E -> G -> S_{i+1} -> the next E needs no
//    exchange and no barrier.  The state is held negated (Sf = -S): then
//    E = V + K Sf^T and Sf_{i+1} = a Sf + K^T (-beta E), all plain sums.
//  * Output waves 2, 3 each own two of the four token tiles ({0, 3} | {1, 2},
//    five causal A tiles each) for all 32 rows.  They form A^T = (K Q^T) tiles
//    in registers (again directly the pair-order operand), Q Sf^T from the
//    S pieces the state waves publish, and A (-beta E) one chunk later, when
//    the state waves have published -beta E; all the LDS-DMA traffic, the o
//    stores and the checkpoint stores are theirs.
// One barrier per chunk.  In interval i (between barriers i and i + 1) the
// state waves run chunk i and publish -beta E_i and Sf_{i+1}; the output
// waves issue the copies of chunk i + 2, finish and store o_{i-1}, and form
// A_i and Q_i Sf_i^T.  The published operands are double-buffered by chunk
// parity and kept in register order (lane l's 16 bytes at 16 l), so they are
// written and read with conflict-free 16-byte accesses and no index math.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

#include <type_traits>

namespace gmdn {

constexpr int FD_WAVES = 4;
constexpr int FD_THREADS = 64 * FD_WAVES;

template <int D>
struct FwdDeltaLds {
  static constexpr int NKB = D / 32;
  static constexpr int TILE = CB_C * D * 2;  // one Q or K chunk (bytes)
  static constexpr int VT = CB_C * 32 * 2;   // the workgroup's 32 columns of V
  static constexpr int GT = 2 * CB_C * 4;    // beta and g of a chunk
  static constexpr int Q0 = 0;
  static constexpr int K0 = Q0 + RING * TILE;
  static constexpr int V0 = K0 + RING * TILE;
  static constexpr int G0 = V0 + RING * VT;
  // per state wave and chunk parity: Sf pieces (NKB k-blocks x hi, lo) and
  // -beta E pieces (2 token blocks x hi, lo), 1 KiB per operand register set
  static constexpr int SPW = NKB * 2 * 1024;
  static constexpr int EPW = 2 * 2 * 1024;
  static constexpr int SP0 = G0 + RING * GT;
  static constexpr int EP0 = SP0 + 2 * 2 * SPW;
  static constexpr int BYTES = EP0 + 2 * 2 * EPW;
  static_assert(BYTES <= 160 * 1024, "delta forward LDS exceeds the 160 KiB of a CU");
};

template <int D>
__global__ void __launch_bounds__(FD_THREADS) chunk_fwd_delta(ChunkArgs p) {
  using LQ = BSwz<D>;
  using LV = BSwz<32>;
  using L = FwdDeltaLds<D>;
  constexpr int NKB = D / 32;  // k-blocks over the state's columns
  constexpr int NCT = D / 16;  // column tiles of a state row block
  constexpr int ROWB = D * 2;  // bytes per Q / K row
  using DQ = DmaPlan<LQ, CB_C, 128>;
  using DV = DmaPlan<LV, CB_C, 128>;
  extern __shared__ __align__(16) char smem[];

  int64_t bh;
  int blk;
  map_block(p.B * p.H, D / 32, bh, blk);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const lds_ptr L0 = lds_base(smem);
  const int N = p.N;

  // pair-order row operand of a Q or K tile: lane (m, G) takes row 16 rb + m,
  // columns 32 kb + 4G .. +3 (slots 0-3) and 32 kb + 16 + 4G .. +3 (4-7).
  // Whole 16-row tiles leave the row's swizzle term unchanged, so the row
  // tile, region and stage parts are immediates on a per-(kb, half) base.
  lds_cptr rowp[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int h = 0; h < 2; ++h) rowp[kb][h] = L0 + swz_off<LQ>(lc, 32 * kb + 16 * h + 4 * G);
  auto row_op = [&](uint32_t off, int kb) {
    return cat8(lds_ld<bf16x4>(rowp[kb][0] + off), lds_ld<bf16x4>(rowp[kb][1] + off));
  };

  if (w < 2) {
    // ======================================================== state waves
    // transposing reads of K columns 16 ct + i (rows 32 kb + 16 h + 4G + i/4)
    lds_cptr colp[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) colp[ct] = L0 + swz_off<LQ>(4 * G + (lc >> 2), 16 * ct + 4 * (lc & 3));
    auto col_op = [&](uint32_t off, int ct, int kb) {
      return cat8(lds_tr16(colp[ct] + off + 32 * kb * ROWB), lds_tr16(colp[ct] + off + (32 * kb + 16) * ROWB));
    };
    // V: tokens 16 st + 4G + j of the wave's column 16 w + lc
    const lds_cptr vp = L0 + swz_off<LV>(4 * G + (lc >> 2), 16 * w + 4 * (lc & 3));
    const lds_cptr bp = L0 + (L::G0 + 16 * G);      // beta[16 st + 4G ..]
    const lds_cptr gp = L0 + (L::G0 + 256 + 4 * l);  // g[l]
    const lds_ptr spw = L0 + (L::SP0 + w * L::SPW + 16 * l);
    const lds_ptr epw = L0 + (L::EP0 + w * L::EPW + 16 * l);

    f32x4 Sf[NCT];  // -S, lane (r, G): columns 16 ct + 4G + j of row r
    Op<2> Sp[NKB];  // its pieces, pair order
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) Sf[ct] = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sp[kb] = pack_tiles<2>(Sf[2 * kb], Sf[2 * kb + 1]);
    auto publish_S = [&](int par) {
      const uint32_t po = (uint32_t)par * (2 * L::SPW);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + po + (kb * 2 + u) * 1024, Sp[kb].v[u]);
    };
    publish_S(0);
    __syncthreads();  // barrier 0: chunk 0 landed, Sf_0 published

    auto state_chunk = [&](auto stg_tag, int i) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      const float a = expf(wave_sum(fmaxf(lds_ld<float>(gp + STG * L::GT), LOG_FLOOR)));
      // E = V + K Sf^T, token tiles st (lane (r, G): tokens 16 st + 4G + j)
      f32x4 E[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x4 vb = lds_tr16(vp + (L::V0 + STG * L::VT + st * 16 * 64));
        E[st] = f32x4{(float)vb[0], (float)vb[1], (float)vb[2], (float)vb[3]};
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        bf16x8 Kr[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) Kr[st] = row_op(L::K0 + SQK + st * 16 * ROWB, kb);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int st = 0; st < 4; ++st) E[st] = mfma(Kr[st], Sp[kb].v[u], E[st]);
      }
      // -beta E pieces: the operand of G and of the output waves' A (-beta E)
      Op<2> WE[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const f32x4 b0 = lds_ld<f32x4>(bp + (STG * L::GT + 2 * kt * 64));
        const f32x4 b1 = lds_ld<f32x4>(bp + (STG * L::GT + (2 * kt + 1) * 64));
        WE[kt] = pack_tiles<2>(-(b0 * E[2 * kt]), -(b1 * E[2 * kt + 1]));
      }
      const uint32_t eo = (uint32_t)(i & 1) * (2 * L::EPW);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_st<bf16x8>(epw + eo + (kt * 2 + u) * 1024, WE[kt].v[u]);
      // Sf_{i+1} = a Sf_i + K^T (-beta E), column tiles ct (transposed tiles:
      // lane (r, G) gets columns 16 ct + 4G + j of row r)
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) Sf[ct] = a * Sf[ct];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        bf16x8 Kc[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Kc[ct] = col_op(L::K0 + SQK, ct, kt);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) Sf[ct] = mfma(Kc[ct], WE[kt].v[u], Sf[ct]);
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Sp[kb] = pack_tiles<2>(Sf[2 * kb], Sf[2 * kb + 1]);
      publish_S((i + 1) & 1);
      __syncthreads();  // barrier i + 1
    };
    for (int i = 0; i < N; i += RING) {
      state_chunk(std::integral_constant<int, 0>{}, i);
      if (i + 1 < N) state_chunk(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < N) state_chunk(std::integral_constant<int, 2>{}, i + 2);
    }
    return;
  }

  // ========================================================== output waves
  const int ow = w - 2;
  const uint32_t lds0 = lds_addr(smem);
  const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
  const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
  const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + 32 * blk;
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + 32 * blk + 4 * G;
  // gates: lanes 0-15 beta, 16-31 g (16 bytes each); copied by wave 2's low half
  const float* gsrc = (G == 1 ? p.g : p.beta) + bh * p.T + 4 * lc;
  DQ dq, dk;
  DV dv;
  dq.init(ow, p.sq[2]);
  dk.init(ow, p.sk[2]);
  dv.init(ow, p.sv[2]);
  auto issue_loads = [&](int i, int stg) {
    const int64_t t0 = (int64_t)i * CB_C;
    dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + stg * L::TILE, ow);
    dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + stg * L::TILE, ow);
    dv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + stg * L::VT, ow);
    if (ow == 0 && l < 32) lds_dma16(gsrc + t0, smem + L::G0 + stg * L::GT);
  };
  // vector-memory operations this wave issues per chunk copy
  constexpr int ND1 = 2 * DQ::NOPS + DV::NOPS;
  const lds_cptr spr = L0 + (L::SP0 + 16 * l);
  const lds_cptr epr = L0 + (L::EP0 + 16 * l);

  // prologue: chunks 0 and 1 in flight, chunk 0 waited for
  issue_loads(0, 0);
  if (N > 1) {
    issue_loads(1, 1);
    if (ow == 0)
      wait_vmem_le<ND1 + 1>();
    else
      wait_vmem_le<ND1>();
  } else {
    wait_vmem();
  }
  __syncthreads();  // barrier 0

  // token tiles TA, TB of this wave; A pieces per (token tile, key block)
  auto run = [&](auto ta_tag, auto tb_tag) {
    constexpr int TT[2] = {decltype(ta_tag)::value, decltype(tb_tag)::value};
    Op<2> Ap[2][2], Aq[2][2];  // this chunk's and the previous chunk's
    f32x4 O[2][2], Oq[2][2];   // -o^T tiles [row tile][token tile], likewise
    const bf16x8 z8 = bf16x8{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
#pragma unroll
    for (int a_ = 0; a_ < 2; ++a_)
#pragma unroll
      for (int b_ = 0; b_ < 2; ++b_) {
        Ap[a_][b_].v[0] = Ap[a_][b_].v[1] = z8;
        Aq[a_][b_] = Ap[a_][b_];
        O[a_][b_] = Oq[a_][b_] = zero4();
      }
    auto finish_prev = [&](int i) {  // o_{i-1} += A (-beta E), stored
      const uint32_t eo = (uint32_t)((i - 1) & 1) * (2 * L::EPW);
      Op<2> WE[2][2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int u = 0; u < 2; ++u) WE[rt][kt].v[u] = lds_ld<bf16x8>(epr + eo + rt * L::EPW + (kt * 2 + u) * 1024);
      // (hi, hi), (hi, lo), (lo, hi) of each operand pair
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int pc = 0; pc < 3; ++pc)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int x = 0; x < 2; ++x)
              if (2 * kt <= TT[x])
                Oq[rt][x] = mfma(WE[rt][kt].v[pc == 2 ? 1 : 0], Aq[x][kt].v[pc == 1 ? 1 : 0], Oq[rt][x]);
      // lane (t, G) of tile (rt, x): token 16 TT[x] + t, columns 16 rt + 4G ..
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const f32x4 v = Oq[rt][x];
          *reinterpret_cast<bf16x4*>(og + ((int64_t)(i - 1) * CB_C + 16 * TT[x] + lc) * p.so[2] + 16 * rt) =
              to_bf16x4(-v);
        }
    };
    auto out_chunk = [&](auto stg_tag, int i) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      const bool dma = i + 2 < N, prev = i >= 1;
      const bool ck = p.states && (i & 1) == 0;
      if (dma) issue_loads(i + 2, (STG + 2) % RING);
      if (prev) finish_prev(i);
      // A^T tiles (K Q^T, causal part) -> pair-order A operands of chunk i
      bf16x8 Qr[2][NKB];
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) Qr[x][kb] = row_op(L::Q0 + SQK + TT[x] * 16 * ROWB, kb);
      f32x4 At[2][4];
#pragma unroll
      for (int x = 0; x < 2; ++x)
#pragma unroll
        for (int st = 0; st < 4; ++st) At[x][st] = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        bf16x8 Kr[4];
#pragma unroll
        for (int st = 0; st < 4; ++st)
          if (st <= TT[1]) Kr[st] = row_op(L::K0 + SQK + st * 16 * ROWB, kb);
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
          for (int x = 0; x < 2; ++x)
            if (st <= TT[x]) At[x][st] = mfma(Kr[st], Qr[x][kb], At[x][st]);
      }
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        // keep s <= t on the diagonal tile: lane (t, G) row 4G + j is s
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (4 * G + j > lc) At[x][TT[x]][j] = 0.f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          if (2 * kt <= TT[x]) Ap[x][kt] = pack_tiles<2>(At[x][2 * kt], At[x][2 * kt + 1]);
      }
      // -o^T = Sf Q^T (+ A (-beta E) next interval)
      const uint32_t sbo = (uint32_t)(i & 1) * (2 * L::SPW);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        Op<2> Sr[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int u = 0; u < 2; ++u) Sr[kb].v[u] = lds_ld<bf16x8>(spr + sbo + rt * L::SPW + (kb * 2 + u) * 1024);
        O[rt][0] = O[rt][1] = zero4();
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int x = 0; x < 2; ++x) O[rt][x] = mfma(Sr[kb].v[u], Qr[x][kb], O[rt][x]);
        // checkpoint S_i of the even chunks (the backward rebuilds the odd
        // ones): rows 16 ow + lc from the pieces just read, negated back
        if (ck && rt == ow) {
          const int64_t plane = bh * ((N + 1) / 2) + i / 2;
          float* sp = p.states + (plane * D + 32 * blk + 16 * ow + lc) * (int64_t)D + 4 * G;
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            *reinterpret_cast<bf16x8*>(sp + 32 * kb) =
                neg8(__builtin_shufflevector(Sr[kb].v[0], Sr[kb].v[1], 0, 1, 2, 3, 8, 9, 10, 11));
            *reinterpret_cast<bf16x8*>(sp + 32 * kb + 16) =
                neg8(__builtin_shufflevector(Sr[kb].v[0], Sr[kb].v[1], 4, 5, 6, 7, 12, 13, 14, 15));
          }
        }
      }
      // chunk i + 1 must have landed; what this wave issued after its copy
      // (the copy of chunk i + 2, o_{i-1}, the checkpoint) may stay in flight
      if (i + 1 < N) {
        constexpr int C = 2 * NKB;
        if (ow == 0) {
          if (dma) {
            if (prev) {
              if (ck) wait_vmem_le<ND1 + 1 + 4 + C>(); else wait_vmem_le<ND1 + 1 + 4>();
            } else {
              if (ck) wait_vmem_le<ND1 + 1 + C>(); else wait_vmem_le<ND1 + 1>();
            }
          } else {
            if (prev) {
              if (ck) wait_vmem_le<4 + C>(); else wait_vmem_le<4>();
            } else {
              if (ck) wait_vmem_le<C>(); else wait_vmem_le<0>();
            }
          }
        } else {
          if (dma) {
            if (prev) {
              if (ck) wait_vmem_le<ND1 + 4 + C>(); else wait_vmem_le<ND1 + 4>();
            } else {
              if (ck) wait_vmem_le<ND1 + C>(); else wait_vmem_le<ND1>();
            }
          } else {
            if (prev) {
              if (ck) wait_vmem_le<4 + C>(); else wait_vmem_le<4>();
            } else {
              if (ck) wait_vmem_le<C>(); else wait_vmem_le<0>();
            }
          }
        }
      }
      __syncthreads();  // barrier i + 1
#pragma unroll
      for (int a_ = 0; a_ < 2; ++a_)
#pragma unroll
        for (int b_ = 0; b_ < 2; ++b_) {
          Aq[a_][b_] = Ap[a_][b_];
          Oq[a_][b_] = O[a_][b_];
        }
    };
    for (int i = 0; i < N; i += RING) {
      out_chunk(std::integral_constant<int, 0>{}, i);
      if (i + 1 < N) out_chunk(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < N) out_chunk(std::integral_constant<int, 2>{}, i + 2);
    }
    finish_prev(N);
  };
  if (ow == 0)
    run(std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{});
  else
    run(std::integral_constant<int, 1>{}, std::integral_constant<int, 2>{});
}

template <int D>
static hipError_t launch_fwd_delta(const ChunkArgs& a, hipStream_t stream) {
  auto kern = chunk_fwd_delta<D>;
  constexpr int lds = FwdDeltaLds<D>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (D / 32);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(FD_THREADS), lds, stream, a);
  return hipGetLastError();
}

hipError_t chunk_fwd_delta_launch(const ChunkArgs& a, int d, hipStream_t s) {
  return d == 128 ? launch_fwd_delta<128>(a, s) : launch_fwd_delta<64>(a, s);
}

}  // namespace gmdn
