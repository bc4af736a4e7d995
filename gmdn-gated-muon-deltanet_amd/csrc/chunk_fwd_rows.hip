// Level B forward with state rows owned by single waves: the delta rule and
// adam.
//
// Same mathematics as chunk_fwd<D, RULE> (reference train_ablation.py:142-187
// with fast_scan.py:72-95, E-form): per (b, h) and chunk i with state S_i,
//   E = V - K S_i^T,   o = Q S_i^T + tril(Q K^T) diag(beta) E,
//   delta: S_{i+1} = a S_i + E^T diag(beta) K
//   adam : G = E^T K,  M <- m M + (1-m) G,  V <- n V + (1-n) G^2,
//          S_{i+1} = a S_i + b M / (sqrt(V) + eps)
// (fast_scan.py:86-94), with b = mean beta and m, n from gmu, gnu as a from g.
//
// Work split.  A workgroup of eight waves, two per SIMD, owns 32 rows of S
// for the whole sequence (B H D / 32 workgroups, the D/32 of one (b, h) on
// one XCD).  Wave w runs on SIMD w % 4.
//  * State waves 0, 1 each own 16 whole rows.  The chunk's recurrence stays in
//    the wave's registers: E is formed as D-layout tiles (token rows, state-row
//    columns), and two such tiles stacked along the tokens are the pair-order
//    operand of G.  G's tiles come out transposed with the state columns of a
//    32-column block permuted (tile u of block kb holds, in lane group G,
//    columns 32 kb + 8G + 4u .. +3: its K^T operand is read with that column
//    permutation), so the two tiles of a block are the next E's operand in
//    natural column order and every K, Q row operand is one 16-byte read.
//    E -> G -> S_{i+1} -> the next E needs no exchange and no barrier (adam's
//    moments M, V sit beside S in the same layout).  The state is held
//    negated (Sf = -S): then E = V + K Sf^T and, for delta,
//    Sf_{i+1} = a Sf + K^T (-beta E), all plain sums.  Each
//    product is ordered so that its first half's results can be split into
//    pieces (and published) while its second half is still in the MFMA pipe.
//  * Output waves 2, 3, 6, 7 own token tiles 3, 2, 0, 1 (so SIMDs 2 and 3 each
//    carry 5 of the 10 causal A tiles) for all 32 rows.  They form A^T = K Q^T
//    tiles in registers (again directly the pair-order operand), Q Sf^T from
//    the S pieces the state waves publish, and A (-beta E) one chunk later,
//    when the state waves have published -beta E; they store o and the
//    checkpoint.
//  * Copy waves 4, 5 (on the state waves' SIMDs) issue every LDS-DMA copy,
//    wait for it and reduce the chunk decay a_i into an LDS slot, so no
//    compute wave waits on vector memory or on the issue of a copy.
// One barrier per chunk.  In interval i (between barriers i and i + 1) the
// state waves run chunk i and publish -beta E_i and Sf_{i+1}; the output
// waves finish and store o_{i-1} and form A_i and Q_i Sf_i^T; the copy waves
// issue chunk i + 2 and wait for chunk i + 1.  The published operands are
// double-buffered by chunk parity and kept in register order (lane l's 16
// bytes at 16 l): conflict-free 16-byte writes and reads, no index math.
//
// Adam (d = 64) splits each row block's state work over two waves, ten waves
// in all: state waves 0-3 (row block w & 1, half h = w >> 1), output waves
// 4-7 (token tiles 0, 1, 3, 2), copy waves 8, 9.  State wave h forms E for
// token block h from its own S pieces (k-blocks of half h) and the other
// half's published ones, publishes -E of that block, and after a mid-chunk
// barrier forms G and the moment update for the state columns of half h
// from both blocks' -E.  The exchanges go through the regions the output
// waves read anyway.  The update's VALU work (two quarter-rate
// transcendentals per value) is halved per wave, which pays for the second
// barrier; the copy waves reduce chunk i's scalars before it and issue the
// next copies after it.  The delta rule keeps one state wave per row block:
// split the same way it measured slower, its output waves becoming the chain.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

#include <type_traits>

namespace gmdn {

// An LDS base the compiler cannot see into: per-region bases that share the
// same lane offset are otherwise merged into one register plus the region's
// offset, which no longer fits the 16-bit immediate of ds_read / ds_write.
GMDN_DEV lds_cptr opaque_base(lds_cptr p) {
  uint32_t v = (uint32_t)(uintptr_t)p;
  asm volatile("" : "+v"(v));
  return (lds_cptr)(uintptr_t)v;
}

// waves per workgroup: adam splits each row block's state work over two
// waves (see the state waves below), the delta rule keeps one
template <int RULE>
constexpr int fd_threads() { return 64 * (RULE == 2 ? 10 : 8); }

template <int D, int RULE>
struct FwdRowsLds {
  static constexpr int NKB = D / 32;
  static constexpr int TILE = CB_C * D * 2;  // one Q or K chunk (bytes)
  static constexpr int VT = CB_C * 32 * 2;   // the workgroup's 32 columns of V
  // beta and g of a chunk (adam: and gmu, gnu)
  static constexpr int GT = (RULE == 2 ? 4 : 2) * CB_C * 4;
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
  // chunk scalars {a, b, m, n} per ring stage (delta: a only)
  static constexpr int SC0 = EP0 + 2 * 2 * EPW;
  // adam's training forward: M_i, V_i staged by the state waves for the
  // output waves' stores, [chunk parity][state wave][M, V][column tile]
  static constexpr int MV0 = SC0 + RING * 16;
  static constexpr int MVW = 2 * (D / 16) * 1024;
  static constexpr int BYTES = MV0 + (RULE == 2 ? 2 * 2 * MVW : 0);
  static_assert(BYTES <= 160 * 1024, "delta forward LDS exceeds the 160 KiB of a CU");
};

template <int D, int RULE>
__global__ void __launch_bounds__(fd_threads<RULE>()) chunk_fwd_rows(ChunkArgs p) {
  // Q, K tiles: conflict-free row operands, two-way permuted K^T operands
  using LQ = RowSwz<D>;
  using LV = BSwz<32>;
  using L = FwdRowsLds<D, RULE>;
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

  // adam: state waves 0-3, output waves 4-7, copy waves 8, 9; delta: state
  // waves 0, 1, output waves 2, 3, 6, 7, copy waves 4, 5
  constexpr bool SPLIT = RULE == 2;
  if (SPLIT ? w >= 8 : (w == 4 || w == 5)) {
    // ========================================================= copy waves
    const int cw = SPLIT ? w - 8 : w - 4;
    const uint32_t lds0 = lds_addr(smem);
    const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
    const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
    const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + 32 * blk;
    // gates, 16 bytes per lane: wave 4 lanes 0-15 beta, 16-31 g; adam's
    // wave 5 lanes 0-15 gmu, 16-31 gnu (each wave reduces what it copies)
    const bool gcopy = cw == 0 || RULE == 2;
    const float* gsrc =
        (cw == 0 ? (G == 0 ? p.beta : p.g) : (G == 0 ? p.gmu : p.gnu)) + bh * p.T + 4 * lc;
    DQ dq, dk;
    DV dv;
    dq.init(cw, p.sq[2]);
    dk.init(cw, p.sk[2]);
    dv.init(cw, p.sv[2]);
    auto issue_loads = [&](int i, int stg) {
      const int64_t t0 = (int64_t)i * CB_C;
      dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + stg * L::TILE, cw);
      dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + stg * L::TILE, cw);
      dv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + stg * L::VT, cw);
      if (gcopy && l < 32) lds_dma16(gsrc + t0, smem + L::G0 + stg * L::GT + 512 * cw);
    };
    // vector-memory operations this wave issues per chunk copy
    constexpr int ND = 2 * DQ::NOPS + DV::NOPS;
    // chunk i + 1 landed (the copy of chunk i + 2, if issued, in flight)
    auto wait_next = [&](bool issued) {
      if (!issued)
        wait_vmem();
      else if (gcopy)
        wait_vmem_le<ND + 1>();
      else
        wait_vmem_le<ND>();
    };
    // a = exp(sum over the chunk of max(g, log 1e-6)) of the chunk in stage
    // stg (wave 4); adam: b = mean(beta) (wave 4), m, n as a from gmu, gnu
    // (wave 5).  The copy waves share SIMDs with the state waves, so the
    // reductions run as two interleaved chains per wave.
    auto decay = [&](int stg) {
      const lds_cptr gg = L0 + (L::G0 + stg * L::GT + 4 * l);
      float* sc = reinterpret_cast<float*>(smem + L::SC0 + stg * 16);
      if (cw == 0) {
        if constexpr (RULE == 2) {
          const f32x2 s = wave_sum2(fmaxf(lds_ld<float>(gg + 256), LOG_FLOOR), lds_ld<float>(gg));
          if (l == 0) *reinterpret_cast<f32x2*>(sc) = f32x2{expf(s[0]), s[1] * (1.f / CB_C)};
        } else {
          const float a = expf(wave_sum(fmaxf(lds_ld<float>(gg + 256), LOG_FLOOR)));
          if (l == 0) *sc = a;
        }
      } else if constexpr (RULE == 2) {
        const f32x2 s = wave_sum2(fmaxf(lds_ld<float>(gg + 512), LOG_FLOOR), fmaxf(lds_ld<float>(gg + 768), LOG_FLOOR));
        if (l == 0) *reinterpret_cast<f32x2*>(sc + 2) = f32x2{expf(s[0]), expf(s[1])};
      }
    };
    issue_loads(0, 0);
    if (N > 1) issue_loads(1, 1);
    wait_next(N > 1);
    decay(0);
    __syncthreads();  // barrier 0
    for (int i = 0; i < N; ++i) {
      const bool dma = i + 2 < N;
      if constexpr (SPLIT) {
        // chunk i's scalars (its tiles landed in interval i - 1) are first
        // read after the mid-chunk barrier; the copies go out after it, off
        // the way to it
        if (i >= 1) decay(i % RING);
        __syncthreads();  // the mid-chunk barrier of chunk i
        if (dma) issue_loads(i + 2, (i + 2) % RING);
        if (i + 1 < N) wait_next(dma);
      } else {
        if (dma) issue_loads(i + 2, (i + 2) % RING);
        if (i + 1 < N) {
          wait_next(dma);
          decay((i + 1) % RING);
        }
      }
      __syncthreads();  // barrier i + 1
    }
    return;
  }

  // natural-order row operand of a Q or K tile: lane (m, G) takes row
  // 16 rb + m, columns 32 kb + 8G .. +7 (one 16-byte read).  Whole 16-row
  // tiles leave the row's swizzle term unchanged, so the row tile and stage
  // parts are immediates on a per-(region, kb) base: one base set per region
  // keeps every immediate within 16 bits.
  lds_cptr rowK[NKB], rowQ[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    rowK[kb] = opaque_base(L0 + (L::K0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
    rowQ[kb] = opaque_base(L0 + (L::Q0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
  }
  auto row_op = [&](const lds_cptr (&base)[NKB], uint32_t off, int kb) { return lds_ld<bf16x8>(base[kb] + off); };

  if (SPLIT && w < 4) {
    // ================================================ state waves (adam)
    // Wave w: row block rb = w & 1 (rows 16 rb .. 16 rb + 15 of the
    // workgroup's 32) and half h = w >> 1, which forms E for token block h
    // (tokens 32 h .. 32 h + 31) and the update for the state columns of
    // k-blocks h NKB/2 .. (h + 1) NKB/2 - 1.  E's other k-blocks come from the
    // other half's published S pieces, the update's other token block from
    // its published -beta E pieces: the regions the output waves read.
    const int rb = w & 1;
    // K^T operand of G's tile ct = 2 kb + u: lane (m, G) takes K[s][c] for
    // the pair-order tokens s of block kt and column c = 32 kb + 4u + 8 (m / 4)
    // + m % 4; in transposing reads lane (i, G) addresses row
    // 32 kt + 16 h + 4G + i / 4, columns 32 kb + 4u + 8 (i % 4) ..
    lds_cptr colp[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
      colp[ct] = opaque_base(
          L0 + (L::K0 + swz_off<LQ>(4 * G + (lc >> 2), 32 * (ct >> 1) + 4 * (ct & 1) + 8 * (lc & 3))));
    auto col_op = [&](uint32_t off, int ct, int kt) {
      return cat8(lds_tr16(colp[ct] + off + 32 * kt * ROWB), lds_tr16(colp[ct] + off + (32 * kt + 16) * ROWB));
    };
    // V: tokens 16 st + 4G + j of the row block's column 16 rb + lc
    const lds_cptr vp = L0 + swz_off<LV>(4 * G + (lc >> 2), 16 * rb + 4 * (lc & 3));
    const lds_cptr bp = L0 + (L::G0 + 16 * G);  // beta[16 st + 4G ..]
    const lds_ptr spw = L0 + (L::SP0 + rb * L::SPW + 16 * l);
    const lds_ptr epw = L0 + (L::EP0 + rb * L::EPW + 16 * l);

    auto halves = [&](auto h_tag) {
      constexpr int H = decltype(h_tag)::value;
      constexpr int NKH = NKB / 2, NCH = NCT / 2;  // k-blocks, column tiles of a half
      constexpr int KB0 = H * NKH, KBO = (1 - H) * NKH, CT0 = H * NCH;
      // -S, lane (r, G) of tile c: columns 32 ((CT0 + c) / 2) + 8G + 4 (c % 2) + j
      f32x4 Sf[NCH];
      Op<2> Sp[NKH];  // its pieces, k-blocks KB0 .., natural order
      f32x4 Mm[NCH], Vv[NCH];  // adam's moments, same layout
#pragma unroll
      for (int c = 0; c < NCH; ++c) Sf[c] = Mm[c] = Vv[c] = zero4();
#pragma unroll
      for (int k = 0; k < NKH; ++k) Sp[k] = pack_tiles<2>(Sf[2 * k], Sf[2 * k + 1]);
#pragma unroll
      for (int k = 0; k < NKH; ++k)
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + ((KB0 + k) * 2 + u) * 1024, Sp[k].v[u]);
      // adam's training forward: M_i, V_i for the backward, staged for the
      // output waves' stores at the end of chunk i - 1 (zeros for chunk 0)
      auto stage_mv = [&](int i) {
        if constexpr (RULE == 2) {
          if (p.states) {
            const lds_ptr mv = L0 + (L::MV0 + ((i & 1) * 2 + rb) * L::MVW + 16 * l);
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
              lds_st<f32x4>(mv + (CT0 + c) * 1024, Mm[c]);
              lds_st<f32x4>(mv + (NCT + CT0 + c) * 1024, Vv[c]);
            }
          }
        }
      };
      stage_mv(0);
      __syncthreads();  // barrier 0: chunk 0 landed, Sf_0 published

      auto state_chunk = [&](auto stg_tag, int i) {
        constexpr int STG = decltype(stg_tag)::value;
        constexpr uint32_t SQK = STG * L::TILE;
        // E = V + K Sf^T, token tiles 2H, 2H + 1 (lane (r, G): tokens
        // 16 st + 4G + j): the own k-blocks from registers, the other half's
        // from its pieces published at the end of the last chunk
        const uint32_t so = (uint32_t)(i & 1) * (2 * L::SPW);
        Op<2> Sq[NKH];
#pragma unroll
        for (int k = 0; k < NKH; ++k)
#pragma unroll
          for (int u = 0; u < 2; ++u) Sq[k].v[u] = lds_ld<bf16x8>(spw + so + ((KBO + k) * 2 + u) * 1024);
        f32x4 E[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const bf16x4 vb = lds_tr16(vp + (L::V0 + STG * L::VT + (2 * H + s) * 16 * 64));
          E[s] = f32x4{(float)vb[0], (float)vb[1], (float)vb[2], (float)vb[3]};
        }
        bf16x8 Kr[2][NKB];
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) Kr[s][kb] = row_op(rowK, SQK + (2 * H + s) * 16 * ROWB, kb);
#pragma unroll
        for (int k = 0; k < NKH; ++k)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            E[0] = mfma(Kr[0][KB0 + k], Sp[k].v[u], E[0]);
            E[1] = mfma(Kr[1][KB0 + k], Sp[k].v[u], E[1]);
          }
#pragma unroll
        for (int k = 0; k < NKH; ++k)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            E[0] = mfma(Kr[0][KBO + k], Sq[k].v[u], E[0]);
            E[1] = mfma(Kr[1][KBO + k], Sq[k].v[u], E[1]);
          }
        // -beta E (delta), -E (adam) of token block H, published for the
        // other half and the output waves
        const uint32_t eo = (uint32_t)(i & 1) * (2 * L::EPW);
        Op<2> WE[2];  // [token block]
        if constexpr (RULE == 0) {
          f32x4 bt[2];
#pragma unroll
          for (int s = 0; s < 2; ++s) bt[s] = lds_ld<f32x4>(bp + (STG * L::GT + (2 * H + s) * 64));
          WE[H] = pack_tiles<2>(-(bt[0] * E[0]), -(bt[1] * E[1]));
        } else {
          WE[H] = pack_tiles<2>(-E[0], -E[1]);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_st<bf16x8>(epw + eo + (H * 2 + u) * 1024, WE[H].v[u]);
        // the update's K^T operands, read while the barrier waits
        bf16x8 Kc[2][NCH];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int c = 0; c < NCH; ++c) Kc[kt][c] = col_op(SQK, CT0 + c, kt);
        __syncthreads();  // mid-chunk barrier: both token blocks' -beta E published
#pragma unroll
        for (int u = 0; u < 2; ++u) WE[1 - H].v[u] = lds_ld<bf16x8>(epw + eo + ((1 - H) * 2 + u) * 1024);
        const uint32_t po = (uint32_t)((i + 1) & 1) * (2 * L::SPW);
        if constexpr (RULE == 0) {
          // Sf_{i+1} = a Sf_i + K^T (-beta E) for the half's column tiles
          // (transposed tiles in the permuted column order above): the own
          // token block for every tile, then the other block tile pair by
          // tile pair, each pair split and published while the next is in
          // the MFMA pipe
          const float a = lds_ld<float>(L0 + (L::SC0 + STG * 16));
#pragma unroll
          for (int c = 0; c < NCH; ++c) Sf[c] = a * Sf[c];
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int c = 0; c < NCH; ++c) Sf[c] = mfma(Kc[H][c], WE[H].v[u], Sf[c]);
#pragma unroll
          for (int k = 0; k < NKH; ++k) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              Sf[2 * k] = mfma(Kc[1 - H][2 * k], WE[1 - H].v[u], Sf[2 * k]);
              Sf[2 * k + 1] = mfma(Kc[1 - H][2 * k + 1], WE[1 - H].v[u], Sf[2 * k + 1]);
            }
            Sp[k] = pack_tiles<2>(Sf[2 * k], Sf[2 * k + 1]);
#pragma unroll
            for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + po + ((KB0 + k) * 2 + u) * 1024, Sp[k].v[u]);
          }
        } else {
          // adam: Gn = K^T (-E) = -G^T tiles, then per tile pair
          //   M = m M + (1 - m) G,  V = n V + (1 - n) G^2,
          //   Sf = a Sf - b M / (sqrt(V) + eps)
          // split and published while the next pair is in the MFMA pipe
          const f32x4 sc = lds_ld<f32x4>(L0 + (L::SC0 + STG * 16));
          const float a = sc[0], b = sc[1], m = sc[2], n = sc[3];
          f32x4 Gn[NCH];
#pragma unroll
          for (int c = 0; c < NCH; ++c) Gn[c] = zero4();
#pragma unroll
          for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int c = 0; c < NCH; ++c) Gn[c] = mfma(Kc[H][c], WE[H].v[u], Gn[c]);
          auto update = [&](int c) {
            Mm[c] = m * Mm[c] - (1.f - m) * Gn[c];
            Vv[c] = n * Vv[c] + (1.f - n) * (Gn[c] * Gn[c]);
#pragma unroll
            for (int j = 0; j < 4; ++j) Sf[c][j] = a * Sf[c][j] - b * Mm[c][j] * hw_rcp(hw_sqrt(Vv[c][j]) + p.eps);
          };
#pragma unroll
          for (int k = 0; k < NKH; ++k) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              Gn[2 * k] = mfma(Kc[1 - H][2 * k], WE[1 - H].v[u], Gn[2 * k]);
              Gn[2 * k + 1] = mfma(Kc[1 - H][2 * k + 1], WE[1 - H].v[u], Gn[2 * k + 1]);
            }
            update(2 * k);
            update(2 * k + 1);
            Sp[k] = pack_tiles<2>(Sf[2 * k], Sf[2 * k + 1]);
#pragma unroll
            for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + po + ((KB0 + k) * 2 + u) * 1024, Sp[k].v[u]);
          }
        }
        if (i + 1 < N) stage_mv(i + 1);  // M_{i+1}, V_{i+1}: chunk i + 1's
        __syncthreads();  // barrier i + 1
      };
      for (int i = 0; i < N; i += RING) {
        state_chunk(std::integral_constant<int, 0>{}, i);
        if (i + 1 < N) state_chunk(std::integral_constant<int, 1>{}, i + 1);
        if (i + 2 < N) state_chunk(std::integral_constant<int, 2>{}, i + 2);
      }
    };
    if (w >> 1)
      halves(std::integral_constant<int, 1>{});
    else
      halves(std::integral_constant<int, 0>{});
    return;
  }

  if (!SPLIT && w < 2) {
    // ======================================================== state waves
    // K^T operand of G's tile ct = 2 kb + u: lane (m, G) takes K[s][c] for
    // the pair-order tokens s of block kt and column c = 32 kb + 4u + 8 (m / 4)
    // + m % 4; in transposing reads lane (i, G) addresses row
    // 32 kt + 16 h + 4G + i / 4, columns 32 kb + 4u + 8 (i % 4) ..
    lds_cptr colp[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
      colp[ct] = opaque_base(
          L0 + (L::K0 + swz_off<LQ>(4 * G + (lc >> 2), 32 * (ct >> 1) + 4 * (ct & 1) + 8 * (lc & 3))));
    auto col_op = [&](uint32_t off, int ct, int kt) {
      return cat8(lds_tr16(colp[ct] + off + 32 * kt * ROWB), lds_tr16(colp[ct] + off + (32 * kt + 16) * ROWB));
    };
    // V: tokens 16 st + 4G + j of the wave's column 16 w + lc
    const lds_cptr vp = L0 + swz_off<LV>(4 * G + (lc >> 2), 16 * w + 4 * (lc & 3));
    const lds_cptr bp = L0 + (L::G0 + 16 * G);  // beta[16 st + 4G ..]
    const lds_ptr spw = L0 + (L::SP0 + w * L::SPW + 16 * l);
    const lds_ptr epw = L0 + (L::EP0 + w * L::EPW + 16 * l);

    f32x4 Sf[NCT];  // -S, lane (r, G): columns 32 (ct / 2) + 8G + 4 (ct % 2) + j of row r
    Op<2> Sp[NKB];  // its pieces, natural order
    f32x4 Mm[NCT], Vv[NCT];  // adam's moments, same layout
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) Sf[ct] = Mm[ct] = Vv[ct] = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sp[kb] = pack_tiles<2>(Sf[2 * kb], Sf[2 * kb + 1]);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + (kb * 2 + u) * 1024, Sp[kb].v[u]);
    // adam's training forward: M_i, V_i for the backward, staged for the
    // output waves' stores at the end of chunk i - 1 (zeros for chunk 0)
    auto stage_mv = [&](int i) {
      if constexpr (RULE == 2) {
        if (p.states) {
          const lds_ptr mv = L0 + (L::MV0 + ((i & 1) * 2 + w) * L::MVW + 16 * l);
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) {
            lds_st<f32x4>(mv + ct * 1024, Mm[ct]);
            lds_st<f32x4>(mv + (NCT + ct) * 1024, Vv[ct]);
          }
        }
      }
    };
    stage_mv(0);
    __syncthreads();  // barrier 0: chunk 0 landed, Sf_0 published

    auto state_chunk = [&](auto stg_tag, int i) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      // E = V + K Sf^T, token tiles st (lane (r, G): tokens 16 st + 4G + j),
      // one token block (two tiles) at a time: the first block's -beta E is
      // split and published while the second block is in the MFMA pipe
      f32x4 E[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x4 vb = lds_tr16(vp + (L::V0 + STG * L::VT + st * 16 * 64));
        E[st] = f32x4{(float)vb[0], (float)vb[1], (float)vb[2], (float)vb[3]};
      }
      f32x4 bt[4];
      if constexpr (RULE == 0) {
#pragma unroll
        for (int st = 0; st < 4; ++st) bt[st] = lds_ld<f32x4>(bp + (STG * L::GT + st * 64));
      }
      bf16x8 Kr[4][NKB], Kc[2][NCT];
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) Kr[st][kb] = row_op(rowK, SQK + st * 16 * ROWB, kb);
      // LDS reads return in issue order and at most 15 are counted in flight:
      // G's operands are read between E's products, each well ahead of its use
      __builtin_amdgcn_sched_barrier(0);
      auto e_block = [&](int kt) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            E[2 * kt] = mfma(Kr[2 * kt][kb], Sp[kb].v[u], E[2 * kt]);
            E[2 * kt + 1] = mfma(Kr[2 * kt + 1][kb], Sp[kb].v[u], E[2 * kt + 1]);
          }
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Kc[kt][ct] = col_op(SQK, ct, kt);
      };
      const uint32_t eo = (uint32_t)(i & 1) * (2 * L::EPW);
      Op<2> WE[2];
      auto we_block = [&](int kt) {  // -beta E (delta), -E (adam)
        if constexpr (RULE == 0)
          WE[kt] = pack_tiles<2>(-(bt[2 * kt] * E[2 * kt]), -(bt[2 * kt + 1] * E[2 * kt + 1]));
        else
          WE[kt] = pack_tiles<2>(-E[2 * kt], -E[2 * kt + 1]);
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_st<bf16x8>(epw + eo + (kt * 2 + u) * 1024, WE[kt].v[u]);
      };
      // token block 0: 4 NKB products, 2 NCT column reads interleaved
      e_block(0);
#pragma unroll
      for (int k = 0; k < 4 * NKB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (k < 2 * NCT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      // block 0's -beta E split and published while block 1 is in the pipe
      we_block(0);
      e_block(1);
#pragma unroll
      for (int k = 0; k < 4 * NKB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (k < 2 * NCT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      we_block(1);
      const uint32_t po = (uint32_t)((i + 1) & 1) * (2 * L::SPW);
      if constexpr (RULE == 0) {
        // Sf_{i+1} = a Sf_i + K^T (-beta E), column tiles ct (transposed tiles
        // in the permuted column order above): token block 0 for every tile,
        // then block 1 tile pair by tile pair, each pair split and published
        // while the next is in the MFMA pipe
        const float a = lds_ld<float>(L0 + (L::SC0 + STG * 16));
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Sf[ct] = a * Sf[ct];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) Sf[ct] = mfma(Kc[0][ct], WE[0].v[u], Sf[ct]);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            Sf[2 * kb] = mfma(Kc[1][2 * kb], WE[1].v[u], Sf[2 * kb]);
            Sf[2 * kb + 1] = mfma(Kc[1][2 * kb + 1], WE[1].v[u], Sf[2 * kb + 1]);
          }
          Sp[kb] = pack_tiles<2>(Sf[2 * kb], Sf[2 * kb + 1]);
#pragma unroll
          for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + po + (kb * 2 + u) * 1024, Sp[kb].v[u]);
        }
      } else {
        // adam: Gn = K^T (-E) = -G^T tiles, then per tile pair
        //   M = m M + (1 - m) G,  V = n V + (1 - n) G^2,
        //   Sf = a Sf - b M / (sqrt(V) + eps)
        // split and published while the next pair is in the MFMA pipe
        const f32x4 sc = lds_ld<f32x4>(L0 + (L::SC0 + STG * 16));
        const float a = sc[0], b = sc[1], m = sc[2], n = sc[3];
        f32x4 Gn[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Gn[ct] = zero4();
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) Gn[ct] = mfma(Kc[0][ct], WE[0].v[u], Gn[ct]);
        auto update = [&](int ct) {
          Mm[ct] = m * Mm[ct] - (1.f - m) * Gn[ct];
          Vv[ct] = n * Vv[ct] + (1.f - n) * (Gn[ct] * Gn[ct]);
#pragma unroll
          for (int j = 0; j < 4; ++j) Sf[ct][j] = a * Sf[ct][j] - b * Mm[ct][j] * hw_rcp(hw_sqrt(Vv[ct][j]) + p.eps);
        };
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            Gn[2 * kb] = mfma(Kc[1][2 * kb], WE[1].v[u], Gn[2 * kb]);
            Gn[2 * kb + 1] = mfma(Kc[1][2 * kb + 1], WE[1].v[u], Gn[2 * kb + 1]);
          }
          update(2 * kb);
          update(2 * kb + 1);
          Sp[kb] = pack_tiles<2>(Sf[2 * kb], Sf[2 * kb + 1]);
#pragma unroll
          for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + po + (kb * 2 + u) * 1024, Sp[kb].v[u]);
        }
      }
      if (i + 1 < N) stage_mv(i + 1);  // M_{i+1}, V_{i+1}: chunk i + 1's
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
  // token tile TT of waves 2, 3, 6, 7: 3, 2, 0, 1; the checkpoint share of
  // wave index ow (0..3): row tile ow & 1, k-blocks of half ow >> 1
  // (adam: waves 4, 5, 6, 7 take token tiles 0, 1, 3, 2, the lighter tiles
  // on the copy waves' SIMDs)
  const int ow = SPLIT ? ((w - 4) ^ 2) : ((w & 1) | ((w >> 1) & 2));
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + 32 * blk + 4 * G;
  const lds_cptr spr = L0 + (L::SP0 + 16 * l);
  // adam's M_i, V_i rows from the staging, as contiguous rows: output wave
  // ow stores rows 8 (ow & 1) .. +7 of state wave ow >> 1's 16, D / 32
  // instructions per moment; lane l of instruction k takes the 16-byte unit
  // q = l % U of row 8 (ow & 1) + (64 k + l) / U (U = D / 4 units per row),
  // which the state wave's tile 2 (q / 8) + q % 2 holds in lane r + 16 ((q / 2) % 4)
  constexpr int UPR = D / 4, NMV = D / 32;
  uint32_t mvo[NMV], mvg[NMV];
#pragma unroll
  for (int k = 0; k < NMV; ++k) {
    const int f = 64 * k + l, r = 8 * (ow & 1) + f / UPR, q = f % UPR;
    const int ct = 2 * (q >> 3) + (q & 1), gq = (q >> 1) & 3;
    mvo[k] = (uint32_t)((ow >> 1) * L::MVW + ct * 1024 + 16 * (r + 16 * gq));
    mvg[k] = (uint32_t)((16 * (ow >> 1) + r) * D + 4 * q);
  }
  // the checkpoint's rows: output wave ow stores units 64 (NCK ow + k) + l
  // of the workgroup's 32 rows (row R = f / U, unit q = f % U: columns
  // 4q .. 4q + 3), whose hi and lo halves state wave R / 16 published in the
  // k-block q / 8 planes, lane R % 16 + 16 ((q / 2) % 4), half q % 2
  constexpr int NCK = D / 32;
  uint32_t cko[NCK], ckg[NCK];
#pragma unroll
  for (int k = 0; k < NCK; ++k) {
    const int f = 64 * (NCK * ow + k) + l, R = f / UPR, q = f % UPR;
    cko[k] = (uint32_t)((R >> 4) * L::SPW + (q >> 3) * 2 * 1024 + 16 * ((R & 15) + 16 * ((q >> 1) & 3)) + 8 * (q & 1));
    ckg[k] = (uint32_t)(R * D + 4 * q);
  }
  auto store_mv = [&](int i) {
    if (!p.states) return;
    const int64_t plane = p.B * p.H * (int64_t)N * D * D;
    float* mp = p.states + plane + ((bh * N + i) * D + 32 * blk) * (int64_t)D;
    const uint32_t pb = L::MV0 + (i & 1) * 2 * L::MVW;
#pragma unroll
    for (int k = 0; k < NMV; ++k) {
      const f32x4 m = lds_ld<f32x4>(L0 + (pb + mvo[k]));
      const f32x4 v = lds_ld<f32x4>(L0 + (pb + mvo[k] + NCT * 1024));
      *reinterpret_cast<f32x4*>(mp + mvg[k]) = m;
      *reinterpret_cast<f32x4*>(mp + plane + mvg[k]) = v;
    }
  };
  const lds_cptr epr = L0 + (L::EP0 + 16 * l);
  __syncthreads();  // barrier 0

  auto run = [&](auto tt_tag) {
    constexpr int TT = decltype(tt_tag)::value;
    constexpr int NKT = TT >= 2 ? 2 : 1;  // token blocks of A with s <= t
    constexpr int OW = TT == 3 ? 0 : TT == 2 ? 1 : TT == 0 ? 2 : 3;  // == ow
    Op<2> Ap[2], Aq[2];  // this chunk's and the previous chunk's A pieces
    f32x4 O[2], Oq[2];   // -o^T tiles [row tile], likewise
    const bf16x8 z8 = bf16x8{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      Ap[x].v[0] = Ap[x].v[1] = z8;
      Aq[x] = Ap[x];
      O[x] = Oq[x] = zero4();
    }
    auto finish_prev = [&](int i) {  // o_{i-1} += A (-beta E), stored
      const uint32_t eo = (uint32_t)((i - 1) & 1) * (2 * L::EPW);
      Op<2> WE[2][2];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int u = 0; u < 2; ++u) WE[rt][kt].v[u] = lds_ld<bf16x8>(epr + eo + rt * L::EPW + (kt * 2 + u) * 1024);
      // (hi, hi), (hi, lo), (lo, hi) of each operand pair
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int pc = 0; pc < 3; ++pc)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
            Oq[rt] = mfma(WE[rt][kt].v[pc == 2 ? 1 : 0], Aq[kt].v[pc == 1 ? 1 : 0], Oq[rt]);
      // lane (t, G) of row tile rt: token 16 TT + t, columns 16 rt + 4G ..
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        *reinterpret_cast<bf16x4*>(og + ((int64_t)(i - 1) * CB_C + 16 * TT + lc) * p.so[2] + 16 * rt) =
            to_bf16x4(-Oq[rt]);
    };
    auto out_chunk = [&](auto stg_tag, int i) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      if (RULE == 2) store_mv(i);  // staged before barrier i
      if (i >= 1) finish_prev(i);
      if constexpr (SPLIT) __syncthreads();  // the mid-chunk barrier of chunk i
      // A^T tiles (K Q^T, causal part) -> pair-order A operands of chunk i
      bf16x8 Qr[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Qr[kb] = row_op(rowQ, SQK + TT * 16 * ROWB, kb);
      f32x4 At[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) At[st] = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        bf16x8 Kr[TT + 1];
#pragma unroll
        for (int st = 0; st <= TT; ++st) Kr[st] = row_op(rowK, SQK + st * 16 * ROWB, kb);
#pragma unroll
        for (int st = 0; st <= TT; ++st) At[st] = mfma(Kr[st], Qr[kb], At[st]);
      }
      // adam publishes -E (not -beta E): beta goes on A's columns s
      if constexpr (RULE == 2) {
#pragma unroll
        for (int st = 0; st <= TT; ++st) At[st] *= lds_ld<f32x4>(L0 + (L::G0 + STG * L::GT + 4 * (16 * st + 4 * G)));
      }
      // keep s <= t on the diagonal tile: lane (t, G) row 4G + j is s
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * G + j > lc) At[TT][j] = 0.f;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) Ap[kt] = pack_tiles<2>(At[2 * kt], At[2 * kt + 1]);
      // -o^T = Sf Q^T (+ A (-beta E) next interval)
      const uint32_t sbo = (uint32_t)(i & 1) * (2 * L::SPW);
      Op<2> Sr[2][NKB];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int u = 0; u < 2; ++u)
            Sr[rt][kb].v[u] = lds_ld<bf16x8>(spr + sbo + rt * L::SPW + (kb * 2 + u) * 1024);
      O[0] = O[1] = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) O[rt] = mfma(Sr[rt][kb].v[u], Qr[kb], O[rt]);
      // checkpoint S_i from the published pieces, negated back, as
      // contiguous rows (partial-line stores are slow).  The delta rule
      // keeps the even chunks only (its backward rebuilds the odd ones);
      // adam every chunk.
      if (p.states && (RULE == 2 || (i & 1) == 0)) {
        const int64_t plane = RULE == 2 ? bh * N + i : bh * ((N + 1) / 2) + i / 2;
        float* sp = p.states + (plane * D + 32 * blk) * (int64_t)D;
#pragma unroll
        for (int k = 0; k < NCK; ++k) {
          const lds_cptr src = L0 + (L::SP0 + sbo + cko[k]);
          const bf16x4 hi = lds_ld<bf16x4>(src), lo = lds_ld<bf16x4>(src + 1024);
          *reinterpret_cast<bf16x8*>(sp + ckg[k]) = neg8(cat8(hi, lo));
        }
      }
      __syncthreads();  // barrier i + 1
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        Aq[x] = Ap[x];
        Oq[x] = O[x];
      }
    };
    for (int i = 0; i < N; i += RING) {
      out_chunk(std::integral_constant<int, 0>{}, i);
      if (i + 1 < N) out_chunk(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < N) out_chunk(std::integral_constant<int, 2>{}, i + 2);
    }
    finish_prev(N);
  };
  switch (ow) {
    case 0: run(std::integral_constant<int, 3>{}); break;
    case 1: run(std::integral_constant<int, 2>{}); break;
    case 2: run(std::integral_constant<int, 0>{}); break;
    default: run(std::integral_constant<int, 1>{}); break;
  }
}

template <int D, int RULE>
static hipError_t launch_fwd_rows(const ChunkArgs& a, hipStream_t stream) {
  auto kern = chunk_fwd_rows<D, RULE>;
  constexpr int lds = FwdRowsLds<D, RULE>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (D / 32);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(fd_threads<RULE>()), lds, stream, a);
  return hipGetLastError();
}

hipError_t chunk_fwd_rows_launch(const ChunkArgs& a, int d, int rule, hipStream_t s) {
  if (rule == 0) return d == 128 ? launch_fwd_rows<128, 0>(a, s) : launch_fwd_rows<64, 0>(a, s);
  if (rule == 2 && d == 64) return launch_fwd_rows<64, 2>(a, s);
  return hipErrorNotSupported;
}

}  // namespace gmdn
