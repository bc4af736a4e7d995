// Level B forward of the delta rule with state rows owned by single waves.
//
// Same mathematics as chunk_fwd<D, 0> (reference train_ablation.py:142-187
// with fast_scan.py:72-85, E-form): per (b, h) and chunk i with state S_i,
//   E = V - K S_i^T,   o = Q S_i^T + tril(Q K^T) diag(beta) E,
//   S_{i+1} = a S_i + E^T diag(beta) K.
// (Adam at d = 64 runs chunk_fwd_adam16, whose rows split over four waves.)
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
//    E -> G -> S_{i+1} -> the next E needs no exchange and no barrier.  The
//    state is held
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
// Splitting each row block's state work over two waves (a mid-chunk barrier
// exchanging the halves of E) measured slower: the output waves became the
// chain.
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

constexpr int FD_THREADS = 512;  // eight waves, two per SIMD

template <int D, int RULE>
struct FwdRowsLds {
  static constexpr int NKB = D / 32;
  static constexpr int TILE = CB_C * D * 2;  // one Q or K chunk (bytes)
  static constexpr int VT = CB_C * 32 * 2;   // the workgroup's 32 columns of V
  static constexpr int GT = 2 * CB_C * 4;  // beta and g of a chunk
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
  // the chunk decay a per ring stage
  static constexpr int SC0 = EP0 + 2 * 2 * EPW;
  static constexpr int BYTES = SC0 + RING * 16;
  static_assert(BYTES <= 160 * 1024, "delta forward LDS exceeds the 160 KiB of a CU");
};

template <int D, int RULE>
__global__ void __launch_bounds__(FD_THREADS) chunk_fwd_rows(ChunkArgs p) {
  static_assert(RULE == 0, "the delta rule (adam runs chunk_fwd_adam16)");
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

  // state waves 0, 1, output waves 2, 3, 6, 7, copy waves 4, 5
  if (w == 4 || w == 5) {
    // ========================================================= copy waves
    const int cw = w - 4;
    const uint32_t lds0 = lds_addr(smem);
    const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
    const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
    const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + 32 * blk;
    // gates, 16 bytes per lane: wave 4 lanes 0-15 beta, 16-31 g
    const float* gsrc = (G == 0 ? p.beta : p.g) + bh * p.T + 4 * lc;
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
      if (cw == 0 && l < 32) lds_dma16(gsrc + t0, smem + L::G0 + stg * L::GT);
    };
    // vector-memory operations this wave issues per chunk copy
    constexpr int ND = 2 * DQ::NOPS + DV::NOPS;
    // chunk i + 1 landed (the copy of chunk i + 2, if issued, in flight)
    auto wait_next = [&](bool issued) {
      if (!issued)
        wait_vmem();
      else if (cw == 0)
        wait_vmem_le<ND + 1>();
      else
        wait_vmem_le<ND>();
    };
    // a = exp(sum over the chunk of max(g, log 1e-6)) of the chunk in stage
    // stg (wave 4)
    auto decay = [&](int stg) {
      if (cw != 0) return;
      const lds_cptr gg = L0 + (L::G0 + stg * L::GT + 4 * l);
      const float a = expf(wave_sum(fmaxf(lds_ld<float>(gg + 256), LOG_FLOOR)));
      if (l == 0) *reinterpret_cast<float*>(smem + L::SC0 + stg * 16) = a;
    };
    issue_loads(0, 0);
    if (N > 1) issue_loads(1, 1);
    wait_next(N > 1);
    decay(0);
    __syncthreads();  // barrier 0
    for (int i = 0; i < N; ++i) {
      const bool dma = i + 2 < N;
      if (dma) issue_loads(i + 2, (i + 2) % RING);
      if (i + 1 < N) {
        wait_next(dma);
        decay((i + 1) % RING);
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

  if (w < 2) {
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
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) Sf[ct] = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sp[kb] = pack_tiles<2>(Sf[2 * kb], Sf[2 * kb + 1]);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) lds_st<bf16x8>(spw + (kb * 2 + u) * 1024, Sp[kb].v[u]);
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
#pragma unroll
      for (int st = 0; st < 4; ++st) bt[st] = lds_ld<f32x4>(bp + (STG * L::GT + st * 64));
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
      auto we_block = [&](int kt) {  // -beta E
        WE[kt] = pack_tiles<2>(-(bt[2 * kt] * E[2 * kt]), -(bt[2 * kt + 1] * E[2 * kt + 1]));
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
  const int ow = (w & 1) | ((w >> 1) & 2);
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + 32 * blk + 4 * G;
  const lds_cptr spr = L0 + (L::SP0 + 16 * l);
  constexpr int UPR = D / 4;
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
  const lds_cptr epr = L0 + (L::EP0 + 16 * l);
  __syncthreads();  // barrier 0

  auto run = [&](auto tt_tag) {
    constexpr int TT = decltype(tt_tag)::value;
    constexpr int NKT = TT >= 2 ? 2 : 1;  // token blocks of A with s <= t
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
      if (i >= 1) finish_prev(i);
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
      // contiguous rows (partial-line stores are slow): the even chunks
      // only (the backward rebuilds the odd ones)
      if (p.states && (i & 1) == 0) {
        const int64_t plane = bh * ((N + 1) / 2) + i / 2;
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
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(FD_THREADS), lds, stream, a);
  return hipGetLastError();
}

hipError_t chunk_fwd_rows_launch(const ChunkArgs& a, int d, int rule, hipStream_t s) {
  if (rule == 0) return d == 128 ? launch_fwd_rows<128, 0>(a, s) : launch_fwd_rows<64, 0>(a, s);
  return hipErrorNotSupported;
}

}  // namespace gmdn
