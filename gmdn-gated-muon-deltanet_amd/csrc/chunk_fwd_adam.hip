// Level B forward of the adam rule at d = 64 with 16-row workgroups.
//
// The fused E-form (reference train_ablation.py:142-187 with
// fast_scan.py:86-94), as chunk_fwd<D, 2> computes it: per (b, h) and chunk i
// with state S_i,
//   E = V - K S_i^T,   o = Q S_i^T + tril(Q K^T) diag(beta) E,
//   G = E^T K,  M <- m M + (1-m) G,  V <- n V + (1-n) G^2,
//   S_{i+1} = a S_i + b M / (sqrt(V) + eps).
// Row r of G needs only row r of S (column r of E), and the moment update is
// elementwise, so the rows of the state evolve independently: a workgroup
// owns 16 rows for the whole sequence (B H D / 16 workgroups, the D/16 of
// one (b, h) on one XCD), twice the grid of the 32-row kernel.
//
// Work split: ten waves.
//  * State waves 0-3 (SIMDs 0-3): wave q owns column tile q of the 16 x D
//    state (its moments M, V beside it) and token tile q of E.  Per chunk it
//    forms E's token tile q from every wave's published S pieces (2 k-blocks
//    x hi, lo; K rows are exact bf16), publishes -E of that tile, and after
//    a mid-chunk barrier forms G's column tile q from all four -E tiles,
//    updates M, V, S in registers and publishes its S pieces.  Each wave does
//    a quarter of the row block's products and of the update's VALU work
//    (two quarter-rate transcendentals per value, four values per lane).
//  * Output waves 4-7 own token tiles 0, 1, 3, 2 (the heavier causal rows on
//    SIMDs 2, 3, beside no copy wave): A^T = K Q^T tiles with beta on the
//    key columns, -o^T = Sf Q^T from the published S pieces, and A (-E) one
//    interval later; they store o.
//  * Copy waves 8, 9 issue the LDS-DMA copies of chunk i + 3 after the
//    mid-chunk barrier of chunk i (4-stage ring) and wait for chunk i + 1
//    before it, so that the state waves read chunk i + 1's K and V operands
//    while their moment update runs.  They reduce the chunk scalars a, b, m,
//    n lane-parallel (lane c: chunk 64 J + c) straight from the gate arrays,
//    64 chunks at a time (before the first chunk, then in interval
//    64 J - 1), off every per-chunk chain; only beta is copied per chunk.
//    In the training forward they also store the S_i checkpoint and M_i,
//    V_i from the state waves' LDS pieces, as contiguous 16-byte units.
// The S and -E pieces are exchanged in the MFMA operand's register order:
// the k-block operand of lane l is 16 bytes at 16 l, of which the tile
// u = 0, 1 of the pair writes bytes 8 u .. 8 u + 7 (hi and lo in separate
// planes).  Both are double-buffered by chunk parity.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

#include <type_traits>

namespace gmdn {

namespace {

// An LDS base the compiler cannot see into (keeps ds_read immediates small).
GMDN_DEV lds_cptr opaque(lds_cptr p) {
  uint32_t v = (uint32_t)(uintptr_t)p;
  asm volatile("" : "+v"(v));
  return (lds_cptr)(uintptr_t)v;
}

constexpr int FA_THREADS = 640;
constexpr int FA_RING = 4;  // LDS ring depth: chunk i + 3 is copied in interval i

template <int D>
struct FwdAdamLds {
  static constexpr int NKB = D / 32;
  static constexpr int NCT = D / 16;
  static constexpr int TILE = CB_C * D * 2;  // one Q or K chunk (bytes)
  static constexpr int VT = CB_C * 16 * 2;   // the workgroup's 16 columns of V
  static constexpr int GT = CB_C * 4;        // beta of a chunk
  static constexpr int Q0 = 0;
  static constexpr int K0 = Q0 + FA_RING * TILE;
  static constexpr int V0 = K0 + FA_RING * TILE;
  static constexpr int G0 = V0 + FA_RING * VT;
  // per chunk parity: S pieces [k-block][hi, lo][lane][tile u], 8 bytes
  static constexpr int SPB = NKB * 2 * 1024;
  // per chunk parity: -E pieces [token block][hi, lo][lane][tile u]
  static constexpr int EPB = 2 * 2 * 1024;
  static constexpr int SP0 = G0 + FA_RING * GT;
  static constexpr int EP0 = SP0 + 2 * SPB;
  // {a, b, m, n} of 64 chunks, double-buffered by block parity
  static constexpr int SC0 = EP0 + 2 * EPB;
  // training forward: S_i (split pieces of -Sf), M_i, V_i staged for the
  // copy waves' stores, [chunk parity][S, M, V][row][16-byte unit], unit u4
  // of row R at slot u4 ^ R (both the state waves' writes, 16 rows of one
  // unit, and the copy waves' reads, 16 units of one row, are conflict-free)
  static constexpr int CKP = 16 * (D / 4) * 16;  // one plane: 16 rows x D/4 units
  static constexpr int CKB = 3 * CKP;
  static constexpr int CK0 = SC0 + 2 * 64 * 16;
  static constexpr int BYTES = CK0 + 2 * CKB;
  static_assert(BYTES <= 160 * 1024, "adam forward LDS exceeds the 160 KiB of a CU");
};

}  // namespace

template <int D>
__global__ void __launch_bounds__(FA_THREADS) chunk_fwd_adam16(ChunkArgs p) {
  static_assert(D == 64, "one column tile per state wave: d = 64");
  using LQ = RowSwz<D>;
  using LV = BSwz<16>;
  using L = FwdAdamLds<D>;
  constexpr int NKB = D / 32;
  constexpr int NCT = D / 16;
  constexpr int ROWB = D * 2;  // bytes per Q / K row
  using DQ = DmaPlan<LQ, CB_C, 128>;
  using DV = DmaPlan<LV, CB_C, 128>;
  extern __shared__ __align__(16) char smem[];

  int64_t bh;
  int blk;
  map_block(p.B * p.H, D / 16, bh, blk);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const lds_ptr L0 = lds_base(smem);
  const int N = p.N;

  if (w >= 8) {
    // ========================================================= copy waves
    const int cw = w - 8;
    const uint32_t lds0 = lds_addr(smem);
    const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
    const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
    const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + 16 * blk;
    DQ dq, dk;
    DV dv;
    dq.init(cw, p.sq[2]);
    dk.init(cw, p.sk[2]);
    dv.init(cw, p.sv[2]);
    // beta of the chunk, 16 bytes per lane of wave 8's lanes 0-15
    const float* bsrc = p.beta + bh * p.T + 4 * lc;
    auto issue_loads = [&](int i, int stg) {
      const int64_t t0 = (int64_t)i * CB_C;
      dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + stg * L::TILE, cw);
      dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + stg * L::TILE, cw);
      dv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + stg * L::VT, cw);
      if (cw == 0 && l < 16) lds_dma16(bsrc + t0, smem + L::G0 + stg * L::GT);
    };
    // vector-memory operations of one chunk copy (wave 8 also copies beta)
    constexpr int ND = 2 * DQ::NOPS + DV::NOPS;
    // wait until at most `ahead` chunk copies issued after the awaited one
    // are still in flight
    auto wait_chunks = [&](int ahead) {
      if (cw == 0) {
        if (ahead >= 2)
          wait_vmem_le<2 * (ND + 1)>();
        else if (ahead == 1)
          wait_vmem_le<ND + 1>();
        else
          wait_vmem();
      } else {
        if (ahead >= 2)
          wait_vmem_le<2 * ND>();
        else if (ahead == 1)
          wait_vmem_le<ND>();
        else
          wait_vmem();
      }
    };
    // chunk scalars of chunks 64 J .. 64 J + 63, lane c: chunk 64 J + c.
    // Wave 8: a = exp(sum of max(g, log 1e-6)), b = mean(beta); wave 9: m, n
    // as a from gmu, gnu.  (Its loads complete in order after any copy
    // issued before them.)
    auto scalar_block = [&](int J) {
      const int c = 64 * J + l;
      if (c >= N) return;
      const int64_t t0 = bh * p.T + (int64_t)c * CB_C;
      const float* x0 = (cw == 0 ? p.g : p.gmu) + t0;
      const float* x1 = (cw == 0 ? p.beta : p.gnu) + t0;
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int k = 0; k < CB_C / 4; ++k) {
        const f32x4 u = *reinterpret_cast<const f32x4*>(x0 + 4 * k);
        const f32x4 v = *reinterpret_cast<const f32x4*>(x1 + 4 * k);
        s0 += (fmaxf(u[0], LOG_FLOOR) + fmaxf(u[1], LOG_FLOOR)) + (fmaxf(u[2], LOG_FLOOR) + fmaxf(u[3], LOG_FLOOR));
        if (cw == 0)
          s1 += (v[0] + v[1]) + (v[2] + v[3]);
        else
          s1 += (fmaxf(v[0], LOG_FLOOR) + fmaxf(v[1], LOG_FLOOR)) + (fmaxf(v[2], LOG_FLOOR) + fmaxf(v[3], LOG_FLOOR));
      }
      const f32x2 r = cw == 0 ? f32x2{expf(s0), s1 * (1.f / CB_C)} : f32x2{expf(s0), expf(s1)};
      lds_st<f32x2>(L0 + (L::SC0 + (J & 1) * 1024 + 16 * l + 8 * cw), r);
    };
    // training forward: the checkpoint S_i (split pieces) and M_i, V_i
    // (float32) of the workgroup's 16 rows from the staging, as contiguous
    // 16-byte units: lane L = 64 cw + l stores units f = 128 k + L (row
    // f / (D/4), columns 4 u4 .. 4 u4 + 3 for u4 = f % (D/4)).  The staging
    // of chunk i stays in place until the end of interval i + 1.
    constexpr int UPR = D / 4, NU = 16 * UPR / 128;
    uint32_t cko[NU];
    int64_t ckg[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int f = 128 * k + 64 * cw + l, R = f / UPR, u4 = f % UPR;
      cko[k] = (uint32_t)(R * UPR * 16 + 16 * (u4 ^ R));
      ckg[k] = (int64_t)R * D + 4 * u4;
    }
    const int64_t plane = p.B * p.H * (int64_t)N * D * D;
    auto store_states = [&](int i) {
      if (!p.states) return;
      float* sp = p.states + ((bh * N + i) * D + 16 * blk) * (int64_t)D;
      const lds_cptr ck = L0 + (L::CK0 + (i & 1) * L::CKB);
#pragma unroll
      for (int k = 0; k < NU; ++k) {
        const bf16x8 ss = lds_ld<bf16x8>(ck + cko[k]);
        const f32x4 mm = lds_ld<f32x4>(ck + L::CKP + cko[k]), vv = lds_ld<f32x4>(ck + 2 * L::CKP + cko[k]);
        // streaming stores (read back only by the backward)
        __builtin_nontemporal_store(ss, reinterpret_cast<bf16x8*>(sp + ckg[k]));
        __builtin_nontemporal_store(mm, reinterpret_cast<f32x4*>(sp + plane + ckg[k]));
        __builtin_nontemporal_store(vv, reinterpret_cast<f32x4*>(sp + 2 * plane + ckg[k]));
      }
    };
    const int pre = N < FA_RING - 1 ? N : FA_RING - 1;
    for (int i = 0; i < pre; ++i) issue_loads(i, i);
    scalar_block(0);
    wait_chunks(pre - 1);
    __syncthreads();  // barrier 0
    for (int i = 0; i < N; ++i) {
      // chunk i + 1 (copied since interval i - 2) lands before the mid-chunk
      // barrier; chunk i + 3's copies go out after it, into the stage of
      // chunk i - 1, which nothing reads any more
      if (i + 1 < N) wait_chunks(i + 2 < N ? 1 : 0);
      __syncthreads();  // the mid-chunk barrier of chunk i
      // the stores go out before the next copy: vector-memory operations
      // retire in order, so the copy waits above never wait on them
      store_states(i);
      if (i + 3 < N) issue_loads(i + 3, (i + 3) % FA_RING);
      if ((i & 63) == 63 && i + 1 < N) scalar_block((i + 1) >> 6);
      __syncthreads();  // barrier i + 1
    }
    return;
  }

  // natural-order row operand of a Q or K tile: lane (m, G) takes row
  // 16 tt + m, columns 32 kb + 8G .. +7 (one 16-byte read)
  lds_cptr rowK[NKB], rowQ[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    rowK[kb] = opaque(L0 + (L::K0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
    rowQ[kb] = opaque(L0 + (L::Q0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
  }
  auto row_op = [&](const lds_cptr (&base)[NKB], uint32_t off, int kb) { return lds_ld<bf16x8>(base[kb] + off); };
  // the k-block operands of S (lane l's 16 bytes) and of -E
  const lds_cptr spr = L0 + (L::SP0 + 16 * l);
  const lds_cptr epr = L0 + (L::EP0 + 16 * l);

  if (w < 4) {
    // ========================================================= state waves
    const int q = w;
    // K^T operand of G's column tile q = 2 kb + u: lane (m, G) takes K[s][c]
    // for the pair-order tokens s of block kt and column
    // c = 32 kb + 4u + 8 (m / 4) + m % 4; in transposing reads lane (i, G)
    // addresses row 32 kt + 16 h + 4G + i / 4, columns 32 kb + 4u + 8 (i % 4) ..
    const lds_cptr colp =
        opaque(L0 + (L::K0 + swz_off<LQ>(4 * G + (lc >> 2), 32 * (q >> 1) + 4 * (q & 1) + 8 * (lc & 3))));
    auto col_op = [&](uint32_t off, int kt) {
      return cat8(lds_tr16(colp + off + 32 * kt * ROWB), lds_tr16(colp + off + (32 * kt + 16) * ROWB));
    };
    // V: tokens 16 q + 4G + j of the workgroup's column lc
    const lds_cptr vp = L0 + (L::V0 + q * 16 * 32 + swz_off<LV>(4 * G + (lc >> 2), 4 * (lc & 3)));
    // this wave's 8-byte slots: S pieces of column tile q, -E of token tile q
    const lds_ptr spw = L0 + (L::SP0 + (q >> 1) * 2048 + 16 * l + 8 * (q & 1));
    const lds_ptr epw = L0 + (L::EP0 + (q >> 1) * 2048 + 16 * l + 8 * (q & 1));

    // -S, M, V: lane (r, G) holds columns 32 (q / 2) + 8G + 4 (q % 2) + j of row r
    f32x4 Sf = zero4(), Mm = zero4(), Vv = zero4();
    // the staging slot of this lane's unit: row lc, columns
    // 32 (q / 2) + 8G + 4 (q % 2) .. +3, i.e. unit u4 = 8 (q / 2) + 2G + q % 2
    const lds_ptr ckw = L0 + (L::CK0 + lc * (D / 4) * 16 + 16 * ((8 * (q >> 1) + 2 * G + (q & 1)) ^ lc));
    // publish S_i's pieces (for E and the output waves) and, in the
    // training forward, stage S_i, M_i, V_i for the copy waves' stores
    auto publish_s = [&](int i) {
      bf16x4 hi, lo;
      split4(Sf, hi, lo);
      const uint32_t par = (uint32_t)(i & 1);
      lds_st<bf16x4>(spw + par * L::SPB, hi);
      lds_st<bf16x4>(spw + par * L::SPB + 1024, lo);
      if (p.states && i < N) {
        const lds_ptr ck = ckw + par * L::CKB;
        lds_st<bf16x8>(ck, neg8(cat8(hi, lo)));
        lds_st<f32x4>(ck + L::CKP, Mm);
        lds_st<f32x4>(ck + 2 * L::CKP, Vv);
      }
    };
    // chunk i's operands that do not depend on the state: K rows of token
    // tile q, V, and G's K^T operands (read one interval ahead)
    struct Ops {
      bf16x8 Kr[NKB], Kc[2];
      bf16x4 vb;
    };
    auto load_ops = [&](auto stg_tag) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      Ops o;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) o.Kc[kt] = col_op(SQK, kt);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) o.Kr[kb] = row_op(rowK, SQK + q * 16 * ROWB, kb);
      o.vb = lds_tr16(vp + STG * L::VT);
      return o;
    };
    publish_s(0);
    __syncthreads();  // barrier 0: chunk 0 landed, S_0 published
    Ops cur = load_ops(std::integral_constant<int, 0>{});

    auto state_chunk = [&](auto stg_tag, int i) {
      constexpr int STG = decltype(stg_tag)::value;
      // E = V + K Sf^T, token tile q, from every wave's S_i pieces
      const uint32_t so = (uint32_t)(i & 1) * L::SPB;
      bf16x8 Sr[NKB][2];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) Sr[kb][pc] = lds_ld<bf16x8>(spr + so + kb * 2048 + pc * 1024);
      const f32x4 sc = lds_ld<f32x4>(L0 + (L::SC0 + ((i >> 6) & 1) * 1024 + (i & 63) * 16));
      f32x4 E = f32x4{(float)cur.vb[0], (float)cur.vb[1], (float)cur.vb[2], (float)cur.vb[3]};
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        E = mfma(cur.Kr[kb], Sr[kb][0], E);
        E = mfma(cur.Kr[kb], Sr[kb][1], E);
      }
      // the parts of the update that do not depend on G
      const float a = sc[0], b = sc[1], m = sc[2], n = sc[3];
      const float cm = 1.f - m, cn = 1.f - n;
      const f32x4 aS = a * Sf, mM = m * Mm, nV = n * Vv;
      // -E of token tile q, published for the other state waves (G) and the
      // output waves (A E, next interval)
      const uint32_t eo = (uint32_t)(i & 1) * L::EPB;
      {
        bf16x4 hi, lo;
        split4(-E, hi, lo);
        lds_st<bf16x4>(epw + eo, hi);
        lds_st<bf16x4>(epw + eo + 1024, lo);
      }
      __syncthreads();  // mid-chunk barrier: every token tile's -E published
      bf16x8 We[2][2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) We[kt][pc] = lds_ld<bf16x8>(epr + eo + kt * 2048 + pc * 1024);
      // Gn = K^T (-E) = -G^T, column tile q
      f32x4 Gn = zero4();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        Gn = mfma(cur.Kc[kt], We[kt][0], Gn);
        Gn = mfma(cur.Kc[kt], We[kt][1], Gn);
      }
      // chunk i + 1's operands (landed before the mid-chunk barrier), read
      // while the update runs
      if (i + 1 < N) cur = load_ops(std::integral_constant<int, (STG + 1) % FA_RING>{});
      //   M = m M + (1 - m) G,  V = n V + (1 - n) G^2,
      //   Sf = a Sf - b M / (sqrt(V) + eps)
      Mm = mM - cm * Gn;
      Vv = nV + cn * (Gn * Gn);
#pragma unroll
      for (int j = 0; j < 4; ++j) Sf[j] = aS[j] - b * Mm[j] * hw_rcp(hw_sqrt(Vv[j]) + p.eps);
      publish_s(i + 1);
      __syncthreads();  // barrier i + 1
    };
    for (int i = 0; i < N; i += FA_RING) {
      state_chunk(std::integral_constant<int, 0>{}, i);
      if (i + 1 < N) state_chunk(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < N) state_chunk(std::integral_constant<int, 2>{}, i + 2);
      if (i + 3 < N) state_chunk(std::integral_constant<int, 3>{}, i + 3);
    }
    return;
  }

  // ========================================================== output waves
  // waves 4, 5, 6, 7 take token tiles 0, 1, 3, 2
  const int ow = w - 4;
  bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + 16 * blk + 4 * G;
  __syncthreads();  // barrier 0

  auto run = [&](auto tt_tag) {
    constexpr int TT = decltype(tt_tag)::value;
    constexpr int NKT = TT >= 2 ? 2 : 1;  // token blocks of A with s <= t
    Op<2> Ap[2], Aq[2];                   // this chunk's and the previous chunk's A pieces
    f32x4 O = zero4(), Oq = zero4();      // -o^T tiles, likewise
    const bf16x8 z8 = bf16x8{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      Ap[x].v[0] = Ap[x].v[1] = z8;
      Aq[x] = Ap[x];
    }
    auto finish_prev = [&](int i) {  // o_{i-1} += A diag(beta) E, stored
      const uint32_t eo = (uint32_t)((i - 1) & 1) * L::EPB;
      bf16x8 We[2][2];
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) We[kt][pc] = lds_ld<bf16x8>(epr + eo + kt * 2048 + pc * 1024);
      // (hi, hi), (hi, lo), (lo, hi) of each operand pair
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int pc = 0; pc < 3; ++pc) Oq = mfma(We[kt][pc == 2 ? 1 : 0], Aq[kt].v[pc == 1 ? 1 : 0], Oq);
      // lane (t, G): token 16 TT + t, state rows 4G ..
      *reinterpret_cast<bf16x4*>(og + ((int64_t)(i - 1) * CB_C + 16 * TT + lc) * p.so[2]) = to_bf16x4(-Oq);
    };
    auto out_chunk = [&](auto stg_tag, int i) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      if (i >= 1) finish_prev(i);
      __syncthreads();  // the mid-chunk barrier of chunk i
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
      // beta on A's key columns s (the state waves publish -E, not -beta E)
#pragma unroll
      for (int st = 0; st <= TT; ++st) At[st] *= lds_ld<f32x4>(L0 + (L::G0 + STG * L::GT + 4 * (16 * st + 4 * G)));
      // keep s <= t on the diagonal tile: lane (t, G) row 4G + j is s
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * G + j > lc) At[TT][j] = 0.f;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) Ap[kt] = pack_tiles<2>(At[2 * kt], At[2 * kt + 1]);
      // -o^T = Sf Q^T (+ A (-E) next interval)
      const uint32_t sbo = (uint32_t)(i & 1) * L::SPB;
      bf16x8 Sr[NKB][2];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) Sr[kb][pc] = lds_ld<bf16x8>(spr + sbo + kb * 2048 + pc * 1024);
      O = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) O = mfma(Sr[kb][pc], Qr[kb], O);
      __syncthreads();  // barrier i + 1
#pragma unroll
      for (int x = 0; x < 2; ++x) Aq[x] = Ap[x];
      Oq = O;
    };
    for (int i = 0; i < N; i += FA_RING) {
      out_chunk(std::integral_constant<int, 0>{}, i);
      if (i + 1 < N) out_chunk(std::integral_constant<int, 1>{}, i + 1);
      if (i + 2 < N) out_chunk(std::integral_constant<int, 2>{}, i + 2);
      if (i + 3 < N) out_chunk(std::integral_constant<int, 3>{}, i + 3);
    }
    finish_prev(N);
  };
  switch (ow) {
    case 0: run(std::integral_constant<int, 0>{}); break;
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 3>{}); break;
    default: run(std::integral_constant<int, 2>{}); break;
  }
}

hipError_t chunk_fwd_adam16_launch(const ChunkArgs& a, int d, hipStream_t stream) {
  if (d != 64) return hipErrorNotSupported;
  auto kern = chunk_fwd_adam16<64>;
  constexpr int lds = FwdAdamLds<64>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (64 / 16);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(FA_THREADS), lds, stream, a);
  return hipGetLastError();
}

}  // namespace gmdn
