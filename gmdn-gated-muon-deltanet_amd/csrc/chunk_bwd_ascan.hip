// Level B backward, adam rule at d = 64: the reverse scan of the state and
// moment cotangents with each 16-row block split over four state waves.
//
// Per (b, h), chunks i = N-1 .. 0 with Sb = dL/dS_{i+1}, Mb = dL/dM_{i+1},
// Vb = dL/dV_{i+1} (all zero after the last chunk): the reference's
// manual_backward (fast_scan.py:134-186, adam branch :167-182) in the
// fused E-form (train_ablation.py:142-187).  With the forward's E = V - K S^T,
// G = E^T K, Mi = m Mp + (1-m) G, Vi = n Vp + (1-n) G^2, den = sqrt(Vi) + eps,
//   Mtot = Mb + b Sb / den,  Vtot = Vb - b Sb Mi / den^2 / (2 max(sqrt(Vi), 1e-12)),
//   Gb = (1-m) Mtot + (1-n) 2 G Vtot,  Mb <- m Mtot,  Vb <- n Vtot,
//   da = <Sb, S>,  db = <Sb, Mi / den>,  dm = <Mtot, Mp - G>,  dn = <Vtot, Vp - G^2>,
//   dE = A^T dO + K Gb^T,  Sb <- a Sb + dO^T Q - dE^T K.
// Row r of Sb_i needs only row r of Sb_{i+1}, and the moment VJP is
// elementwise, so each workgroup owns 16 rows (B H D / 16 workgroups).
// Everything but the cotangents depends on the forward alone and is formed
// one step ahead, off the serial chain.  Gb_i (every chunk, split pieces)
// and the per-(chunk, row block) partial sums of da, db, dm, dn go to the
// token-gradient kernel chunk_bwd_tok<64, 2>.
//
// Work split: ten waves; step j works on chunk c1-1-j of the launch's
// segment, with three barriers Z(j), Y(j), X(j) (phases A, B, C end at them).
//  * State waves 0-3 (SIMDs 0-3): wave q owns column tile q of Sb, Mb, Vb
//    (4 values per lane, the forward's column-permuted state layout) and
//    token tile q of X and -dE.  A: the elementwise VJP of its tile from the
//    step's factors; Gb's tile published as split pieces (the staging the
//    store also reads); the partial products of da, db, dm, dn.  B: X = K Gb^T
//    of token tile q from every wave's Gb pieces, -dE = -(X + P) published.
//    C: Sb^T = a Sb^T + C + K^T (-dE) of column tile q from every token
//    tile's -dE, then, for the next step, G's column tile q from the
//    published -E tiles and the tile's seven elementwise factors (the
//    forward's Mi, Vi recomputed), kept in registers.  Each wave does a
//    quarter of the row block's products and elementwise work.
//  * Token waves 4-7 (tile tw = w - 4), one step ahead.  A: -E = K S^T - V of
//    token tile tw of the next chunk (from the forward's S checkpoint).
//    B: the causal A tiles of key tile {0, 1, 3, 2}[tw] with P = A^T dO, and
//    C = dO^T Q of column tile tw.  C: wave 6 reduces the step's partial sums.
//  * Copy waves 8, 9: the LDS-DMA copies (the chunk's tiles three steps
//    ahead, the checkpoint's rows two), Gb_i's store from the staging, and
//    the chunk scalars a, b, m, n lane-parallel (lane c: chunk 64 J + c) from
//    the gate arrays, 64 chunks at a time.
// LDS rings: K 4 stages (read by the state waves in their step, by the token
// waves in the step before), the checkpoint's rows 2, everything else 3.
// Exchanges of split pieces keep the MFMA operand's register order: lane l's
// 16 bytes at 16 l, of which the tile u = 0, 1 of a pair writes bytes 8 u ..
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

#include <type_traits>

namespace gmdn {

namespace {

constexpr int ASC_THREADS = 640;

GMDN_DEV lds_cptr opaque_ptr(lds_cptr p) {
  uint32_t v = (uint32_t)(uintptr_t)p;
  asm volatile("" : "+v"(v));
  return (lds_cptr)(uintptr_t)v;
}

template <int D>
struct AScanLds {
  static_assert(D == 64, "the adam reverse scan is built for d = 64");
  static constexpr int RK = 4;                   // K ring depth
  static constexpr int TILE = CB_C * D * 2;      // one Q or K chunk (bytes)
  static constexpr int CT = CB_C * 16 * 2;       // the workgroup's 16 columns of V or dO
  static constexpr int RT = 16 * D * 4;          // 16 rows of a float32 (or piece) plane
  static constexpr int BT = CB_C * 4;            // beta of a chunk
  static constexpr int K0 = 0;
  static constexpr int Q0 = K0 + RK * TILE;
  static constexpr int V0 = Q0 + RING * TILE;
  static constexpr int O0 = V0 + RING * CT;
  // the checkpoint's rows: 2 stages, copied two steps ahead
  static constexpr int S0 = O0 + RING * CT;      // S_i pieces (rows)
  static constexpr int M0 = S0 + 2 * RT;         // M_i
  static constexpr int W0 = M0 + 2 * RT;         // V_i (the second moment)
  static constexpr int B0 = W0 + 2 * RT;         // beta ring
  static constexpr int SC0 = B0 + RING * BT;     // {a, b, m, n} of 64 chunks x 2 blocks
  // exchanges, 1 KiB per operand register set
  static constexpr int EX0 = SC0 + 2 * 64 * 16;  // -E pieces [token block 2][hi, lo]
  static constexpr int P0 = EX0 + 4 * 1024;          // [parity][key tile 4]
  static constexpr int C0 = P0 + 2 * 4 * 1024;       // [parity][column tile 4]
  // Gb staging: 16 rows x D/4 units {hi[4], lo[4]}, unit u4 of row r at slot u4 ^ r
  static constexpr int GB0 = C0 + 2 * 4 * 1024;
  static constexpr int ND0 = GB0 + 16 * (D / 4) * 16;  // -dE pieces [token block 2][hi, lo]
  static constexpr int PS0 = ND0 + 4 * 1024;           // partial products [state wave 4]
  static constexpr int BYTES = PS0 + 4 * 1024;
  static_assert(BYTES <= 160 * 1024, "adam reverse scan LDS exceeds the 160 KiB of a CU");
};

}  // namespace

// One launch of the reverse scan: chunks c1 - 1 .. c0 (steps j = 0 ..
// c1 - c0 - 1 on chunk c1 - 1 - j).  Sb, Mb, Vb enter from `carry` unless the
// segment starts at the last chunk, and leave into it unless it ends at
// chunk 0 (each state wave's tiles, [b h][row block][wave][Sb, Mb, Vb][lane]).
struct AScanSeg {
  ChunkArgs p;
  float* carry;
  int c0, c1;
};

template <int D>
__global__ void __launch_bounds__(ASC_THREADS) chunk_bwd_ascan(AScanSeg sg) {
  const ChunkArgs& p = sg.p;
  using LQ = RowSwz<D>;    // Q, K tiles
  using LC = BSwz<16>;     // the workgroup's V, dO columns
  using LR = BSwz<128>;    // float32 / piece rows (256 bytes, as 128 bf16)
  using L = AScanLds<D>;
  constexpr int NKB = D / 32;
  constexpr int ROWB = D * 2;
  constexpr int UPR = D / 4;  // 16-byte units per state row
  using DQ = DmaPlan<LQ, CB_C, 128>;
  using DC = DmaPlan<LC, CB_C, 128>;
  using DR = DmaPlan<LR, 16, 128>;
  extern __shared__ __align__(16) char smem[];

  int64_t bh;
  int blk;
  map_block(p.B * p.H, D / 16, bh, blk);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const lds_ptr L0 = lds_base(smem);
  const int N = p.N;            // chunks of the sequence (the planes' layout)
  const int NS = sg.c1 - sg.c0;  // steps of this launch
  const int ctop = sg.c1 - 1;    // the chunk of step 0
  const int r0 = 16 * blk;  // the workgroup's first state row
  // step t works on chunk ctop - t: K in stage t % 4, the rows in t % 2,
  // the rest in t % 3
  auto kstage = [](int t) { return (uint32_t)((t & 3) * L::TILE); };
  // the chunk scalars {a, b, m, n} of chunk i
  auto scalars = [&](int i) { return lds_ld<f32x4>(L0 + (L::SC0 + ((i >> 6) & 1) * 1024 + (i & 63) * 16)); };

  if (w >= 8) {
    // ========================================================= copy waves
    const int cw = w - 8;
    const uint32_t lds0 = lds_addr(smem);
    const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
    const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
    const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + r0;
    const bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + r0;  // dO
    const int64_t plane = p.B * p.H * (int64_t)N * D * D;
    const float* bsrc = p.beta + bh * p.T + 4 * lc;  // wave 8, lanes 0-15
    DQ dq, dk;
    DC dv, dd;
    DR ds;
    dq.init(cw, p.sq[2]);
    dk.init(cw, p.sk[2]);
    dv.init(cw, p.sv[2]);
    dd.init(cw, p.so[2]);
    ds.init(cw, 2 * D);
    auto issue_loads = [&](int j) {  // the tiles and beta of step j
      const int i = ctop - j, s3 = j % RING, s4 = j % L::RK;
      const int64_t t0 = (int64_t)i * CB_C;
      dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + s4 * L::TILE, cw);
      dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + s3 * L::TILE, cw);
      dv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + s3 * L::CT, cw);
      dd.issue(og + t0 * p.so[2], lds0 + L::O0 + s3 * L::CT, cw);
      if (cw == 0 && l < 16) lds_dma16(bsrc + t0, smem + L::B0 + s3 * L::BT);
    };
    auto issue_rows = [&](int j) {  // the checkpoint rows of step j
      const int i = ctop - j, s2 = j & 1;
      const bf16* st = reinterpret_cast<const bf16*>(p.states + ((bh * N + i) * D + r0) * (int64_t)D);
      ds.issue(st, lds0 + L::S0 + s2 * L::RT, cw);
      ds.issue(st + 2 * plane, lds0 + L::M0 + s2 * L::RT, cw);
      ds.issue(st + 4 * plane, lds0 + L::W0 + s2 * L::RT, cw);
    };
    // operations of one issue_loads (wave 8: and beta)
    constexpr int ND = 2 * DQ::NOPS + 2 * DC::NOPS;
    // everything issued before the last issue_loads landed
    auto wait_landed = [&](bool more) {
      if (!more)
        wait_vmem();
      else if (cw == 0)
        wait_vmem_le<ND + 1>();
      else
        wait_vmem_le<ND>();
    };
    // chunk scalars of chunks 64 J .. 64 J + 63, lane c: chunk 64 J + c.
    // Wave 8: a = exp(sum of max(g, log 1e-6)), b = mean(beta); wave 9: m, n
    // as a from gmu, gnu.  (Its loads complete in order after any copy
    // issued before them.)
    auto scalar_block = [&](int J) {
      const int c = 64 * J + l;
      if (J < 0 || c >= N) return;
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
    // Gb_i's store: units f = 128 k + 64 cw + l of the staging (row f / 16,
    // columns 4 (f % 16) ..), contiguous rows
    constexpr int NU = 16 * UPR / 128;
    uint32_t gso[NU];
    int64_t gsg[NU];
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int f = 128 * k + 64 * cw + l, R = f / UPR, u4 = f % UPR;
      gso[k] = (uint32_t)(L::GB0 + R * UPR * 16 + 16 * (u4 ^ R));
      gsg[k] = (int64_t)R * D + 4 * u4;
    }
    auto store_gb = [&](int j) {
      const int i = ctop - j;
      float* gp = p.gb + ((bh * N + i) * D + r0) * (int64_t)D;
#pragma unroll
      for (int k = 0; k < NU; ++k) *reinterpret_cast<bf16x8*>(gp + gsg[k]) = lds_ld<bf16x8>(L0 + gso[k]);
    };
    const int jtop = ctop >> 6;  // the block of the first step's chunk
    issue_loads(0);
    issue_rows(0);
    if (NS > 1) {
      issue_loads(1);
      issue_rows(1);
    }
    if (NS > 2) issue_loads(2);
    scalar_block(jtop);
    scalar_block(jtop - 1);
    wait_landed(NS > 2);  // steps 0 and 1
    __syncthreads();     // B0
    __syncthreads();     // B1
    __syncthreads();     // B2
    for (int j = 0; j < NS; ++j) {
      const int i = ctop - j;
      // step j + 2's rows go into the stage step j's held (last read in the
      // step before, by the token waves)
      if (j + 2 < NS) issue_rows(j + 2);
      __syncthreads();  // Z
      // entering block J = i / 64 from above: block J - 1 into the parity
      // block J + 1 held (first read 64 steps on)
      if ((i & 63) == 63 && (i >> 6) < jtop) scalar_block((i >> 6) - 1);
      // the stores go out before the next copies: vector-memory operations
      // retire in order, so the wait below never waits on the young copies
      store_gb(j);
      if (j + 3 < NS) issue_loads(j + 3);
      __syncthreads();  // Y
      if (j + 2 < NS) wait_landed(j + 3 < NS);
      __syncthreads();  // X
    }
    return;
  }

  // natural-order row operands of Q, K tiles (lane (m, G): row 16 tt + m,
  // columns 32 kb + 8G .. +7)
  lds_cptr rowK[NKB], rowQ[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    rowK[kb] = opaque_ptr(L0 + (L::K0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
    rowQ[kb] = opaque_ptr(L0 + (L::Q0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
  }
  // transposed operand, column tile ct = 2 kb + u: lane (m, G) takes X[s][c]
  // for the pair-order tokens s of block kt and c = 32 kb + 4u + 8 (m / 4) + m % 4
  auto col_base = [&](int region, int ct) {
    return opaque_ptr(L0 + (region + swz_off<LQ>(4 * G + (lc >> 2), 32 * (ct >> 1) + 4 * (ct & 1) + 8 * (lc & 3))));
  };
  auto col_op = [&](lds_cptr base, uint32_t off, int kt) {
    return cat8(lds_tr16(base + off + 32 * kt * ROWB), lds_tr16(base + off + (32 * kt + 16) * ROWB));
  };
  const lds_ptr xl = L0 + 16 * l;  // register-order exchanges
  constexpr int NPRE = 7;  // rden, qv, g2, Mi/den, Mp - G, Vp - G^2, S
  // G's column tile ct of step t (from the published -E pieces) and the
  // seven elementwise factors of that tile, for the state wave that owns it
  auto factors = [&](int t, lds_cptr colKt, uint32_t rto, f32x4 (&fx)[NPRE]) {
    const uint32_t SK = kstage(t), s2 = (uint32_t)(t & 1) * L::RT;
    bf16x8 NE[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) NE[kt][pc] = lds_ld<bf16x8>(xl + (L::EX0 + kt * 2048 + pc * 1024));
    bf16x8 kc[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) kc[kt] = col_op(colKt, SK, kt);
    const f32x4 sc = scalars(ctop - t);
    const f32x4 Mp = lds_ld<f32x4>(L0 + (L::M0 + s2 + rto));
    const f32x4 Vp = lds_ld<f32x4>(L0 + (L::W0 + s2 + rto));
    const bf16x8 Spc = lds_ld<bf16x8>(L0 + (L::S0 + s2 + rto));
    f32x4 Gn = zero4();  // K^T (-E) = -G^T
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int pc = 0; pc < 2; ++pc) Gn = mfma(kc[kt], NE[kt][pc], Gn);
    const float m = sc[2], n = sc[3];
    const f32x4 Sv = unsplit_piece(Spc);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float g = -Gn[jj];
      const float mi = m * Mp[jj] + (1.f - m) * g;
      const float vi = n * Vp[jj] + (1.f - n) * g * g;
      const float sq = hw_sqrt(vi);
      const float rden = hw_rcp(sq + p.eps);
      fx[0][jj] = rden;                                                 // Mtot = Mb + b Sb rden
      fx[1][jj] = mi * rden * rden * hw_rcp(2.f * fmaxf(sq, 1e-12f));  // Vtot = Vb - b Sb qv
      fx[2][jj] = (1.f - n) * 2.f * g;                                 // Gb = (1-m) Mtot + g2 Vtot
      fx[3][jj] = mi * rden;                                           // db: <Sb, Mi / den>
      fx[4][jj] = Mp[jj] - g;                                          // dm: <Mtot, Mp - G>
      fx[5][jj] = Vp[jj] - g * g;                                      // dn: <Vtot, Vp - G^2>
      fx[6][jj] = Sv[jj];                                              // da: <Sb, S>
    }
  };

  if (w < 4) {
    // ========================================================= state waves
    const int q = w;
    // lane (r, G) of tile q holds columns 32 (q / 2) + 8G + 4 (q % 2) .. +3
    // of row r: unit u4 = 8 (q / 2) + 2G + q % 2 of the Gb staging
    const lds_ptr gbw = L0 + (L::GB0 + lc * UPR * 16 + 16 * ((8 * (q >> 1) + 2 * G + (q & 1)) ^ lc));
    // X's Gb operand of k-block kb: units 8 kb + 2G, 8 kb + 2G + 1 of row lc
    lds_cptr gbr[NKB][2];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int h = 0; h < 2; ++h) gbr[kb][h] = L0 + (L::GB0 + lc * UPR * 16 + 16 * ((8 * kb + 2 * G + h) ^ lc));
    // this wave's 8-byte slots of -dE (token tile q)
    const lds_ptr ndw = L0 + (L::ND0 + (q >> 1) * 2048 + 16 * l + 8 * (q & 1));
    const lds_cptr colK = col_base(L::K0, q);
    // the state-layout tile q of a row plane: lane (r, G) holds columns
    // 32 (q / 2) + 8G + 4 (q % 2) .. +3 of row r (16 bytes)
    const uint32_t rtq = swz_off<LR>(lc, 2 * (32 * (q >> 1) + 8 * G + 4 * (q & 1)));
    f32x4 Sb = zero4(), Mb = zero4(), Vb = zero4();
    f32x4* const cy = reinterpret_cast<f32x4*>(sg.carry) + ((bh * (D / 16) + blk) * 4 + q) * 3 * 64 + l;
    if (sg.c1 < N) {  // the cotangents of the later chunks' segment
      Sb = cy[0];
      Mb = cy[64];
      Vb = cy[128];
    }
    f32x4 f[NPRE];  // the step's elementwise factors (formed in the step before)
    // step t's K operands: the rows of token tile q (X) and K^T of column tile q
    struct KOps {
      bf16x8 Kr[NKB], Kc[2];
    };
    auto load_k = [&](int t) {
      KOps o;
      const uint32_t SK = kstage(t);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) o.Kr[kb] = lds_ld<bf16x8>(rowK[kb] + (SK + q * 16 * ROWB));
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) o.Kc[kt] = col_op(colK, SK, kt);
      return o;
    };
    __syncthreads();  // B0
    KOps ko = load_k(0);
    __syncthreads();  // B1
    factors(0, colK, rtq, f);
    __syncthreads();  // B2
    for (int j = 0; j < NS; ++j) {
      const int i = ctop - j;
      const uint32_t par = (uint32_t)(j & 1);
      // ---- A: the elementwise VJP of the moment update -> Gb, column tile q
      const f32x4 sc = scalars(i);
      const float a = sc[0], b = sc[1], m = sc[2], n = sc[3];
      const f32x4 ub = b * Sb;
      const f32x4 MT = Mb + ub * f[0];
      const f32x4 VT = Vb - ub * f[1];
      const f32x4 Gb = (1.f - m) * MT + f[2] * VT;
      {
        bf16x4 hi, lo;
        split4(Gb, hi, lo);
        lds_st<bf16x8>(gbw, cat8(hi, lo));
      }
      // partial products of da = <Sb, S>, db = <Sb, Mi / den>,
      // dm = <Mtot, Mp - G>, dn = <Vtot, Vp - G^2>
      f32x4 ps = zero4();
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        ps[0] += Sb[jj] * f[6][jj];
        ps[1] += Sb[jj] * f[3][jj];
        ps[2] += MT[jj] * f[4][jj];
        ps[3] += VT[jj] * f[5][jj];
      }
      lds_st<f32x4>(xl + (L::PS0 + q * 1024), ps);
      Mb = m * MT;
      Vb = n * VT;
      Sb = a * Sb;  // the decay part of the update
      __syncthreads();  // Z
      // ---- B: X = K Gb^T, token tile q (lane (r, G): tokens 16 q + 4G + jj),
      // then -dE = -(X + P)
      Op<2> Gp[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Gp[kb] = join_pieces(lds_ld<bf16x8>(gbr[kb][0]), lds_ld<bf16x8>(gbr[kb][1]));
      const f32x4 Pt = lds_ld<f32x4>(xl + (L::P0 + par * 4096 + q * 1024));
      f32x4 X = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) X = mfma(ko.Kr[kb], Gp[kb].v[u], X);
      {
        bf16x4 hi, lo;
        split4(-(X + Pt), hi, lo);
        lds_st<bf16x4>(ndw, hi);
        lds_st<bf16x4>(ndw + 1024, lo);
      }
      __syncthreads();  // Y
      // ---- C: Sb^T = a Sb^T + C + K^T (-dE), column tile q
      bf16x8 NDp[2][2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) NDp[kt][pc] = lds_ld<bf16x8>(xl + (L::ND0 + kt * 2048 + pc * 1024));
      Sb += lds_ld<f32x4>(xl + (L::C0 + par * 4096 + q * 1024));
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int pc = 0; pc < 2; ++pc) Sb = mfma(ko.Kc[kt], NDp[kt][pc], Sb);
      if (j + 1 < NS) {
        ko = load_k(j + 1);
        factors(j + 1, colK, rtq, f);  // -E of step j + 1 was published before Z
      }
      __syncthreads();  // X
    }
    if (sg.c0 > 0) {  // for the earlier chunks' segment
      cy[0] = Sb;
      cy[64] = Mb;
      cy[128] = Vb;
    }
    return;
  }

  // =========================================================== token waves
  // tile tw: token tile tw of -E, column tile tw of G and C, key tile
  // {0, 1, 3, 2}[tw] of A and P
  const int tw = w - 4;
  const lds_cptr vp = L0 + (L::V0 + tw * 16 * 32 + swz_off<LC>(4 * G + (lc >> 2), 4 * (lc & 3)));
  // the S checkpoint's pieces of k-block kb, row lc: columns 32 kb + 8G .. +3 and +4 ..
  lds_cptr sp[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) sp[kb][hf] = opaque_ptr(L0 + (L::S0 + swz_off<LR>(lc, 2 * (32 * kb + 8 * G + 4 * hf))));
  // this wave's 8-byte slots of -E (token tile tw)
  const lds_ptr exw = L0 + (L::EX0 + (tw >> 1) * 2048 + 16 * l + 8 * (tw & 1));
  // dO operand, pair-order tokens of block kt (rows 32 kt + 4G + i / 4 and
  // + 16, the workgroup's columns 4 (i % 4) ..)
  const lds_cptr obase = opaque_ptr(L0 + (L::O0 + swz_off<LC>(4 * G + (lc >> 2), 4 * (lc & 3))));
  const lds_cptr colQ = col_base(L::Q0, tw);

  // A: -E = K S^T - V of step t's chunk, token tile tw (lane (r, G): tokens
  // 16 tw + 4G + jj of row r), published as G's pair-order operand
  auto minus_e = [&](int t) {
    const uint32_t SK = kstage(t), s2 = (uint32_t)(t & 1) * L::RT;
    Op<2> Sp[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sp[kb] = join_pieces(lds_ld<bf16x8>(sp[kb][0] + s2), lds_ld<bf16x8>(sp[kb][1] + s2));
    bf16x8 Kr[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Kr[kb] = lds_ld<bf16x8>(rowK[kb] + (SK + tw * 16 * ROWB));
    const bf16x4 vb = lds_tr16(vp + (t % RING) * L::CT);
    f32x4 NE = f32x4{-(float)vb[0], -(float)vb[1], -(float)vb[2], -(float)vb[3]};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) NE = mfma(Kr[kb], Sp[kb].v[u], NE);
    bf16x4 hi, lo;
    split4(NE, hi, lo);
    lds_st<bf16x4>(exw, hi);
    lds_st<bf16x4>(exw + 1024, lo);
  };
  // the step's partial sums of da, db, dm, dn over the row block, from the
  // state waves' partial products
  auto sums = [&](int j) {
    f32x4 s = lds_ld<f32x4>(xl + L::PS0);
#pragma unroll
    for (int x = 1; x < 4; ++x) s += lds_ld<f32x4>(xl + (L::PS0 + x * 1024));
    const f32x2 s0 = wave_sum2(s[0], s[1]), s1 = wave_sum2(s[2], s[3]);
    if (l == 0)
      *reinterpret_cast<f32x4*>(p.part + ((bh * N + (ctop - j)) * (D / 16) + blk) * 4) =
          f32x4{s0[0], s0[1], s1[0], s1[1]};
  };

  auto run = [&](auto st_tag) {
    constexpr int ST = decltype(st_tag)::value;
    constexpr int KB0 = ST / 2;  // token blocks with t >= s
    // C: P of key tile ST and C of column tile tw for step t
    auto apc = [&](int t) {
      const uint32_t SK = kstage(t), par = (uint32_t)(t & 1);
      const int s3 = t % RING;
      bf16x8 dO8[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        dO8[kt] = cat8(lds_tr16(obase + (s3 * L::CT + 32 * kt * 32)), lds_tr16(obase + (s3 * L::CT + (32 * kt + 16) * 32)));
      bf16x8 Kr[NKB], Qr[4 - ST][NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Kr[kb] = lds_ld<bf16x8>(rowK[kb] + (SK + ST * 16 * ROWB));
#pragma unroll
      for (int tt = ST; tt < 4; ++tt)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) Qr[tt - ST][kb] = lds_ld<bf16x8>(rowQ[kb] + (s3 * L::TILE + tt * 16 * ROWB));
      const float bs = lds_ld<float>(L0 + (L::B0 + s3 * L::BT + 4 * (16 * ST + lc)));
      // A^T operand of key tile ST (m = s, k = t pair order over token block
      // kt) from (Q K^T) D-layout tiles; A[t][s] = (q_t . k_s) beta_s for t >= s
      Op<2> Aop[2];
#pragma unroll
      for (int kt = KB0; kt < 2; ++kt) {
        f32x4 Xt[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int tt = 2 * kt + hf;
          Xt[hf] = zero4();
          if (tt < ST) continue;
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) Xt[hf] = mfma(Qr[tt - ST][kb], Kr[kb], Xt[hf]);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) Xt[hf][jj] = (tt > ST || 4 * G + jj >= lc) ? Xt[hf][jj] * bs : 0.f;
        }
        Aop[kt] = pack_tiles<2>(Xt[0], Xt[1]);
      }
      f32x4 P = zero4();
#pragma unroll
      for (int kt = KB0; kt < 2; ++kt) P = mma<2, 1>(Aop[kt], Op<1>{{dO8[kt]}}, P);
      lds_st<f32x4>(xl + (L::P0 + par * 4096 + ST * 1024), P);
      // C = dO^T Q, column tile tw (transposed, permuted as the state tiles)
      f32x4 Ct = zero4();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) Ct = mfma(col_op(colQ, s3 * L::TILE, kt), dO8[kt], Ct);
      lds_st<f32x4>(xl + (L::C0 + par * 4096 + tw * 1024), Ct);
    };
    __syncthreads();  // B0
    minus_e(0);
    apc(0);
    __syncthreads();  // B1
    __syncthreads();  // B2
    for (int j = 0; j < NS; ++j) {
      const bool ahead = j + 1 < NS;
      if (ahead) minus_e(j + 1);
      __syncthreads();  // Z
      if (ahead) apc(j + 1);
      __syncthreads();  // Y
      if (tw == 2) sums(j);
      __syncthreads();  // X
    }
  };
  switch (tw) {
    case 0: run(std::integral_constant<int, 0>{}); break;
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 3>{}); break;
    default: run(std::integral_constant<int, 2>{}); break;
  }
}

hipError_t chunk_bwd_ascan_launch(const ChunkArgs& a, int d, float* carry, int c0, int c1, hipStream_t stream) {
  if (d != 64 || c0 < 0 || c1 > a.N || c0 >= c1 || ((c0 > 0 || c1 < a.N) && !carry)) return hipErrorInvalidValue;
  auto kern = chunk_bwd_ascan<64>;
  constexpr int lds = AScanLds<64>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (64 / 16);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(ASC_THREADS), lds, stream, AScanSeg{a, carry, c0, c1});
  return hipGetLastError();
}

}  // namespace gmdn
