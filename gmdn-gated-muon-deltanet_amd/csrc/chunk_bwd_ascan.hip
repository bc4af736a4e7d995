// Level B backward, adam rule: the reverse scan of the state and moment
// cotangents with state rows owned by a single wave.
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
// Everything but the cotangents depends on the forward alone, so it is
// formed one step ahead, off the serial chain.  Gb_i (every chunk, split
// pieces) and the per-(chunk, row block) partial sums of da, db, dm, dn go
// to the token-gradient kernel chunk_bwd_tok<64, 2>.
//
// Work split.  A workgroup of eight waves owns 16 rows (B H D / 16
// workgroups); wave w runs on SIMD w % 4.  Step j works on chunk N-1-j; two
// barriers per step, Y(j) in its middle and X(j) at its end.
//  * State wave 0 holds Sb, Mb, Vb of its 16 rows in registers (four tiles
//    each, the column-permuted layout of the forward's state tiles).  Before
//    Y(j): the elementwise VJP from the step's precomputed factors, Gb split
//    into the natural-order operand, X = K Gb^T.  After Y(j): -dE = -(X + P)
//    and Sb^T = a Sb^T + C + K^T (-dE).  It never waits on another wave's
//    work of the same step.
//  * Wave 1 forms, one step ahead, E of the next chunk (from the forward's S
//    checkpoint) and publishes -E as G's operand; after Y(j), the step's
//    partial sums of da, db, dm, dn from what the state wave published.
//  * Token waves 2, 3, 6, 7 (tile tw = 0, 1, 2, 3), one step ahead: before
//    Y(j), the causal A tiles of key tile {0, 1, 3, 2}[tw] with P = A^T dO,
//    C = dO^T Q of column tile tw, and (tw = 0) the chunk scalars; after
//    Y(j), G's column tile tw and
//    its elementwise factors (the forward's Mi, Vi recomputed); after X(j),
//    Gb_i's store from the state wave's LDS staging.
//  * Copy waves 4, 5 issue the LDS-DMA copies (the chunk's tiles three
//    steps ahead, the checkpoint's rows two) and wait for the next-but-one
//    step's chunk.
// LDS rings: K 4 stages (read until the step's own update), the checkpoint's
// rows 2, everything else 3 (read only in the step before).
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

#include <type_traits>

namespace gmdn {

constexpr int ASC_WAVES = 8;
constexpr int ASC_THREADS = 64 * ASC_WAVES;

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
  static constexpr int GT = 4 * CB_C * 4;        // beta, g, gmu, gnu
  static constexpr int K0 = 0;
  static constexpr int Q0 = K0 + RK * TILE;
  static constexpr int V0 = Q0 + RING * TILE;
  static constexpr int O0 = V0 + RING * CT;
  // the checkpoint's rows: 2 stages, copied two steps ahead
  static constexpr int S0 = O0 + RING * CT;      // S_i pieces (rows)
  static constexpr int M0 = S0 + 2 * RT;         // M_i
  static constexpr int W0 = M0 + 2 * RT;         // V_i (the second moment)
  static constexpr int G0 = W0 + 2 * RT;
  // exchanges, 1 KiB per operand register set (lane l's 16 bytes at 16 l)
  static constexpr int EX0 = G0 + RING * GT;     // -E pieces [token block 2][hi, lo]
  static constexpr int NPRE = 7;                 // rden, qv, g2, upd, dMP, dVP, S
  static constexpr int PRE0 = EX0 + 4 * 1024;    // [factor][column tile 4]
  static constexpr int P0 = PRE0 + NPRE * 4 * 1024;  // [parity][key tile 4]
  static constexpr int C0 = P0 + 2 * 4 * 1024;       // [parity][column tile 4]
  static constexpr int GB0 = C0 + 2 * 4 * 1024;      // Gb staging: hi plane, lo plane (16 rows)
  static constexpr int GBP = 16 * D * 2;
  static constexpr int SCL0 = GB0 + 2 * GBP;         // [parity] {a, b, m, n}
  // the state wave's Sb_{i+1}, Mtot, Vtot of the step [3][column tile 4],
  // for wave 1's partial sums of da, db, dm, dn
  static constexpr int XS0 = SCL0 + 2 * 16;
  static constexpr int BYTES = XS0 + 3 * 4 * 1024;
  static_assert(BYTES <= 160 * 1024, "adam reverse scan LDS exceeds the 160 KiB of a CU");
};

template <int D>
__global__ void __launch_bounds__(ASC_THREADS) chunk_bwd_ascan(ChunkArgs p) {
  using LQ = RowSwz<D>;    // Q, K tiles
  using LC = BSwz<16>;     // the workgroup's V, dO columns
  using LR = BSwz<128>;    // float32 / piece rows (256 bytes, as 128 bf16)
  using L = AScanLds<D>;
  constexpr int NKB = D / 32;
  constexpr int NCT = D / 16;
  constexpr int ROWB = D * 2;
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
  const int N = p.N;
  const int r0 = 16 * blk;  // the workgroup's first state row
  // step j works on chunk N - 1 - j: K in stage j % 4, the rest in j % 3

  if (w == 4 || w == 5) {
    // ========================================================= copy waves
    const int cw = w - 4;
    const uint32_t lds0 = lds_addr(smem);
    const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
    const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
    const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + r0;
    const bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + r0;  // dO
    const int64_t plane = p.B * p.H * (int64_t)N * D * D;
    // gates: lanes 0-15 beta, 16-31 g, 32-47 gmu, 48-63 gnu (wave 4)
    const float* gsrc = (G == 0 ? p.beta : G == 1 ? p.g : G == 2 ? p.gmu : p.gnu) + bh * p.T + 4 * lc;
    DQ dq, dk;
    DC dv, dd;
    DR ds;
    dq.init(cw, p.sq[2]);
    dk.init(cw, p.sk[2]);
    dv.init(cw, p.sv[2]);
    dd.init(cw, p.so[2]);
    ds.init(cw, 2 * D);
    auto issue_loads = [&](int j) {  // the tiles and gates of step j
      const int i = N - 1 - j, s3 = j % RING, s4 = j % L::RK;
      const int64_t t0 = (int64_t)i * CB_C;
      dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + s4 * L::TILE, cw);
      dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + s3 * L::TILE, cw);
      dv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + s3 * L::CT, cw);
      dd.issue(og + t0 * p.so[2], lds0 + L::O0 + s3 * L::CT, cw);
      if (cw == 0) lds_dma16(gsrc + t0, smem + L::G0 + s3 * L::GT);
    };
    auto issue_rows = [&](int j) {  // the checkpoint rows of step j
      const int i = N - 1 - j, s2 = j & 1;
      const bf16* st = reinterpret_cast<const bf16*>(p.states + ((bh * N + i) * D + r0) * (int64_t)D);
      ds.issue(st, lds0 + L::S0 + s2 * L::RT, cw);
      ds.issue(st + 2 * plane, lds0 + L::M0 + s2 * L::RT, cw);
      ds.issue(st + 4 * plane, lds0 + L::W0 + s2 * L::RT, cw);
    };
    // operations of one issue_loads (wave 4: and the gates)
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
    issue_loads(0);
    issue_rows(0);
    if (N > 1) {
      issue_loads(1);
      issue_rows(1);
    }
    if (N > 2) issue_loads(2);
    wait_landed(N > 2);  // steps 0 and 1
    __syncthreads();     // B0
    __syncthreads();     // B1
    __syncthreads();     // B2
    // step j + 2's rows go into the stage step j's held: its last reader
    // (the token waves' phase 2 of step j, in the step before) is done
    for (int j = 0; j < N; ++j) {
      if (j + 2 < N) issue_rows(j + 2);
      if (j + 3 < N) issue_loads(j + 3);
      __syncthreads();  // Y
      if (j + 2 < N) wait_landed(j + 3 < N);
      __syncthreads();  // X
    }
    return;
  }

  // natural-order row operands of Q, K tiles (lane (m, G): row 16 rb + m,
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
  // the state-layout tile ct of a row plane: lane (r, G) holds columns
  // 32 (ct / 2) + 8G + 4 (ct % 2) .. +3 of row r (16 bytes)
  auto rtile_off = [&](int ct) { return swz_off<LR>(lc, 2 * (32 * (ct >> 1) + 8 * G + 4 * (ct & 1))); };
  const lds_ptr xl = L0 + 16 * l;  // register-order exchanges
  auto kstage = [](int t) { return (uint32_t)((t & 3) * L::TILE); };
  auto stage3 = [](int t) { return t % RING; };

  if (w == 0) {
    // ========================================================= state wave
    lds_cptr colK[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) colK[ct] = col_base(L::K0, ct);
    f32x4 Sb[NCT], Mb[NCT], Vb[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) Sb[ct] = Mb[ct] = Vb[ct] = zero4();
    // Gb staging, hi and lo planes: unit q = 8 kb + 2G + h (columns 4q ..
    // 4q + 3) of row lc at unit q ^ (lc & 7)
    lds_ptr gsw[2];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) gsw[hf] = L0 + (L::GB0 + lc * D * 2 + 8 * ((2 * G + hf) ^ (lc & 7)));
    __syncthreads();  // B0
    __syncthreads();  // B1
    __syncthreads();  // B2
    for (int j = 0; j < N; ++j) {
      const int i = N - 1 - j;
      const uint32_t SK = kstage(j), par = (uint32_t)(j & 1);
      lds_cptr kr[NKB], kc[NCT];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) kr[kb] = rowK[kb] + SK;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) kc[ct] = colK[ct] + SK;
      // every read of the step's first half issued at once, in the order used:
      // the scalars, Gb's factors (rden, qv, g2), the K rows of X
      const f32x4 sc = lds_ld<f32x4>(L0 + (L::SCL0 + par * 16));
      f32x4 f0[NCT], f1[NCT], f2[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        f0[ct] = lds_ld<f32x4>(xl + (L::PRE0 + (0 * 4 + ct) * 1024));
        f1[ct] = lds_ld<f32x4>(xl + (L::PRE0 + (1 * 4 + ct) * 1024));
        f2[ct] = lds_ld<f32x4>(xl + (L::PRE0 + (2 * 4 + ct) * 1024));
      }
      bf16x8 Kr[4][NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int st = 0; st < 4; ++st) Kr[st][kb] = lds_ld<bf16x8>(kr[kb] + st * 16 * ROWB);
      __builtin_amdgcn_sched_barrier(0);
      const float a = sc[0], b = sc[1], m = sc[2], n = sc[3];
      // ---- the elementwise VJP of the moment update -> Gb, tile by tile
      f32x4 Gb[NCT], S0[NCT], MT[NCT], VT[NCT];
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const f32x4 ub = b * Sb[ct];
        MT[ct] = Mb[ct] + ub * f0[ct];
        VT[ct] = Vb[ct] - ub * f1[ct];
        Gb[ct] = (1.f - m) * MT[ct] + f2[ct] * VT[ct];
        Mb[ct] = m * MT[ct];
        Vb[ct] = n * VT[ct];
        S0[ct] = Sb[ct];
        Sb[ct] = a * Sb[ct];  // the decay part of the update (X needs Gb only)
      }
      Op<2> Gp[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Gp[kb] = pack_tiles<2>(Gb[2 * kb], Gb[2 * kb + 1]);
      __builtin_amdgcn_sched_barrier(0);
      // ---- X = K Gb^T (lane (r, G) of tile st: tokens 16 st + 4G + jj); Sb,
      // Mtot, Vtot published for wave 1's partial sums meanwhile
      f32x4 X[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) X[st] = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int st = 0; st < 4; ++st) X[st] = mfma(Kr[st][kb], Gp[kb].v[u], X[st]);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        lds_st<f32x4>(xl + (L::XS0 + (0 * 4 + ct) * 1024), S0[ct]);
        lds_st<f32x4>(xl + (L::XS0 + (1 * 4 + ct) * 1024), MT[ct]);
        lds_st<f32x4>(xl + (L::XS0 + (2 * 4 + ct) * 1024), VT[ct]);
      }
      bf16x8 Kc[2][NCT];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Kc[kt][ct] = col_op(kc[ct], 0, kt);
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        if (k < 12) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // Y
      // ---- -dE = -(X + P), then Sb^T = a Sb^T + C + K^T (-dE)
      f32x4 Pt[4], Ct[NCT];
#pragma unroll
      for (int st = 0; st < 4; ++st) Pt[st] = lds_ld<f32x4>(xl + (L::P0 + par * 4096 + st * 1024));
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) Ct[ct] = lds_ld<f32x4>(xl + (L::C0 + par * 4096 + ct * 1024));
      Op<2> ND[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) ND[kt] = pack_tiles<2>(-(X[2 * kt] + Pt[2 * kt]), -(X[2 * kt + 1] + Pt[2 * kt + 1]));
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) Sb[ct] += Ct[ct];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) Sb[ct] = mfma(Kc[kt][ct], ND[kt].v[u], Sb[ct]);
      // Gb_i to the staging planes (the token waves store it after X)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        lds_st<bf16x4>(gsw[0] + 64 * kb, __builtin_shufflevector(Gp[kb].v[0], Gp[kb].v[0], 0, 1, 2, 3));
        lds_st<bf16x4>(gsw[1] + 64 * kb, __builtin_shufflevector(Gp[kb].v[0], Gp[kb].v[0], 4, 5, 6, 7));
        lds_st<bf16x4>(gsw[0] + (64 * kb + L::GBP), __builtin_shufflevector(Gp[kb].v[1], Gp[kb].v[1], 0, 1, 2, 3));
        lds_st<bf16x4>(gsw[1] + (64 * kb + L::GBP), __builtin_shufflevector(Gp[kb].v[1], Gp[kb].v[1], 4, 5, 6, 7));
      }
      __syncthreads();  // X
    }
    return;
  }

  if (w == 1) {
    // ================================================ E wave: -E and scalars
    // -E = K S^T - V of step t's chunk, tiles st (lane (r, G): tokens
    // 16 st + 4G + jj of row r), from the S checkpoint's pieces; published
    // as G's pair-order operand
    const lds_cptr vp = L0 + (L::V0 + swz_off<LC>(4 * G + (lc >> 2), 4 * (lc & 3)));
    lds_cptr sp[NKB][2];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) sp[kb][hf] = opaque_ptr(L0 + (L::S0 + swz_off<LR>(lc, 2 * (32 * kb + 8 * G + 4 * hf))));
    auto prep = [&](int t) {
      const uint32_t SK = kstage(t);
      const int s3 = stage3(t);
      Op<2> Sp[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        Sp[kb] = join_pieces(lds_ld<bf16x8>(sp[kb][0] + (t & 1) * L::RT), lds_ld<bf16x8>(sp[kb][1] + (t & 1) * L::RT));
      bf16x8 Kr[4][NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int st = 0; st < 4; ++st) Kr[st][kb] = lds_ld<bf16x8>(rowK[kb] + (SK + st * 16 * ROWB));
      f32x4 NE[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const bf16x4 vb = lds_tr16(vp + (s3 * L::CT + st * 16 * 32));
        NE[st] = f32x4{-(float)vb[0], -(float)vb[1], -(float)vb[2], -(float)vb[3]};
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int st = 0; st < 4; ++st) NE[st] = mfma(Kr[st][kb], Sp[kb].v[u], NE[st]);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const Op<2> ne = pack_tiles<2>(NE[2 * kt], NE[2 * kt + 1]);
#pragma unroll
        for (int u = 0; u < 2; ++u) lds_st<bf16x8>(xl + (L::EX0 + (kt * 2 + u) * 1024), ne.v[u]);
      }
    };
    __syncthreads();  // B0
    prep(0);
    __syncthreads();  // B1
    __syncthreads();  // B2
    for (int j = 0; j < N; ++j) {
      // the partial sums' factors of step j (the token waves overwrite them
      // after Y): Mi / den, Mp - G, Vp - G^2, S
      f32x4 fu[4], fm[4], fv[4], fs[4];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        fu[ct] = lds_ld<f32x4>(xl + (L::PRE0 + (3 * 4 + ct) * 1024));
        fm[ct] = lds_ld<f32x4>(xl + (L::PRE0 + (4 * 4 + ct) * 1024));
        fv[ct] = lds_ld<f32x4>(xl + (L::PRE0 + (5 * 4 + ct) * 1024));
        fs[ct] = lds_ld<f32x4>(xl + (L::PRE0 + (6 * 4 + ct) * 1024));
      }
      if (j + 1 < N) prep(j + 1);
      __syncthreads();  // Y
      // da = <Sb, S>, db = <Sb, Mi / den>, dm = <Mtot, Mp - G>, dn = <Vtot, Vp - G^2>
      // over the row block (the state wave published Sb, Mtot, Vtot before Y)
      float da = 0.f, db = 0.f, dm = 0.f, dn = 0.f;
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const f32x4 sb = lds_ld<f32x4>(xl + (L::XS0 + (0 * 4 + ct) * 1024));
        const f32x4 mt = lds_ld<f32x4>(xl + (L::XS0 + (1 * 4 + ct) * 1024));
        const f32x4 vt = lds_ld<f32x4>(xl + (L::XS0 + (2 * 4 + ct) * 1024));
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          da += sb[jj] * fs[ct][jj];
          db += sb[jj] * fu[ct][jj];
          dm += mt[jj] * fm[ct][jj];
          dn += vt[jj] * fv[ct][jj];
        }
      }
      const f32x2 s0 = wave_sum2(da, db), s1 = wave_sum2(dm, dn);
      if (l == 0)
        *reinterpret_cast<f32x4*>(p.part + ((bh * N + (N - 1 - j)) * (D / 16) + blk) * 4) =
            f32x4{s0[0], s0[1], s1[0], s1[1]};
      __syncthreads();  // X
    }
    return;
  }

  // =========================================================== token waves
  // tile tw: key tile {0, 1, 3, 2}[tw] of A and P, column tile tw of C and G
  const int tw = (w & 1) | ((w >> 1) & 2);  // 2 -> 0, 3 -> 1, 6 -> 2, 7 -> 3
  // dO operand, pair-order tokens of block kt (rows 32 kt + 4G + i / 4 and
  // + 16, the workgroup's columns 4 (i % 4) ..)
  const lds_cptr obase = opaque_ptr(L0 + (L::O0 + swz_off<LC>(4 * G + (lc >> 2), 4 * (lc & 3))));
  const lds_cptr colQ = col_base(L::Q0, tw), colKt = col_base(L::K0, tw);
  const uint32_t rto = rtile_off(tw);
  // Gb stores: 1 KiB of contiguous rows per wave; unit f = 64 tw + l of the
  // staging (row f / 16, columns 4 (f % 16) ..)
  const int gr = (64 * tw + l) >> 4, gq = (64 * tw + l) & 15;
  const uint32_t glo = (uint32_t)(L::GB0 + gr * D * 2 + 8 * (gq ^ (gr & 7)));
  auto store_gb = [&](int j) {
    const int i = N - 1 - j;
    const bf16x8 v = cat8(lds_ld<bf16x4>(L0 + glo), lds_ld<bf16x4>(L0 + (glo + L::GBP)));
    float* gp = p.gb + ((bh * N + i) * D + r0 + gr) * (int64_t)D + 4 * gq;
    *reinterpret_cast<bf16x8*>(gp) = v;
  };
  auto run = [&](auto st_tag) {
    constexpr int ST = decltype(st_tag)::value;
    constexpr int KB0 = ST / 2;  // token blocks with t >= s
    // phase 1 of step t: P of key tile ST and C of column tile tw
    auto phase1 = [&](int t) {
      const uint32_t SK = kstage(t), par = (uint32_t)(t & 1);
      const int s3 = stage3(t);
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
      const float bs = lds_ld<float>(L0 + (L::G0 + s3 * L::GT + 4 * (16 * ST + lc)));
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
      if (tw == 0) {  // the chunk scalars a, b, m, n into slot t & 1
        const lds_cptr gg = L0 + (L::G0 + s3 * L::GT + 4 * l);
        const f32x2 s0 = wave_sum2(fmaxf(lds_ld<float>(gg + 256), LOG_FLOOR), lds_ld<float>(gg));
        const f32x2 s1 = wave_sum2(fmaxf(lds_ld<float>(gg + 512), LOG_FLOOR), fmaxf(lds_ld<float>(gg + 768), LOG_FLOOR));
        if (l == 0)
          *reinterpret_cast<f32x4*>(smem + L::SCL0 + par * 16) =
              f32x4{expf(s0[0]), s0[1] * (1.f / CB_C), expf(s1[0]), expf(s1[1])};
      }
    };
    // phase 2 of step t: G's column tile tw and the elementwise factors
    auto phase2 = [&](int t) {
      const uint32_t SK = kstage(t), par = (uint32_t)(t & 1);
      const int s3 = stage3(t);
      // every read first: G's operands, then the forward's moments and S
      Op<2> NE[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int u = 0; u < 2; ++u) NE[kt].v[u] = lds_ld<bf16x8>(xl + (L::EX0 + (kt * 2 + u) * 1024));
      bf16x8 kc[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) kc[kt] = col_op(colKt, SK, kt);
      const f32x4 sc = lds_ld<f32x4>(L0 + (L::SCL0 + par * 16));
      const uint32_t s2 = (uint32_t)(t & 1) * L::RT;
      const f32x4 Mp = lds_ld<f32x4>(L0 + (L::M0 + s2 + rto));
      const f32x4 Vp = lds_ld<f32x4>(L0 + (L::W0 + s2 + rto));
      const bf16x8 Spc = lds_ld<bf16x8>(L0 + (L::S0 + s2 + rto));
      __builtin_amdgcn_sched_barrier(0);
      f32x4 Gn = zero4();  // K^T (-E) = -G^T
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int u = 0; u < 2; ++u) Gn = mfma(kc[kt], NE[kt].v[u], Gn);
      const float m = sc[2], n = sc[3];
      const f32x4 Sv = unsplit_piece(Spc);
      f32x4 f[L::NPRE];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float g = -Gn[jj];
        const float mi = m * Mp[jj] + (1.f - m) * g;
        const float vi = n * Vp[jj] + (1.f - n) * g * g;
        const float sq = hw_sqrt(vi);
        const float rden = hw_rcp(sq + p.eps);
        f[0][jj] = rden;                                                  // Mtot = Mb + b Sb rden
        f[1][jj] = mi * rden * rden * hw_rcp(2.f * fmaxf(sq, 1e-12f));   // Vtot = Vb - b Sb qv
        f[2][jj] = (1.f - n) * 2.f * g;                                  // Gb = (1-m) Mtot + g2 Vtot
        f[3][jj] = mi * rden;                                            // db: <Sb, Mi / den>
        f[4][jj] = Mp[jj] - g;                                           // dm: <Mtot, Mp - G>
        f[5][jj] = Vp[jj] - g * g;                                       // dn: <Vtot, Vp - G^2>
        f[6][jj] = Sv[jj];                                               // da: <Sb, S>
      }
#pragma unroll
      for (int x = 0; x < L::NPRE; ++x) lds_st<f32x4>(xl + (L::PRE0 + (x * 4 + tw) * 1024), f[x]);
    };
    __syncthreads();  // B0
    phase1(0);
    __syncthreads();  // B1
    phase2(0);
    __syncthreads();  // B2
    for (int j = 0; j < N; ++j) {
      if (j >= 1) store_gb(j - 1);  // staged by the state wave before X(j - 1)
      if (j + 1 < N) phase1(j + 1);
      __syncthreads();  // Y
      if (j + 1 < N) phase2(j + 1);
      __syncthreads();  // X
    }
    store_gb(N - 1);
  };
  switch (tw) {
    case 0: run(std::integral_constant<int, 0>{}); break;
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 3>{}); break;
    default: run(std::integral_constant<int, 2>{}); break;
  }
}

hipError_t chunk_bwd_ascan_launch(const ChunkArgs& a, int d, hipStream_t stream) {
  if (d != 64) return hipErrorNotSupported;
  auto kern = chunk_bwd_ascan<64>;
  constexpr int lds = AScanLds<64>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (64 / 16);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(ASC_THREADS), lds, stream, a);
  return hipGetLastError();
}

}  // namespace gmdn
