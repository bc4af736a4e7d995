// Level B backward, delta rule: the reverse scan of the state cotangent with
// state rows owned by single waves.
//
// Per (b, h), chunks i = N-1 .. 0 with Sb = dL/dS_{i+1} (Sb_N = 0), the
// reference's mixer core (train_ablation.py:142-187) differentiated through
// its scan (fast_scan.py:72-95) in the E-form:
//   dE = diag(beta) K Sb^T + A^T dO           (A = tril(Q K^T) diag(beta))
//   Sb <- a_i Sb + dO^T Q - dE^T K            (= dL/dS_i)
// The state cotangent Gb_i = Sb_{i+1} of the odd chunks is stored (plane
// i / 2, split pieces) for chunk_bwd_pair, which rebuilds the even chunks'.
//
// Work split.  A workgroup of eight waves, two per SIMD, owns 32 rows of Sb
// (B H D / 32 workgroups, the D/32 of one (b, h) on one XCD); wave w runs on
// SIMD w % 4.  Step j works on chunk N - 1 - j; two barriers per step, Y(j)
// in its middle and X(j) at its end.
//  * State waves 0, 1 each own 16 whole rows and carry the recurrence in
//    registers, as the forward's state waves do.  Before Y(j): X = K Sb^T
//    from the natural-order Sb pieces.  After Y(j): dE = beta X + P, and the
//    transposed update Sb^T = a Sb^T + C - K^T dE, whose K^T operand is read
//    with each 32-column block permuted so that its tiles give the next X's
//    operand in natural order.
//  * Token waves 2, 3, 6, 7 form what does not depend on Sb, one step ahead:
//    between Y(j) and X(j), P = A^T dO of step j + 1 (waves 2, 3, 6, 7 take
//    the key tiles s of 0, 1, 3, 2: five of the ten causal A tiles per SIMD;
//    P is double-buffered by step parity); between X(j) and Y(j + 1),
//    C = dO^T Q of step j + 1 (two column tiles each).  Both are D-layout
//    tiles in the state waves' register order.
//  * Copy waves 4, 5 issue the LDS-DMA copies (step j + 2's chunk after
//    X(j - 1)), wait for step j + 1's chunk before Y(j) and, between Y(j)
//    and X(j), reduce its decay a into an LDS slot.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

#include <type_traits>

namespace gmdn {

constexpr int DSC_WAVES = 8;
constexpr int DSC_THREADS = 64 * DSC_WAVES;

// An LDS base the compiler cannot see into (per-region bases sharing a lane
// offset would otherwise be merged, with offsets past the 16-bit immediate).
GMDN_DEV lds_cptr opaque_lds(lds_cptr p) {
  uint32_t v = (uint32_t)(uintptr_t)p;
  asm volatile("" : "+v"(v));
  return (lds_cptr)(uintptr_t)v;
}

template <int D>
struct DScanLds {
  static constexpr int NCT = D / 16;
  static constexpr int TILE = CB_C * D * 2;  // one Q or K chunk (bytes)
  static constexpr int OT = CB_C * 32 * 2;   // the workgroup's 32 columns of dO
  static constexpr int GT = 2 * CB_C * 4;    // beta and g of a chunk
  static constexpr int Q0 = 0;
  static constexpr int K0 = Q0 + RING * TILE;
  static constexpr int O0 = K0 + RING * TILE;
  static constexpr int G0 = O0 + RING * OT;
  // P tiles [step parity][row tile 2][token tile 4] and C tiles [row tile
  // 2][column tile NCT], 1 KiB each in register order (lane l's 16 bytes at
  // 16 l)
  static constexpr int PB = 2 * 4 * 1024;
  static constexpr int P0 = G0 + RING * GT;
  static constexpr int C0 = P0 + 2 * PB;
  static constexpr int SC0 = C0 + 2 * NCT * 1024;  // chunk decay a per ring stage
  // Gb staging: the workgroup's 32 rows, hi and lo bf16 planes; the 8-byte
  // unit q (columns 4q .. 4q + 3) of row r at unit q ^ (r & 7)
  static constexpr int GS0 = SC0 + RING * 16;
  static constexpr int GSP = 32 * D * 2;  // one plane
  static constexpr int BYTES = GS0 + 2 * GSP;
  static_assert(BYTES <= 160 * 1024, "delta reverse scan LDS exceeds the 160 KiB of a CU");
};

template <int D>
__global__ void __launch_bounds__(DSC_THREADS) chunk_bwd_dscan(ChunkArgs p) {
  // Q, K tiles: the row swizzle under which the permuted transposing reads
  // (four rows by four 16-byte groups per 16 lanes) hit 16 distinct groups
  using LQ = RowSwz<D>;
  using LO = BSwz<32>;
  using L = DScanLds<D>;
  constexpr int NKB = D / 32;  // k-blocks over the state's columns
  constexpr int NCT = D / 16;  // column tiles of a state row block
  constexpr int ROWB = D * 2;  // bytes per Q / K row
  using DQ = DmaPlan<LQ, CB_C, 128>;
  using DO_ = DmaPlan<LO, CB_C, 128>;
  extern __shared__ __align__(16) char smem[];

  int64_t bh;
  int blk;
  map_block(p.B * p.H, D / 32, bh, blk);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const lds_ptr L0 = lds_base(smem);
  const int N = p.N;
  // step j works on chunk N - 1 - j, in ring stage j % RING

  if (w == 4 || w == 5) {
    // ========================================================= copy waves
    const int cw = w - 4;
    const uint32_t lds0 = lds_addr(smem);
    const bf16* qg = p.q + bb * p.sq[0] + hh * p.sq[1];
    const bf16* kg = p.k + bb * p.sk[0] + hh * p.sk[1];
    const bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + 32 * blk;  // dO columns of the block
    // gates: lanes 0-15 beta, 16-31 g (16 bytes each); copied by wave 4's low half
    const float* gsrc = (G == 1 ? p.g : p.beta) + bh * p.T + 4 * lc;
    DQ dq, dk;
    DO_ dd;
    dq.init(cw, p.sq[2]);
    dk.init(cw, p.sk[2]);
    dd.init(cw, p.so[2]);
    auto issue_loads = [&](int i, int stg) {
      const int64_t t0 = (int64_t)i * CB_C;
      dq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + stg * L::TILE, cw);
      dk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + stg * L::TILE, cw);
      dd.issue(og + t0 * p.so[2], lds0 + L::O0 + stg * L::OT, cw);
      if (cw == 0 && l < 32) lds_dma16(gsrc + t0, smem + L::G0 + stg * L::GT);
    };
    constexpr int ND = 2 * DQ::NOPS + DO_::NOPS;  // vector-memory operations per copy
    auto wait_next = [&](bool issued) {  // the next step's chunk landed
      if (!issued)
        wait_vmem();
      else if (cw == 0)
        wait_vmem_le<ND + 1>();
      else
        wait_vmem_le<ND>();
    };
    auto decay = [&](int stg) {  // a = exp(sum over the chunk of max(g, log 1e-6))
      if (cw == 0) {
        const float a = expf(wave_sum(fmaxf(lds_ld<float>(L0 + (L::G0 + stg * L::GT + 256 + 4 * l)), LOG_FLOOR)));
        if (l == 0) *reinterpret_cast<float*>(smem + L::SC0 + stg * 16) = a;
      }
    };
    issue_loads(N - 1, 0);
    if (N > 1) issue_loads(N - 2, 1);
    wait_next(N > 1);
    decay(0);
    __syncthreads();  // barrier 0
    for (int j = 0; j < N; ++j) {
      const bool dma = j + 2 < N;
      if (dma) issue_loads(N - 3 - j, (j + 2) % RING);
      if (j + 1 < N) wait_next(dma);
      __syncthreads();  // Y
      // step j + 1's decay is first read after X(j): reduced here, off the
      // way to Y (the state waves wait at Y for the last wave to arrive, and
      // this one shares a SIMD with state wave 0)
      if (j + 1 < N) decay((j + 1) % RING);
      __syncthreads();  // X
    }
    return;
  }

  // natural-order row operand of a Q or K tile: lane (m, G) takes row
  // 16 rb + m, columns 32 kb + 8G .. +7 (one 16-byte read); the row tile and
  // stage parts are immediates on a per-(region, kb) base
  lds_cptr rowK[NKB], rowQ[NKB];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    rowK[kb] = opaque_lds(L0 + (L::K0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
    rowQ[kb] = opaque_lds(L0 + (L::Q0 + swz_off<LQ>(lc, 32 * kb + 8 * G)));
  }
  auto row_op = [&](const lds_cptr (&base)[NKB], uint32_t off, int kb) { return lds_ld<bf16x8>(base[kb] + off); };
  // X^T operand of the transposed products (X = K or Q), column tile ct = 2 kb + u:
  // lane (m, G) takes X[s][c] for the pair-order tokens s of block kt and
  // column c = 32 kb + 4u + 8 (m / 4) + m % 4 (two transposing reads)
  auto col_base = [&](int region, int ct) {
    return opaque_lds(L0 + (region + swz_off<LQ>(4 * G + (lc >> 2), 32 * (ct >> 1) + 4 * (ct & 1) + 8 * (lc & 3))));
  };
  auto col_op = [&](lds_cptr base, uint32_t off, int kt) {
    return cat8(lds_tr16(base + off + 32 * kt * ROWB), lds_tr16(base + off + (32 * kt + 16) * ROWB));
  };
  const lds_cptr pbase = L0 + (L::P0 + 16 * l);
  const lds_cptr cbase = L0 + (L::C0 + 16 * l);

  if (w < 2) {
    // ======================================================== state waves
    lds_cptr colK[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) colK[ct] = col_base(L::K0, ct);
    const lds_cptr bp = L0 + (L::G0 + 16 * G);  // beta[16 st + 4G ..]
    f32x4 Sb[NCT];  // lane (r, G): columns 32 (ct / 2) + 8G + 4 (ct % 2) + j of row r
    Op<2> Sp[NKB];  // its pieces, natural order
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) Sb[ct] = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sp[kb] = pack_tiles<2>(Sb[2 * kb], Sb[2 * kb + 1]);
    // Gb_{i-1} = Sb_i of an odd chunk i - 1, this wave's rows, to the
    // staging planes (the token waves store them): 8-byte writes straight
    // from the operand registers.  Unit q = 8 kb + 2G + h of row 16 w + lc.
    lds_ptr gsw[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) gsw[h] = L0 + (L::GS0 + (16 * w + lc) * D * 2 + 8 * ((2 * G + h) ^ (lc & 7)));
    auto stage_gb = [&]() {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        lds_st<bf16x4>(gsw[0] + 64 * kb, __builtin_shufflevector(Sp[kb].v[0], Sp[kb].v[0], 0, 1, 2, 3));
        lds_st<bf16x4>(gsw[1] + 64 * kb, __builtin_shufflevector(Sp[kb].v[0], Sp[kb].v[0], 4, 5, 6, 7));
        lds_st<bf16x4>(gsw[0] + (64 * kb + L::GSP), __builtin_shufflevector(Sp[kb].v[1], Sp[kb].v[1], 0, 1, 2, 3));
        lds_st<bf16x4>(gsw[1] + (64 * kb + L::GSP), __builtin_shufflevector(Sp[kb].v[1], Sp[kb].v[1], 4, 5, 6, 7));
      }
    };
    // the step's K row operands; beta is read one step ahead, during the
    // previous step's update (its chunk has landed by that step's Y)
    f32x4 bt[4];
    bf16x8 Kr[4][NKB];
    auto load_kr = [&](auto stg_tag) {  // in the order X's products take them
      constexpr int STG = decltype(stg_tag)::value;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int st = 0; st < 4; ++st) Kr[st][kb] = row_op(rowK, STG * L::TILE + st * 16 * ROWB, kb);
    };
    auto load_bt = [&](auto stg_tag) {
      constexpr int STG = decltype(stg_tag)::value;
#pragma unroll
      for (int st = 0; st < 4; ++st) bt[st] = lds_ld<f32x4>(bp + (STG * L::GT + st * 64));
    };
    __syncthreads();  // barrier 0
    load_bt(std::integral_constant<int, 0>{});

    auto step = [&](auto stg_tag, int j) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      using NEXT = std::integral_constant<int, (STG + 1) % RING>;
      const int i = N - 1 - j;
      bf16x8 Kc[2][NCT];
      load_kr(stg_tag);
      __builtin_amdgcn_sched_barrier(0);
      // X = K Sb^T (lane (r, G) of tile st: tokens 16 st + 4G + j), with
      // K^T's column operands read between the products
      f32x4 X[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) X[st] = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int st = 0; st < 4; ++st) X[st] = mfma(Kr[st][kb], Sp[kb].v[u], X[st]);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Kc[kt][ct] = col_op(colK[ct], SQK, kt);
      // the decay part of the update (X needs only Sp)
      const float a = lds_ld<float>(L0 + (L::SC0 + STG * 16));
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) Sb[ct] = a * Sb[ct];
#pragma unroll
      for (int k = 0; k < 8 * NKB; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (k < 4 * NCT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      __syncthreads();  // Y: P and C of chunk i published
      // every operand of the update read at once (P first: dE needs it first);
      // the token waves publish -P
      f32x4 Pt[4], Ct[NCT];
      const uint32_t po = (uint32_t)(j & 1) * L::PB;
#pragma unroll
      for (int st = 0; st < 4; ++st) Pt[st] = lds_ld<f32x4>(pbase + (po + (w * 4 + st) * 1024));
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) Ct[ct] = lds_ld<f32x4>(cbase + (w * NCT + ct) * 1024);
      __builtin_amdgcn_sched_barrier(0);
      // -dE = -beta X - P in pieces, pair order: the update's operand
      auto ndt = [&](int st) {
        f32x4 r;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) r[jj] = __builtin_fmaf(-bt[st][jj], X[st][jj], Pt[st][jj]);
        return r;
      };
      Op<2> ND[2];
      ND[0] = pack_tiles<2>(ndt(0), ndt(1));
      __builtin_amdgcn_sched_barrier(0);
      // Sb^T = a Sb^T + C - K^T dE (transposed tiles in the permuted order):
      // token block 0 for every tile with block 1's operand split meanwhile,
      // then block 1 tile pair by tile pair, each pair's C added and split
      // while the next pair is in the MFMA pipe
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) Sb[ct] = mfma(Kc[0][ct], ND[0].v[u], Sb[ct]);
      ND[1] = pack_tiles<2>(ndt(2), ndt(3));
#pragma unroll
      for (int k = 0; k < 2 * NCT; ++k) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      auto finish_pair = [&](int kb) {
        Sb[2 * kb] += Ct[2 * kb];
        Sb[2 * kb + 1] += Ct[2 * kb + 1];
        Sp[kb] = pack_tiles<2>(Sb[2 * kb], Sb[2 * kb + 1]);
        // formed here, not sunk to the next step's products
        asm volatile("" : "+v"(Sp[kb].v[0]), "+v"(Sp[kb].v[1]));
      };
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          Sb[2 * kb] = mfma(Kc[1][2 * kb], ND[1].v[u], Sb[2 * kb]);
          Sb[2 * kb + 1] = mfma(Kc[1][2 * kb + 1], ND[1].v[u], Sb[2 * kb + 1]);
        }
        if (kb > 0) finish_pair(kb - 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        if (kb > 0) __builtin_amdgcn_sched_group_barrier(0x002, 32, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      finish_pair(NKB - 1);
      if (j + 1 < N) load_bt(NEXT{});
      if (i >= 1 && ((i - 1) & 1)) stage_gb();
      __syncthreads();  // X
    };
    for (int j = 0; j < N; j += RING) {
      step(std::integral_constant<int, 0>{}, j);
      if (j + 1 < N) step(std::integral_constant<int, 1>{}, j + 1);
      if (j + 2 < N) step(std::integral_constant<int, 2>{}, j + 2);
    }
    return;
  }

  // =========================================================== token waves
  // key tile ST of waves 2, 3, 6, 7: 0, 1, 3, 2; C column tiles CPW tw .. + CPW - 1
  constexpr int CPW = NCT / 4;
  const int tw = (w & 1) | ((w >> 1) & 2);  // 2 -> 0, 3 -> 1, 6 -> 2, 7 -> 3
  // dO operand of row tile rt, pair-order tokens of block kt (rows
  // 32 kt + 4G + i / 4 and + 16, columns 16 rt + 4 (i % 4))
  lds_cptr obase[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) obase[rt] = opaque_lds(L0 + (L::O0 + swz_off<LO>(4 * G + (lc >> 2), 16 * rt + 4 * (lc & 3))));
  lds_cptr colQ[CPW];
#pragma unroll
  for (int u = 0; u < CPW; ++u) colQ[u] = col_base(L::Q0, CPW * tw + u);
  const lds_ptr pw = L0 + (L::P0 + 16 * l);
  const lds_ptr cw_ = L0 + (L::C0 + 16 * l);
  // Gb stores: 1 KiB of contiguous rows per instruction, D / 32 per wave;
  // instruction k takes the 16-byte unit q of row r, 64 k + l = r UPR + q
  constexpr int UPR = D / 4, KPW = D / 32;
  uint32_t gso[KPW], glo[KPW];
#pragma unroll
  for (int k = 0; k < KPW; ++k) {
    const int f = 64 * (KPW * tw + k) + l, r = f / UPR, q = f % UPR;
    gso[k] = (uint32_t)(r * D + 4 * q);
    glo[k] = (uint32_t)(L::GS0 + r * D * 2 + 8 * (q ^ (r & 7)));
  }
  auto gb_plane = [&](int i) { return p.gb + ((bh * (N / 2) + i / 2) * D + 32 * blk) * (int64_t)D; };
  auto store_gb = [&](int i) {  // Gb_i from the staging rows
    bf16x8 v[KPW];
#pragma unroll
    for (int k = 0; k < KPW; ++k) v[k] = cat8(lds_ld<bf16x4>(L0 + glo[k]), lds_ld<bf16x4>(L0 + (glo[k] + L::GSP)));
    float* gp = gb_plane(i);
#pragma unroll
    for (int k = 0; k < KPW; ++k) *reinterpret_cast<bf16x8*>(gp + gso[k]) = v[k];
  };
  if (N > 0 && ((N - 1) & 1)) {  // Gb_{N-1} = Sb_N = 0
    float* gp = gb_plane(N - 1);
#pragma unroll
    for (int k = 0; k < KPW; ++k) *reinterpret_cast<f32x4*>(gp + gso[k]) = zero4();
  }
  __syncthreads();  // barrier 0

  auto run = [&](auto st_tag) {
    constexpr int ST = decltype(st_tag)::value;
    constexpr int KB0 = ST / 2;  // token blocks with t >= s
    bf16x8 dO8[2][2];  // the step's dO operands, kept from part A to part B
    // part A: P = A^T dO of key tile ST for both row tiles, to P buffer `par`
    auto part_a = [&](auto stg_tag, uint32_t par) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      constexpr uint32_t OC = STG * L::OT;
      bf16x8 Kr[NKB], Qr[4 - ST][NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Kr[kb] = row_op(rowK, SQK + ST * 16 * ROWB, kb);
#pragma unroll
      for (int tt = ST; tt < 4; ++tt)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) Qr[tt - ST][kb] = row_op(rowQ, SQK + tt * 16 * ROWB, kb);
      const float bs = lds_ld<float>(L0 + (L::G0 + STG * L::GT + 4 * (16 * ST + lc)));
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kt = KB0; kt < 2; ++kt)
          dO8[rt][kt] = cat8(lds_tr16(obase[rt] + (OC + 32 * kt * 64)), lds_tr16(obase[rt] + (OC + (32 * kt + 16) * 64)));
      __builtin_amdgcn_sched_barrier(0);
      // A^T operand of key tile ST (m = s, k = t pair order over token block
      // kt) from (Q K^T) D-layout tiles; A[t][s] = 0 for t < s
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
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        f32x4 P = zero4();
#pragma unroll
        for (int kt = KB0; kt < 2; ++kt) P = mma<2, 1>(Aop[kt], Op<1>{{dO8[rt][kt]}}, P);
        lds_st<f32x4>(pw + (par * L::PB + (rt * 4 + ST) * 1024), -P);
      }
      // the token blocks below KB0 (all zero in A) still feed part B's C
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int kt = 0; kt < KB0; ++kt)
          dO8[rt][kt] = cat8(lds_tr16(obase[rt] + (OC + 32 * kt * 64)), lds_tr16(obase[rt] + (OC + (32 * kt + 16) * 64)));
    };
    // part B: C = dO^T Q, column tiles CPW tw + u (transposed, permuted as
    // the state waves' Sb tiles), both row tiles
    auto part_b = [&](auto stg_tag) {
      constexpr int STG = decltype(stg_tag)::value;
      constexpr uint32_t SQK = STG * L::TILE;
      bf16x8 Qc[CPW][2];
#pragma unroll
      for (int u = 0; u < CPW; ++u)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) Qc[u][kt] = col_op(colQ[u], SQK, kt);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int u = 0; u < CPW; ++u) {
          f32x4 Ct = zero4();
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) Ct = mfma(Qc[u][kt], dO8[rt][kt], Ct);
          lds_st<f32x4>(cw_ + (rt * NCT + CPW * tw + u) * 1024, Ct);
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    // step j: part B of step j, Y(j), part A of step j + 1, X(j)
    auto step = [&](auto stg_tag, auto nstg_tag, int j) {
      part_b(stg_tag);
      __syncthreads();  // Y
      if (j + 1 < N) part_a(nstg_tag, (uint32_t)((j + 1) & 1));
      __syncthreads();  // X
      if (N - 2 - j >= 0 && ((N - 2 - j) & 1)) store_gb(N - 2 - j);  // staged before X
    };
    part_a(I0{}, 0u);
    for (int j = 0; j < N; j += RING) {
      step(I0{}, I1{}, j);
      if (j + 1 < N) step(I1{}, I2{}, j + 1);
      if (j + 2 < N) step(I2{}, I0{}, j + 2);
    }
  };
  switch (tw) {
    case 0: run(std::integral_constant<int, 0>{}); break;
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 3>{}); break;
    default: run(std::integral_constant<int, 2>{}); break;
  }
}

template <int D>
static hipError_t launch_dscan(const ChunkArgs& a, hipStream_t stream) {
  auto kern = chunk_bwd_dscan<D>;
  constexpr int lds = DScanLds<D>::BYTES;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  const int64_t grid = a.B * a.H * (D / 32);
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(DSC_THREADS), lds, stream, a);
  return hipGetLastError();
}

hipError_t chunk_bwd_dscan_launch(const ChunkArgs& a, int d, hipStream_t s) {
  return d == 128 ? launch_dscan<128>(a, s) : launch_dscan<64>(a, s);
}

}  // namespace gmdn
