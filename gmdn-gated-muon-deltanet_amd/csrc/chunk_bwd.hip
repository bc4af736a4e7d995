// Level B backward: the fused mixer core's VJP (reference train_ablation.py:142-187
// differentiated through fast_scan.py:72-95 and :134-186).
//
// Per (b, h) and chunk i, with the forward's E-form quantities
//   A = tril(Q K^T) diag(beta),  E = V - K S_i^T,  o = Q S_i^T + A E,
//   G = E^T diag(w) K,  delta: S_{i+1} = a_i S_i + G,
// and Sb_{i+1} = dL/dS_{i+1} (Sb_N = 0), the delta rule's cotangents are
//   Gb  = Sb_{i+1}
//   dE  = A^T dO + diag(w) K Gb^T          (= dV)
//   Sb_i = a_i Sb_{i+1} + dO^T Q - dE^T K
//   dA  = tril(dO E^T)                      (before the beta scaling)
//   dQ  = dO S_i + (dA diag(beta)) K
//   dK  = (dA diag(beta))^T Q - dE S_i + diag(w) E Gb
//   dbeta_s = sum_t dA[t,s] (q_t . k_s) + [delta] (E Gb)[s,:] . k_s
//   dg_t = <Sb_{i+1}, S_i> a_i [g_t >= log 1e-6]
//
// Two kernels per rule:
//  * the reverse recurrence of Sb.  Row r of Sb_i needs only row r of Sb_{i+1}
//    (dE[:, r] = A^T dO[:, r] + diag(w) K Sb[r, :]^T), so one workgroup owns 32
//    rows, with an LDS-DMA ring of Q, K and the workgroup's dO columns, and
//    writes Gb_i: chunk_bwd_dscan (delta, odd chunks only;
//    chunk_bwd_dscan.hip) and chunk_bwd_state (adam, every chunk; 4 waves, wave
//    (rt, h) holds 16 rows x column half h and the moment cotangents in
//    registers).
//  * the token gradients, chunk-parallel.  From S_i (saved by the forward)
//    and Gb_i they recompute E, A and dE and form dQ, dK, dV and the gate
//    gradients; every contraction over the state's rows is local to the
//    workgroup.  chunk_bwd_tok (adam) takes one chunk per workgroup; the
//    delta rule runs the same phases over chunk pairs (chunk_bwd_pair.hip).
//    The kernel's template still carries the delta branches those phases
//    share.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"
#include "scan_a.h"

#include <type_traits>

namespace gmdn {

// ============================================================ chunk_bwd_state
// The adam rule's reverse scan (the delta rule's is chunk_bwd_dscan).
template <int D, int RULE>
struct StateBwdLds {
  static_assert(RULE == 2, "the 4-wave reverse scan serves the adam rule");
  static constexpr bool ADAM = RULE == 2;
  static constexpr int NKBH = D / 64;
  static constexpr int TILE = CB_C * D * 2;   // one Q or K chunk (bytes)
  static constexpr int OT = CB_C * 32 * 2;    // the workgroup's 32 columns of dO (or V)
  static constexpr int GT = 4 * CB_C * 4;     // gate chunk
  static constexpr int Q0 = 0;
  static constexpr int K0 = Q0 + RING * TILE;
  static constexpr int O0 = K0 + RING * TILE;
  static constexpr int V0 = O0 + RING * OT;                        // adam: V columns (E recompute)
  static constexpr int G0 = V0 + (ADAM ? RING * OT : 0);
  static constexpr int XS0 = G0 + RING * GT;                       // Gb^T operand exchange
  static constexpr int XE0 = XS0 + CB_WAVES * NKBH * 2 * 1024;     // -dE operand exchange
  static constexpr int XN0 = XE0 + CB_WAVES * 2 * 1024;            // adam: -E operand exchange
  static constexpr int P0 = XN0 + (ADAM ? CB_WAVES * 2 * 1024 : 0);  // adam: 4 partial sums per wave
  static constexpr int BYTES = P0 + CB_WAVES * 16;
  static_assert(BYTES <= 160 * 1024, "state backward LDS exceeds the 160 KiB of a CU");
  static constexpr int DMA_OPS = 2 * (CB_C * D / 8) / CB_THREADS + (ADAM ? 2 : 1) * (CB_C * 32 / 8) / CB_THREADS;
};

template <int D, int RULE>
__global__ void __launch_bounds__(CB_THREADS) chunk_bwd_state(ChunkArgs p) {
  using LQ = BSwz<D>;
  using LO = BSwz<32>;
  using L = StateBwdLds<D, RULE>;
  constexpr int NKB = D / 32;   // k-blocks over the state's columns
  constexpr int NTH = D / 32;   // column tiles in a half
  constexpr int NKBH = L::NKBH;
  constexpr int ROWB = D * 2;   // bytes per Q/K row
  extern __shared__ __align__(16) char smem[];

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
  const bf16* og = p.o + bb * p.so[0] + hh * p.so[1] + 32 * blk;  // dO columns of the block
  const bf16* vg = p.v + bb * p.sv[0] + hh * p.sv[1] + 32 * blk;  // V columns (adam)
  const float* gsrc = (G == 0 ? p.beta : G == 1 ? p.g : G == 2 ? (RULE == 2 ? p.gmu : p.beta)
                                                               : (RULE == 2 ? p.gnu : p.beta)) +
                      bh * p.T + 4 * lc;

  // per-lane LDS byte offsets (stage, row-tile and k offsets are immediates)
  uint32_t rowoff[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) rowoff[kb][hf] = swz_off<LQ>(lc, 32 * kb + 16 * hf + 4 * G);
  uint32_t coloff[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) coloff[t] = swz_off<LQ>(4 * G + (lc >> 2), 16 * (h * NTH + t) + 4 * (lc & 3));
  // transposing reads of dO (rows 32 kbs + 16 u + 4G + lc/4, columns 16 rt + 4 (lc & 3))
  const uint32_t ooff = swz_off<LO>(4 * G + (lc >> 2), 16 * rt + 4 * (lc & 3));
  const uint32_t lds0 = lds_addr(smem);
  const lds_ptr L0 = lds_base(smem);
  lds_cptr qrow[NKB][2], krow[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      qrow[kb][hf] = L0 + (rowoff[kb][hf] + L::Q0);
      krow[kb][hf] = L0 + (rowoff[kb][hf] + L::K0);
    }
  lds_cptr qcol[NTH], kcol[NTH];
#pragma unroll
  for (int t = 0; t < NTH; ++t) {
    qcol[t] = L0 + (coloff[t] + L::Q0);
    kcol[t] = L0 + (coloff[t] + L::K0);
  }
  const lds_cptr oaddr = L0 + (ooff + L::O0);
  const lds_cptr vaddr = L0 + (ooff + L::V0);
  const lds_ptr xsaddr = L0 + (16 * l + L::XS0);
  const lds_ptr xeaddr = L0 + (16 * l + L::XE0);
  const lds_ptr xnaddr = L0 + (16 * l + L::XN0);
  float* psum = reinterpret_cast<float*>(smem + L::P0);

  DmaPlan<LQ, CB_C, CB_THREADS> dmq, dmk;
  DmaPlan<LO, CB_C, CB_THREADS> dmo, dmv;
  dmq.init(w, p.sq[2]);
  dmk.init(w, p.sk[2]);
  dmo.init(w, p.so[2]);
  if constexpr (RULE == 2) dmv.init(w, p.sv[2]);
  auto issue_loads = [&](int i, int stg) {
    const int64_t t0 = (int64_t)i * CB_C;
    dmq.issue(qg + t0 * p.sq[2], lds0 + L::Q0 + stg * L::TILE, w);
    dmk.issue(kg + t0 * p.sk[2], lds0 + L::K0 + stg * L::TILE, w);
    dmo.issue(og + t0 * p.so[2], lds0 + L::O0 + stg * L::OT, w);
    if constexpr (RULE == 2) dmv.issue(vg + t0 * p.sv[2], lds0 + L::V0 + stg * L::OT, w);
    if (w == 0) lds_dma16(gsrc + t0, smem + L::G0 + stg * L::GT);
  };

  f32x4 Sb[NTH];   // dL/dS_{i+1}, this lane's row, the wave's column half
  f32x4 Mb[NTH], Vb[NTH];  // adam: dL/dM_{i+1}, dL/dV_{i+1}
#pragma unroll
  for (int t = 0; t < NTH; ++t) Sb[t] = Mb[t] = Vb[t] = zero4();
  // adam: chunk i's S_i row (pair-order pieces of all columns) and M_i, V_i
  // (the wave's column half), loaded one chunk ahead
  f32x4 Sraw[NKB][2], Mp[NTH], Vp[NTH];
  auto load_states = [&](int i) {
    const int64_t plane = p.B * p.H * p.N * (int64_t)D * D;
    const float* sp = p.states + ((bh * p.N + i) * D + r0 + lc) * (int64_t)D;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      Sraw[kb][0] = unsplit_piece(*reinterpret_cast<const bf16x8*>(sp + 32 * kb + 4 * G));
      Sraw[kb][1] = unsplit_piece(*reinterpret_cast<const bf16x8*>(sp + 32 * kb + 16 + 4 * G));
    }
#pragma unroll
    for (int t = 0; t < NTH; ++t) {
      Mp[t] = *reinterpret_cast<const f32x4*>(sp + plane + 16 * (h * NTH + t) + 4 * G);
      Vp[t] = *reinterpret_cast<const f32x4*>(sp + 2 * plane + 16 * (h * NTH + t) + 4 * G);
    }
  };
  auto xn_addr = [&](int ww) { return xnaddr + (ww * 2) * 1024; };
  auto xs_addr = [&](int ww, int k) { return xsaddr + ((ww * NKBH + k) * 2) * 1024; };
  auto xe_addr = [&](int ww) { return xeaddr + (ww * 2) * 1024; };
  auto publish_Gb = [&](const f32x4 (&X)[NTH]) {
#pragma unroll
    for (int kbl = 0; kbl < NKBH; ++kbl) {
      const Op<2> x = pack_tiles<2>(X[2 * kbl], X[2 * kbl + 1]);
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

  // chunks are visited in reverse: step j handles chunk N-1-j, ring stage j % RING
  for (int j = 0; j < RING - 1 && j < p.N; ++j) issue_loads(p.N - 1 - j, j);
  if (p.N > 0) load_states(p.N - 1);
  wait_vmem();
  __syncthreads();
  if (p.N > 0) chunk_scalars(0);

  auto chunk = [&](auto stg_tag, int j) {
    constexpr int STG = decltype(stg_tag)::value;
    constexpr uint32_t SQK = STG * L::TILE;
    constexpr uint32_t OC = STG * L::OT;
    const float* gates = reinterpret_cast<const float*>(smem + L::G0 + STG * L::GT);
    const int i = p.N - 1 - j;
    const bool ahead = j + RING - 1 < p.N;
    if (ahead) issue_loads(p.N - 1 - (j + RING - 1), (STG + RING - 1) % RING);
    float* gp = p.gb + ((bh * p.N + i) * D + r0 + lc) * (int64_t)D + 4 * G;
    auto rows = [&](const lds_cptr (&base)[NKB][2], int rowtile, int kb) {
      return cat8(lds_ld<bf16x4>(base[kb][0] + SQK + rowtile * 16 * ROWB),
                  lds_ld<bf16x4>(base[kb][1] + SQK + rowtile * 16 * ROWB));
    };
    // dO operand (k = tokens 32 kbs + pair order, n = this lane's state row)
    auto dop = [&](int kbs) {
      return cat8(lds_tr16(oaddr + (OC + (32 * kbs) * 64)), lds_tr16(oaddr + (OC + (32 * kbs + 16) * 64)));
    };
    using std::integral_constant;
    using I0 = integral_constant<int, 0>;
    using I1 = integral_constant<int, 1>;
    if constexpr (RULE == 2) {
      // ---------------- adam A: -E = K S_i^T - V for this wave's tokens (reference
      // fast_scan.py:89-94 recomputed: G_i is needed by the moment VJP)
      auto segA = [&](auto rt_tag, auto h_tag) {
        constexpr int RT = decltype(rt_tag)::value, H = decltype(h_tag)::value;
        constexpr uint32_t VC = STG * L::OT;
        Op<2> Sop[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) Sop[kb] = pack_tiles<2>(Sraw[kb][0], Sraw[kb][1]);
        f32x4 Nt[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const bf16x4 vb = lds_tr16(vaddr + (VC + (32 * H + 16 * u) * 64));
          Nt[u] = f32x4{-(float)vb[0], -(float)vb[1], -(float)vb[2], -(float)vb[3]};
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) Nt[u] = mma<1, 2>(Op<1>{{rows(krow, 2 * H + u, kb)}}, Sop[kb], Nt[u]);
        }
        const Op<2> en = pack_tiles<2>(Nt[0], Nt[1]);
        lds_st<bf16x8>(xn_addr(2 * RT + H), en.v[0]);
        lds_st<bf16x8>(xn_addr(2 * RT + H) + 1024, en.v[1]);
      };
      switch (w) {
        case 0: segA(I0{}, I0{}); break;
        case 1: segA(I0{}, I1{}); break;
        case 2: segA(I1{}, I0{}); break;
        default: segA(I1{}, I1{}); break;
      }
      __syncthreads();  // -E halves published
      // ---------------- adam B: G_i, the moment VJP (reference fast_scan.py:167-182)
      {
        Op<2> EN[2];
#pragma unroll
        for (int hs = 0; hs < 2; ++hs) EN[hs] = read_op(xn_addr(2 * rt + hs));
        f32x4 Gb[NTH];
        float da = 0.f, db = 0.f, dm = 0.f, dn = 0.f;
#pragma unroll
        for (int t = 0; t < NTH; ++t) {
          f32x4 acc = zero4();
#pragma unroll
          for (int kbs = 0; kbs < 2; ++kbs) {
            const uint32_t ro = SQK + kbs * 32 * ROWB;
            const bf16x8 kc = cat8(lds_tr16(kcol[t] + ro), lds_tr16(kcol[t] + ro + 16 * ROWB));
            acc = mma<1, 2>(Op<1>{{kc}}, EN[kbs], acc);
          }
          const int ct = h * NTH + t;  // column tile of S_i held in Sraw
          const f32x4 Si = Sraw[ct >> 1][ct & 1];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float g = -acc[jj];
            const float mn = msc * Mp[t][jj] + (1.f - msc) * g;
            const float vn = nsc * Vp[t][jj] + (1.f - nsc) * g * g;
            const float sq = hw_sqrt(vn);
            const float rden = hw_rcp(sq + p.eps);
            const float sb = Sb[t][jj];
            da += sb * Si[jj];
            db += sb * mn * rden;
            const float mt = Mb[t][jj] + bsc * sb * rden;
            const float vt = Vb[t][jj] - bsc * sb * mn * rden * rden * hw_rcp(2.f * fmaxf(sq, 1e-12f));
            dm += mt * (Mp[t][jj] - g);
            dn += vt * (Vp[t][jj] - g * g);
            Gb[t][jj] = (1.f - msc) * mt + (1.f - nsc) * 2.f * g * vt;
            Mb[t][jj] = msc * mt;
            Vb[t][jj] = nsc * vt;
          }
          *reinterpret_cast<bf16x8*>(gp + 16 * (h * NTH + t)) = split_piece(Gb[t]);
        }
        publish_Gb(Gb);
        da = wave_sum(da);
        db = wave_sum(db);
        dm = wave_sum(dm);
        dn = wave_sum(dn);
        if (l == 0) {  // the wave's own slots, summed below in a fixed order
          psum[4 * w + 0] = da;
          psum[4 * w + 1] = db;
          psum[4 * w + 2] = dm;
          psum[4 * w + 3] = dn;
        }
      }
      __syncthreads();  // Gb halves and the partial sums published
      if (w == 0 && l < 4) {
        static_assert(CB_WAVES == 4, "four partial slots per scalar");
        p.part[((bh * p.N + i) * (D / 32) + blk) * 4 + l] = (psum[l] + psum[4 + l]) + (psum[8 + l] + psum[12 + l]);
      }
    }
    // ---------------- segment 1: dE for this wave's tokens 32H .. 32H+31
    auto segment1 = [&](auto rt_tag, auto h_tag) {
      constexpr int RT = decltype(rt_tag)::value, H = decltype(h_tag)::value;
      Op<2> Sop[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Sop[kb] = read_op(xs_addr(2 * RT + kb / NKBH, kb % NKBH));
      f32x4 dE[2] = {zero4(), zero4()};
      {  // diag(w) K Gb^T
        bf16x8 Kr[2][NKB];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) Kr[u][kb] = rows(krow, 2 * H + u, kb);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int u = 0; u < 2; ++u) dE[u] = mma<1, 2>(Op<1>{{Kr[u][kb]}}, Sop[kb], dE[u]);
      }
      __builtin_amdgcn_sched_barrier(0);
      // + A^T dO over the token blocks kbs >= H (A[t][s] = 0 for t < s).  The
      // A^T operand (m = s, k = t) is the D-layout of (Q K^T) tiles.
#pragma unroll
      for (int kbs = H; kbs < 2; ++kbs) {
        const bf16x8 dO8 = dop(kbs);
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int st = 2 * H + u;
          const float bs = gates[16 * st + lc];
          f32x4 X[2];
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int tt = 2 * kbs + hf;
            X[hf] = zero4();
            if (tt >= st) {
#pragma unroll
              for (int kb = 0; kb < NKB; ++kb) X[hf] = mfma(rows(qrow, tt, kb), rows(krow, st, kb), X[hf]);
#pragma unroll
              for (int jj = 0; jj < 4; ++jj)
                X[hf][jj] = (tt > st || 4 * G + jj >= lc) ? X[hf][jj] * bs : 0.f;
            }
          }
          dE[u] = mma<2, 1>(pack_tiles<2>(X[0], X[1]), Op<1>{{dO8}}, dE[u]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      const Op<2> nd = pack_tiles<2>(-dE[0], -dE[1]);
      lds_st<bf16x8>(xe_addr(2 * RT + H), nd.v[0]);
      lds_st<bf16x8>(xe_addr(2 * RT + H) + 1024, nd.v[1]);
    };
    switch (w) {
      case 0: segment1(I0{}, I0{}); break;
      case 1: segment1(I0{}, I1{}); break;
      case 2: segment1(I1{}, I0{}); break;
      default: segment1(I1{}, I1{}); break;
    }
    __syncthreads();  // -dE halves published
    // ---------------- segment 2: Sb_i = a Sb_{i+1} + dO^T Q - dE^T K (column half h)
    {
      Op<2> ND[2];
#pragma unroll
      for (int hs = 0; hs < 2; ++hs) ND[hs] = read_op(xe_addr(2 * rt + hs));
      f32x4 acc[NTH];
#pragma unroll
      for (int t = 0; t < NTH; ++t) acc[t] = a * Sb[t];
#pragma unroll
      for (int kbs = 0; kbs < 2; ++kbs) {
        const bf16x8 dO8 = dop(kbs);
#pragma unroll
        for (int t = 0; t < NTH; ++t) {
          const uint32_t ro = SQK + kbs * 32 * ROWB;
          const bf16x8 qc = cat8(lds_tr16(qcol[t] + ro), lds_tr16(qcol[t] + ro + 16 * ROWB));
          const bf16x8 kc = cat8(lds_tr16(kcol[t] + ro), lds_tr16(kcol[t] + ro + 16 * ROWB));
          acc[t] = mfma(qc, dO8, acc[t]);
          acc[t] = mma<1, 2>(Op<1>{{kc}}, ND[kbs], acc[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < NTH; ++t) Sb[t] = acc[t];
    }
    __builtin_amdgcn_sched_barrier(0);
    if (i > 0) load_states(i - 1);
    __builtin_amdgcn_sched_barrier(0);
    if (ahead) {
      if (w == 0)
        wait_vmem_le<L::DMA_OPS + 1>();
      else
        wait_vmem_le<L::DMA_OPS>();
    } else {
      wait_vmem();
    }
    __syncthreads();  // next chunk's tiles landed, (delta) Sb_i halves published
    if (j + 1 < p.N) chunk_scalars((STG + 1) % RING);
  };

  for (int j = 0; j < p.N; j += RING) {
    chunk(std::integral_constant<int, 0>{}, j);
    if (j + 1 < p.N) chunk(std::integral_constant<int, 1>{}, j + 1);
    if (j + 2 < p.N) chunk(std::integral_constant<int, 2>{}, j + 2);
  }
}

// ============================================================== chunk_bwd_tok
// One wave per 16 state rows (phase I) and per 16 state columns (phase IIb):
// D / 16 waves, two per SIMD at d = 128, so one wave's global loads overlap
// another's MFMA work (the workgroup's LDS allows one workgroup per CU).
template <int D>
struct TokBwdLds {
  static constexpr int NW = D / 16;
  static constexpr int NTHR = 64 * NW;
  static constexpr int TILE = CB_C * D * 2;
  static constexpr int Q0 = 0, K0 = TILE, V0 = 2 * TILE, O0 = 3 * TILE;
  static constexpr int EH0 = 4 * TILE, EL0 = 5 * TILE;    // E (rows s, columns r), hi / lo
  static constexpr int DH0 = 6 * TILE, DL0 = 7 * TILE;    // dE
  static constexpr int AP = CB_C * CB_C * 2;
  static constexpr int AH0 = 8 * TILE, AL0 = AH0 + AP;    // dA diag(beta), transposed (rows s)
  // floats: per-wave dbeta and (muon) dw partials [NW][64] each, beta, g,
  // gmu, gnu (muon: w), per-wave da partials [NW]
  static constexpr int R0 = AL0 + AP;
  static constexpr int BYTES = R0 + (2 * NW * CB_C + 4 * CB_C + NW) * 4;
  static_assert(BYTES <= 160 * 1024, "token backward LDS exceeds the 160 KiB of a CU");
};

// MAT: S_i and Gb_i are the drop-in scan's float32 rows and the chunk
// scalars' gradients arrive as arrays [da | db | dm | dn] (B H N each) in
// p.part -- muon always, adam when its scan ran in exact float32 (d = 128)
template <int D, int RULE, bool MAT = RULE == 1>
__global__ void __launch_bounds__(TokBwdLds<D>::NTHR) chunk_bwd_tok(ChunkArgs p) {
  using LQ = BSwz<D>;
  using LA = BSwz<CB_C>;
  using L = TokBwdLds<D>;
  constexpr int NKB = D / 32;
  constexpr int NW = L::NW;
  constexpr int NTHR = L::NTHR;
  extern __shared__ __align__(16) char smem[];
  const bf16* Qs = reinterpret_cast<const bf16*>(smem + L::Q0);
  const bf16* Ks = reinterpret_cast<const bf16*>(smem + L::K0);
  const bf16* Vs = reinterpret_cast<const bf16*>(smem + L::V0);
  const bf16* Os = reinterpret_cast<const bf16*>(smem + L::O0);
  bf16* Eh = reinterpret_cast<bf16*>(smem + L::EH0);
  bf16* El = reinterpret_cast<bf16*>(smem + L::EL0);
  bf16* Dh = reinterpret_cast<bf16*>(smem + L::DH0);
  bf16* Dl = reinterpret_cast<bf16*>(smem + L::DL0);
  bf16* Ah = reinterpret_cast<bf16*>(smem + L::AH0);
  bf16* Al = reinterpret_cast<bf16*>(smem + L::AL0);
  // dbeta and da are summed per wave into the wave's own slots, then over
  // the waves in a fixed order: the gradients are bitwise reproducible
  float* red = reinterpret_cast<float*>(smem + L::R0);
  float* pdbeta = red;               // [NW][64]
  float* pdw = red + NW * CB_C;      // [NW][64] (muon: dL/dw_t)
  float* rbeta = red + 2 * NW * CB_C;  // [64]
  float* rg = rbeta + CB_C;          // [64]
  float* rgmu = rbeta + 2 * CB_C;    // [64] (muon, adam)
  float* rgnu = rbeta + 3 * CB_C;    // [64] (adam; muon: the token weights w)
  float* pda = rbeta + 4 * CB_C;     // [NW]
  // muon reads S_i and Gb_i as float32 rows (the drop-in scan's layout), the
  // others as split pieces: the conversion waits until the rows are used
  auto piece = [](const bf16x8& x) {
    if constexpr (MAT)
      return split_piece(__builtin_bit_cast(f32x4, x));
    else
      return x;
  };

  const int64_t bh = blockIdx.x / p.N;
  const int i = (int)(blockIdx.x % p.N);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int64_t bb = bh / p.H, hh = bh % p.H;
  const int64_t t0 = (int64_t)i * CB_C;
  const float* S = p.states + (bh * p.N + i) * (int64_t)D * D;
  const float* Gb = p.gb + (bh * p.N + i) * (int64_t)D * D;
  const int r0 = 16 * w;  // this wave's state rows (phase I) ...
  const int j0 = 16 * w;  // ... and state columns (phase IIb)

  // ---------------- phase 0: gates, then the q, k tiles (all phase I' needs),
  // the v, dO tiles and the rows r0 + lc of S_i and Gb_i (natural k order),
  // which arrive while phase I' runs
  float gv[4];
  if (threadIdx.x < CB_C) {
    const int64_t e = bh * p.T + t0 + threadIdx.x;
    gv[0] = p.beta[e];
    gv[1] = p.g[e];
    if constexpr (RULE >= 1) gv[2] = p.gmu[e];
    if constexpr (RULE == 2) gv[3] = p.gnu[e];
  }
  {
    DmaPlan<LQ, CB_C, NTHR> pq, pk, pv, po;
    pq.init(w, p.sq[2]);
    pk.init(w, p.sk[2]);
    pv.init(w, p.sv[2]);
    po.init(w, p.so[2]);
    const uint32_t lds0 = lds_addr(smem);
    pq.issue(p.q + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2], lds0 + L::Q0, w);
    pk.issue(p.k + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2], lds0 + L::K0, w);
    pv.issue(p.v + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2], lds0 + L::V0, w);
    po.issue(p.o + bb * p.so[0] + hh * p.so[1] + t0 * p.so[2], lds0 + L::O0, w);
  }
  bf16x8 srow[NKB][2], grow[NKB][2];  // split pieces of columns 32 kb + 8G .. +3, +4 .. +7
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    const int64_t off = (int64_t)(r0 + lc) * D + 32 * kb + 8 * G;
    srow[kb][0] = *reinterpret_cast<const bf16x8*>(S + off);
    srow[kb][1] = *reinterpret_cast<const bf16x8*>(S + off + 4);
    grow[kb][0] = *reinterpret_cast<const bf16x8*>(Gb + off);
    grow[kb][1] = *reinterpret_cast<const bf16x8*>(Gb + off + 4);
  }
  // vector-memory operations complete in issue order: with the 4 NKB row
  // loads still in flight, the gates and the four tiles have landed
  wait_vmem_le<4 * NKB>();
  if (threadIdx.x < CB_C) {
    const int e = threadIdx.x;
    rbeta[e] = gv[0];
    rg[e] = gv[1];
    if constexpr (RULE >= 1) rgmu[e] = gv[2];
    if constexpr (RULE == 2) rgnu[e] = gv[3];
    if constexpr (RULE == 1) {
      // w_t = exp(sum_{s > t} max(gmu_s, log 1e-6)) (train_ablation.py:154-156)
      const float lm = fmaxf(gv[2], LOG_FLOOR);
      const float msum = wave_sum(lm);
      float incl = lm;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(incl, o, 64);
        if (e >= o) incl += y;
      }
      rgnu[e] = expf(msum - incl);
    }
  }
  __syncthreads();

  // ---------------- phase I': A^T = (tril(Q K^T) diag(beta))^T, split, into the
  // dA planes (free until phase IIa): tile (tt, st), k = 4 tt + st, goes to
  // wave k % NW; tiles above the diagonal are written as zeros
#pragma unroll
  for (int kk = 0; kk < 16 / NW; ++kk) {
    const int k = w + NW * kk, tt = k >> 2, st = k & 3;
    bf16x4 ah, al;
    if (tt < st) {
      ah = al = bf16x4{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
    } else {
      f32x4 X = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        X = mfma(row8<LQ>(Qs, 16 * tt + lc, 32 * kb), row8<LQ>(Ks, 16 * st + lc, 32 * kb), X);
      // lane (s, G) holds A[t = 16 tt + 4G + jj][s = 16 st + lc]
      const float bs = rbeta[16 * st + lc];
      f32x4 xv;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) xv[jj] = (tt > st || 4 * G + jj >= lc) ? X[jj] * bs : 0.f;
      split4(xv, ah, al);
    }
    const int ao = LA::off(16 * st + lc, 16 * tt + 4 * G);
    *reinterpret_cast<bf16x4*>(Ah + ao) = ah;
    *reinterpret_cast<bf16x4*>(Al + ao) = al;
  }
  __syncthreads();  // the A planes published (the state rows may still be arriving)

  // ---------------- phase I: E^T, (Gb K^T) and dE^T for this wave's 16 state rows
  Op<2> Sa[NKB], Ga[NKB];  // rows r0 + lc of S_i, Gb_i (m = r, k = c natural); reused in IIb
  {
    float ws[4], dbp[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) ws[st] = RULE == 0 ? rbeta[16 * st + lc] : RULE == 1 ? rgnu[16 * st + lc] : 1.f;
    // column block by column block: the MFMA chains of block kb start as soon
    // as its rows have landed (the loads complete in issue order)
    f32x4 Ets[4], GKs[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      // D layout: lane (s, G) holds rows r0 + 4G + jj
      const bf16x4 vv = *reinterpret_cast<const bf16x4*>(Vs + LQ::off(16 * st + lc, r0 + 4 * G));
      Ets[st] = f32x4{-(float)vv[0], -(float)vv[1], -(float)vv[2], -(float)vv[3]};
      GKs[st] = zero4();
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      Sa[kb] = join_pieces(piece(srow[kb][0]), piece(srow[kb][1]));
      Ga[kb] = join_pieces(piece(grow[kb][0]), piece(grow[kb][1]));
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const Op<1> kr{{row8<LQ>(Ks, 16 * st + lc, 32 * kb)}};
        Ets[st] = mma<2, 1>(Sa[kb], kr, Ets[st]);
        GKs[st] = mma<2, 1>(Ga[kb], kr, GKs[st]);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep each block's wait after the previous block's MFMAs
    }
    // the loop below has no cross-lane step, so the LDS reads of one token
    // tile overlap the MFMA chains of the previous one
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const f32x4 Et = -Ets[st];  // E^T = V^T - S K^T
      const f32x4 GK = GKs[st];
      dbp[st] = dot4(Et, GK);  // dbeta's diag(w) term, this lane's 4 rows
      f32x4 dEt = GK * ws[st];
#pragma unroll
      for (int kbt = 0; kbt < 2; ++kbt) {
        if (32 * kbt + 31 < 16 * st) continue;
        const Op<1> dOt{{col8<LQ>(Os, 32 * kbt, r0)}};  // dO^T (m = r, k = t)
        const Op<2> At{{row8<LA>(Ah, 16 * st + lc, 32 * kbt), row8<LA>(Al, 16 * st + lc, 32 * kbt)}};
        dEt = mma<1, 2>(dOt, At, dEt);  // (k = t, n = s)
      }
      bf16x4 eh, el, dh, dl;
      split4(Et, eh, el);
      split4(dEt, dh, dl);
      const int eo = LQ::off(16 * st + lc, r0 + 4 * G);
      *reinterpret_cast<bf16x4*>(Eh + eo) = eh;
      *reinterpret_cast<bf16x4*>(El + eo) = el;
      *reinterpret_cast<bf16x4*>(Dh + eo) = dh;
      *reinterpret_cast<bf16x4*>(Dl + eo) = dl;
    }
    if constexpr (RULE == 0) {
      // dbeta's diag(w) term: sum_r E[s][r] (Gb k_s)[r] over the wave's rows
#pragma unroll
      for (int st = 0; st < 4; ++st) dbp[st] = group_sum(dbp[st]);
      if (G == 0) {
#pragma unroll
        for (int st = 0; st < 4; ++st) pdbeta[w * CB_C + 16 * st + lc] = dbp[st];
      }
      // delta: Gb_i = Sb_{i+1}, so da_i = <Gb_i, S_i>: the trace of this
      // wave's 16 x 16 diagonal block of Gb_i S_i^T (A = Gb rows, B = S rows)
      f32x4 T = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) T = mma<2, 2>(Ga[kb], Sa[kb], T);
      // lane (n, G) holds entries (4G + jj, n): the diagonal is jj = n - 4G
      const float dpart = (lc >> 2) == G ? T[lc & 3] : 0.f;
      const float da_w = wave_sum(dpart);
      if (l == 0) pda[w] = da_w;
    } else {
      if constexpr (RULE == 1) {
        // muon: sum_r E[s][r] (Gb k_s)[r] is dL/dw_s (w depends on gmu only)
#pragma unroll
        for (int st = 0; st < 4; ++st) dbp[st] = group_sum(dbp[st]);
        if (G == 0) {
#pragma unroll
          for (int st = 0; st < 4; ++st) pdw[w * CB_C + 16 * st + lc] = dbp[st];
        }
      }
      if (G == 0) {
#pragma unroll
        for (int st = 0; st < 4; ++st) pdbeta[w * CB_C + 16 * st + lc] = 0.f;
      }
    }
  }
  __syncthreads();

  // ---------------- phase IIa: dA = tril(dO E^T), dbeta's A term, dA diag(beta) -> LDS
  // tiles k = 4 tt + st, k = w, w + NW, ...; tiles above the diagonal are zeroed
  float dbk[16 / NW];
#pragma unroll
  for (int kk = 0; kk < 16 / NW; ++kk) {
    dbk[kk] = 0.f;
    const int k = w + NW * kk, tt = k >> 2, st = k & 3;
    bf16x4 ah, al;
    if (tt < st) {
      ah = al = bf16x4{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
    } else {
      f32x4 P = zero4(), QK = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const Op<1> dOr{{row8<LQ>(Os, 16 * tt + lc, 32 * kb)}};
        const Op<2> Er{{row8<LQ>(Eh, 16 * st + lc, 32 * kb), row8<LQ>(El, 16 * st + lc, 32 * kb)}};
        P = mma<1, 2>(dOr, Er, P);
        QK = mfma(row8<LQ>(Qs, 16 * tt + lc, 32 * kb), row8<LQ>(Ks, 16 * st + lc, 32 * kb), QK);
      }
      const float bs = rbeta[16 * st + lc];
      float db = 0.f;
      f32x4 pb;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float pv = (tt > st || 4 * G + jj >= lc) ? P[jj] : 0.f;
        db += pv * QK[jj];
        pb[jj] = pv * bs;
      }
      split4(pb, ah, al);
      dbk[kk] = db;
    }
    const int ao = LA::off(16 * st + lc, 16 * tt + 4 * G);
    *reinterpret_cast<bf16x4*>(Ah + ao) = ah;
    *reinterpret_cast<bf16x4*>(Al + ao) = al;
  }
  {
    // the wave's tiles k = w + NW kk all have st = w % 4
    static_assert(NW % 4 == 0, "a wave's phase IIa tiles share one token tile");
    float db = 0.f;
#pragma unroll
    for (int kk = 0; kk < 16 / NW; ++kk) {
      const int k = w + NW * kk, tt = k >> 2, st = k & 3;
      const float v = group_sum(dbk[kk]);
      if (tt >= st) db += v;
    }
    if (G == 0) pdbeta[w * CB_C + 16 * (w & 3) + lc] += db;
  }
  __syncthreads();

  // ---------------- gate gradients and dV
  if (w == 0) {
    const int64_t o = bh * p.T + t0 + l;
    const float a = expf(wave_sum(fmaxf(rg[l], LOG_FLOOR)));
    float rdb = 0.f;
#pragma unroll
    for (int q = 0; q < NW; ++q) rdb += pdbeta[q * CB_C + l];
    if constexpr (RULE == 0) {
      float da = 0.f;
#pragma unroll
      for (int q = 0; q < NW; ++q) da += pda[q];
      p.dbeta[o] = rdb;
      p.dg[o] = rg[l] >= LOG_FLOOR ? da * a : 0.f;
    } else if constexpr (RULE == 1) {
      // da, db, dm from the drop-in scan's backward: part = [da | db | dm] (B H N each)
      const int64_t BHN = p.B * p.H * p.N, si = bh * p.N + i;
      const float da = p.part[si], db = p.part[BHN + si], dm = p.part[2 * BHN + si];
      const float m = expf(wave_sum(fmaxf(rgmu[l], LOG_FLOOR)));
      float dw = 0.f;
#pragma unroll
      for (int q = 0; q < NW; ++q) dw += pdw[q * CB_C + l];
      // d/dlm_t: m (all t) and w_s for s < t (w_s = exp(sum_{u > s} lm_u))
      const float x = dw * rgnu[l];
      float incl = x;
#pragma unroll
      for (int q = 1; q < 64; q <<= 1) {
        const float y = __shfl_up(incl, q, 64);
        if (l >= q) incl += y;
      }
      p.dbeta[o] = rdb + db * (1.f / CB_C);  // b = mean(beta)
      p.dg[o] = rg[l] >= LOG_FLOOR ? da * a : 0.f;
      p.dgmu[o] = rgmu[l] >= LOG_FLOOR ? (incl - x) + dm * m : 0.f;
    } else {
      // da, db, dm, dn: sums of the reverse scan's per-row-block partials,
      // or (MAT) the drop-in scan's per-chunk gradients
      float sc[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (MAT) {
        const int64_t BHN = p.B * p.H * p.N, si = bh * p.N + i;
#pragma unroll
        for (int c = 0; c < 4; ++c) sc[c] = p.part[c * BHN + si];
      } else {
        const float* pp = p.part + (bh * p.N + i) * (int64_t)(D / 32) * 4;
#pragma unroll
        for (int r = 0; r < D / 32; ++r)
#pragma unroll
          for (int c = 0; c < 4; ++c) sc[c] += pp[4 * r + c];
      }
      const float m = expf(wave_sum(fmaxf(rgmu[l], LOG_FLOOR)));
      const float n = expf(wave_sum(fmaxf(rgnu[l], LOG_FLOOR)));
      p.dbeta[o] = rdb + sc[1] * (1.f / CB_C);  // b = mean(beta)
      p.dg[o] = rg[l] >= LOG_FLOOR ? sc[0] * a : 0.f;
      p.dgmu[o] = rgmu[l] >= LOG_FLOOR ? sc[2] * m : 0.f;
      p.dgnu[o] = rgnu[l] >= LOG_FLOOR ? sc[3] * n : 0.f;
    }
  }
  {
    bf16* dvg = p.dv + bb * p.sv[0] + hh * p.sv[1] + t0 * p.sv[2];
    for (int e = threadIdx.x; e < CB_C * D / 8; e += NTHR) {
      const int r = e / (D / 8), c8 = (e % (D / 8)) * 8;
      *reinterpret_cast<bf16x8*>(dvg + r * p.sv[2] + c8) = *reinterpret_cast<const bf16x8*>(Dh + LQ::off(r, c8));
    }
  }

  // ---------------- phase IIb: dQ and dK for this wave's 16 state columns
  //   dQ = (dA diag(beta)) K + dO S,   dK = (dA diag(beta))^T Q - dE S + diag(w) E Gb
  // Every product has its operands swapped, so the tiles are the transposes
  // (lane <-> token, registers <-> 4 consecutive state columns) and each
  // leaves in one 8-byte store.
  bf16* dqg = p.dq + bb * p.sq[0] + hh * p.sq[1] + t0 * p.sq[2];
  bf16* dkg = p.dk + bb * p.sk[0] + hh * p.sk[1] + t0 * p.sk[2];
  f32x4 dqa[4], dka[4], des[4], eg[4];
  // the dA terms first: they are the last readers of the Q and K tiles
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    dqa[tt] = zero4();
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (32 * ks > 16 * tt + 15) continue;
      const Op<2> dA{{col8<LA>(Ah, 32 * ks, 16 * tt), col8<LA>(Al, 32 * ks, 16 * tt)}};
      dqa[tt] = mma<1, 2>(Op<1>{{col8<LQ>(Ks, 32 * ks, j0)}}, dA, dqa[tt]);
    }
  }
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    dka[st] = des[st] = eg[st] = zero4();
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      if (32 * kt + 31 < 16 * st) continue;
      const Op<2> dAT{{row8<LA>(Ah, 16 * st + lc, 32 * kt), row8<LA>(Al, 16 * st + lc, 32 * kt)}};
      dka[st] = mma<1, 2>(Op<1>{{col8<LQ>(Qs, 32 * kt, j0)}}, dAT, dka[st]);
    }
  }
  // The products over the state's rows need S_i and Gb_i by columns.  They
  // are transposed on chip: the rows still held from phase I pass through
  // the (now free) Q and K tiles one 32-row block at a time, split planes
  // of [32 rows][D], and every wave reads its 16 columns back transposed.
  bf16* Sh = reinterpret_cast<bf16*>(smem + L::Q0);
  bf16* Sl = Sh + 32 * D;
  bf16* Gh = reinterpret_cast<bf16*>(smem + L::K0);
  bf16* Gl = Gh + 32 * D;
  __syncthreads();  // Q and K tiles free
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    if ((w >> 1) == kb) {  // waves 2kb, 2kb+1 hold rows 32 kb .. 32 kb + 31
      const int lr = 16 * (w & 1) + lc;
#pragma unroll
      for (int kc = 0; kc < NKB; ++kc) {
        const int so = LQ::off(lr, 32 * kc + 8 * G);
        *reinterpret_cast<bf16x8*>(Sh + so) = Sa[kc].v[0];
        *reinterpret_cast<bf16x8*>(Sl + so) = Sa[kc].v[1];
        *reinterpret_cast<bf16x8*>(Gh + so) = Ga[kc].v[0];
        *reinterpret_cast<bf16x8*>(Gl + so) = Ga[kc].v[1];
      }
    }
    __syncthreads();
    // columns j0 + lc, rows 32 kb + (k = 8G .. 8G + 7): (k = r natural, n = j)
    const Op<2> sc{{col8<LQ>(Sh, 0, j0), col8<LQ>(Sl, 0, j0)}};
    const Op<2> gc{{col8<LQ>(Gh, 0, j0), col8<LQ>(Gl, 0, j0)}};
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) dqa[tt] = mma<2, 1>(sc, Op<1>{{row8<LQ>(Os, 16 * tt + lc, 32 * kb)}}, dqa[tt]);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const Op<2> Er{{row8<LQ>(Eh, 16 * st + lc, 32 * kb), row8<LQ>(El, 16 * st + lc, 32 * kb)}};
      const Op<2> Dr{{row8<LQ>(Dh, 16 * st + lc, 32 * kb), row8<LQ>(Dl, 16 * st + lc, 32 * kb)}};
      eg[st] = mma<2, 2>(gc, Er, eg[st]);
      des[st] = mma<2, 2>(sc, Dr, des[st]);
    }
    if (kb + 1 < NKB) __syncthreads();  // before the next block overwrites the staging planes
  }
  // dQ and dK: staged as [64 tokens][D] bf16 tiles in the V tile and the dA
  // planes (both free since phase I / the dA terms), then stored in rows
  bf16* dqs = reinterpret_cast<bf16*>(smem + L::V0);
  bf16* dks = Ah;
  static_assert(2 * L::AP >= L::TILE, "the dA planes hold one [64][D] bf16 tile");
  // lane (t, G) of transposed tile tt holds dQ[16 tt + t][j0 + 4G .. +3]
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
    *reinterpret_cast<bf16x4*>(dqs + LQ::off(16 * tt + lc, j0 + 4 * G)) =
        to_bf16x4(dqa[tt]);
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    f32x4 e = eg[st];
    if constexpr (RULE == 0) e = e * rbeta[16 * st + lc];  // diag(w) E Gb, w = beta of token 16 st + lc
    if constexpr (RULE == 1) e = e * rgnu[16 * st + lc];   // muon: w_t
    const f32x4 acc = dka[st] - des[st] + e;
    *reinterpret_cast<bf16x4*>(dks + LQ::off(16 * st + lc, j0 + 4 * G)) =
        to_bf16x4(acc);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < CB_C * D / 8; e += NTHR) {
    const int r = e / (D / 8), c8 = (e % (D / 8)) * 8;
    *reinterpret_cast<bf16x8*>(dqg + r * p.sq[2] + c8) = *reinterpret_cast<const bf16x8*>(dqs + LQ::off(r, c8));
    *reinterpret_cast<bf16x8*>(dkg + r * p.sk[2] + c8) = *reinterpret_cast<const bf16x8*>(dks + LQ::off(r, c8));
  }
}

template <int D, int RULE>
static hipError_t launch_bwd(const ChunkArgs& a, hipStream_t stream) {
  if constexpr (RULE == 0) {
    // delta: the reverse scan (Gb of the odd chunks), then the token
    // gradients of chunk pairs (even checkpoints, odd Gb)
    hipError_t e = chunk_bwd_dscan_launch(a, D, stream);
    if (e != hipSuccess) return e;
    return chunk_bwd_pair_launch(a, D, stream);
  } else {
    constexpr int lds1 = StateBwdLds<D, 2>::BYTES;
    constexpr int lds2 = TokBwdLds<D>::BYTES;
    constexpr int thr2 = TokBwdLds<D>::NTHR;
    auto k1 = chunk_bwd_state<D, RULE>;
    hipError_t e = hipFuncSetAttribute((const void*)k1, hipFuncAttributeMaxDynamicSharedMemorySize, lds1);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k1, dim3((unsigned)(a.B * a.H * (D / 32))), dim3(CB_THREADS), lds1, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    auto k2 = chunk_bwd_tok<D, RULE>;
    e = hipFuncSetAttribute((const void*)k2, hipFuncAttributeMaxDynamicSharedMemorySize, lds2);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k2, dim3((unsigned)(a.B * a.H * a.N)), dim3(thr2), lds2, stream, a);
    return hipGetLastError();
  }
}

// Muon: the matrix form's per-chunk Kw, Uv and gS (chunk_prep_muon), the
// drop-in muon scan's backward on the forward's S_i, M_i (Newton-Schulz VJP,
// chunks in segments), then the token gradients with Gb_i = dU_i.
size_t chunk_bwd_muon_ws_floats(int64_t BH, int64_t N, int d, int ns) {
  const int64_t BHN = BH * N;
  // (+64: the scan's workspace starts 256-byte aligned after the scalars)
  return (size_t)(4 * BHN * (int64_t)d * d + 8 * BHN + 64 + muon_bwd_ws_total(BH, N, d, ns));
}

template <int D>
static hipError_t launch_bwd_muon_chunks(const ChunkArgs& a, int ns, int precision, float* ws, size_t ws_floats,
                                         hipStream_t stream) {
  const int64_t BH = a.B * a.H, BHN = BH * a.N, mat = (int64_t)D * D;
  float* Kw = ws;
  float* Uv = Kw + BHN * mat;
  float* gS = Uv + BHN * mat;
  float* dU = gS + BHN * mat;
  float* abm = dU + BHN * mat;  // a, b, m, n
  float* part = abm + 4 * BHN;  // da, db, dm, dn
  float* sws = ws + ((part + 4 * BHN - ws + 63) & ~(int64_t)63);  // 16-byte pieces: aligned
  const int64_t sws_floats = (int64_t)ws_floats - (sws - ws);
  hipError_t e = chunk_prep_launch(a, D, 1, true, true, Kw, Uv, gS, abm, stream);
  if (e != hipSuccess) return e;
  ScanArgs sa{};
  sa.U = Uv; sa.K = Kw; sa.a = abm; sa.b = abm + BHN; sa.m = abm + 2 * BHN; sa.n = nullptr;
  sa.S_all = a.states; sa.M_all = a.states + BHN * mat; sa.V_all = nullptr; sa.gS = gS;
  sa.dU = dU; sa.dK = nullptr;
  sa.da = part; sa.db = part + BHN; sa.dm = part + 2 * BHN; sa.dn = part + 3 * BHN;
  sa.BH = BH; sa.N = a.N; sa.dh = D; sa.rule = 1; sa.ns = ns; sa.precision = precision;
  sa.stream = stream;
  e = scan_bwd_muon_launch(sa, sws, sws_floats);
  if (e != hipSuccess) return e;
  ChunkArgs t = a;
  t.gb = dU;
  t.part = part;
  auto k = chunk_bwd_tok<D, 1>;
  e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, TokBwdLds<D>::BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)BHN), dim3(TokBwdLds<D>::NTHR), TokBwdLds<D>::BYTES, stream, t);
  return hipGetLastError();
}

// Adam at d = 128 (exact float32 scan): gS per chunk, the drop-in adam
// reverse scan on the forward's S, M, V and stored Kw, Uv, scalars, then the
// token gradients with Gb_i = dU_i.  states = [S | M | V | Kw | Uv | a b m n].
size_t chunk_bwd_adam_mat_ws_floats(int64_t BH, int64_t N, int d) {
  const int64_t BHN = BH * N;
  return (size_t)(3 * BHN * (int64_t)d * d + 8 * BHN + BHN * (d / 16) * 4 + 64);
}

hipError_t chunk_bwd_adam_mat_launch(const ChunkArgs& a, int d, float* ws, hipStream_t stream) {
  if (d != 128) return hipErrorNotSupported;
  constexpr int D = 128;
  const int64_t BH = a.B * a.H, BHN = BH * a.N, mat = (int64_t)D * D;
  const float* S = a.states;
  const float* Kw = S + 3 * BHN * mat;
  const float* Uv = S + 4 * BHN * mat;
  const float* abm = S + 5 * BHN * mat;
  float* gS = ws;
  float* dU = gS + BHN * mat;
  float* dK = dU + BHN * mat;
  float* abm2 = dK + BHN * mat;  // the prep kernel's copy of the scalars (unused)
  float* sc = abm2 + 4 * BHN;    // da, db, dm, dn
  float* part = ws + ((sc + 4 * BHN - ws + 63) & ~(int64_t)63);
  hipError_t e = chunk_prep_launch(a, D, 2, false, true, nullptr, nullptr, gS, abm2, stream);
  if (e != hipSuccess) return e;
  ScanArgs sa{};
  sa.U = Uv; sa.K = Kw; sa.a = abm; sa.b = abm + BHN; sa.m = abm + 2 * BHN; sa.n = abm + 3 * BHN;
  sa.S_all = a.states; sa.M_all = a.states + BHN * mat; sa.V_all = a.states + 2 * BHN * mat;
  sa.gS = gS; sa.dU = dU; sa.dK = dK;
  sa.da = sc; sa.db = sc + BHN; sa.dm = sc + 2 * BHN; sa.dn = sc + 3 * BHN;
  sa.BH = BH; sa.N = a.N; sa.dh = D; sa.rule = 2; sa.ns = 0; sa.precision = GMDN_PREC_IEEE;
  sa.stream = stream;
  e = scan_bwd_rows_launch(sa, part);
  if (e != hipSuccess) return e;
  e = scan_bwd_dk_launch(sa, part);
  if (e != hipSuccess) return e;
  ChunkArgs t = a;
  t.gb = dU;
  t.part = sc;
  auto k = chunk_bwd_tok<D, 2, true>;
  e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, TokBwdLds<D>::BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)BHN), dim3(TokBwdLds<D>::NTHR), TokBwdLds<D>::BYTES, stream, t);
  return hipGetLastError();
}

hipError_t chunk_bwd_muon_launch(const ChunkArgs& a, int d, int ns, int precision, float* ws, size_t ws_floats,
                                 hipStream_t s) {
  if (d == 128) return launch_bwd_muon_chunks<128>(a, ns, precision, ws, ws_floats, s);
  if (d == 64) return launch_bwd_muon_chunks<64>(a, ns, precision, ws, ws_floats, s);
  return hipErrorNotSupported;
}

hipError_t chunk_bwd_launch(const ChunkArgs& a, int d, int rule, hipStream_t s) {
  if (rule == 0) return d == 128 ? launch_bwd<128, 0>(a, s) : launch_bwd<64, 0>(a, s);
  // adam at d = 128 is refused by the caller: its VJP is ill-conditioned there
  if (rule == 2 && d == 64) return launch_bwd<64, 2>(a, s);
  return hipErrorNotSupported;
}

}  // namespace gmdn
