// Level A: the drop-in chunk state scan, fast_state_scan(U, K, a, b, m, n,
// rule, ns) (reference fast_scan.py:403-414; kernels :206-331; math :72-186).
//
// Row-separable rules (delta, adam).  Row r of G_i = U_i - S_i K_i needs only
// row r of S_i, and the delta/adam updates are elementwise, so every 16-row
// tile of S is an independent recurrence.  One wave owns one row tile for the
// whole sequence and keeps it in registers as D-layout tiles of S^T (lane <->
// row r, registers <-> columns c); a workgroup of two waves shares one
// LDS-staged copy of each chunk's K (fp32, swizzled, double buffered and
// filled by global_load_lds_dwordx4 while the previous chunk computes).
//
//   forward, chunk i, wave tile rows r:
//     G^T = U^T - K^T S^T       (MFMA tiles: A = K^T rows (LDS column reads),
//                                B = -S^T from the wave's own tiles, pair order)
//     delta: S^T <- a S^T + G^T
//     adam : M^T <- m M^T + (1-m) G^T ; V^T <- n V^T + (1-n) G^T.^2 ;
//            S^T <- a S^T + b M^T / (sqrt(V^T) + eps)
//
//   backward (reverse over chunks; Sb = dL/dS_{i+1}):
//     delta: Gb = Sb
//     adam : elementwise VJP of the moments (fast_scan.py:167-182)
//     dU_i = Gb ;  Sb <- a Sb - Gb K^T + gS_i   (A = K rows (LDS row reads),
//                                                B = -Gb^T from registers)
//   dK_i = -S_i^T Gb_i and the scalar gradients are formed per chunk by a
//   second, chunk-parallel kernel (contraction over all rows of S).
#include "prec.h"
#include "scan_a.h"

namespace gmdn {

constexpr int A_WAVES = 2;                 // row tiles per workgroup
constexpr int A_THREADS = A_WAVES * 64;

// blockIdx -> (bh, row block).  Workgroups are dispatched round-robin over
// the 8 XCDs; keep all row blocks of one (b, h) on one XCD so they share its
// K_i stream through that XCD's L2.
GMDN_DEV void map_rows_block(int64_t BH, int nblk, int64_t& bh, int& blk) {
  const int64_t x = blockIdx.x;
  if (BH % 8 == 0) {
    const int64_t xcd = x & 7, slot = x >> 3;
    blk = (int)(slot % nblk);
    bh = (slot / nblk) * 8 + xcd;
  } else {
    bh = x / nblk;
    blk = (int)(x % nblk);
  }
}

template <int D, int RULE, int PREC>
__global__ void __launch_bounds__(A_THREADS)
scan_fwd_rows(const float* __restrict__ U, const float* __restrict__ K,
              const float* __restrict__ av, const float* __restrict__ bv,
              const float* __restrict__ mv, const float* __restrict__ nv,
              float* __restrict__ S_all, float* __restrict__ M_all,
              float* __restrict__ V_all, int64_t BH, int N) {
  using P = typename PrecSel<PREC>::T;
  constexpr int NT = D / 16;   // 16-wide column tiles of a row tile
  constexpr int NKB = D / 32;  // 32-wide k-blocks
  extern __shared__ __align__(16) float smem[];

  int64_t bh;
  int blk;
  map_rows_block(BH, D / (16 * A_WAVES), bh, blk);
  const int l = lane_id(), G = l >> 4, rl = l & 15;
  const int r0 = (blk * A_WAVES + wave_id()) * 16;  // first row of this wave's tile
  const int64_t mat = (int64_t)D * D;
  const float* Ub = U + bh * N * mat;
  const float* Kb = K + bh * N * mat;

  f32x4 S[NT], M[NT], V[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) S[t] = M[t] = V[t] = zero4();

  // row r0+rl, columns 16t + 4G .. +3 of a (D x D) matrix at base
  auto roff = [&](int t) { return (int64_t)(r0 + rl) * D + 16 * t + 4 * G; };

  if (N > 0) lds_dma_matrix<D, A_THREADS>(smem, Kb);
  f32x4 Unext[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) Unext[t] = *reinterpret_cast<const f32x4*>((Ub + roff(t)));
  wait_vmem();
  __syncthreads();

  for (int i = 0; i < N; ++i) {
    const float* kl = (smem + (i & 1) * D * D);
    f32x4 Ucur[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) Ucur[t] = Unext[t];
    if (i + 1 < N) {
      lds_dma_matrix<D, A_THREADS>((smem + ((i + 1) & 1) * D * D), Kb + (i + 1) * mat);
#pragma unroll
      for (int t = 0; t < NT; ++t) Unext[t] = *reinterpret_cast<const f32x4*>((Ub + (i + 1) * mat + roff(t)));
    }
    const int64_t si = bh * N + i;
    // pre-update states
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      *reinterpret_cast<f32x4*>((S_all + si * mat + roff(t))) = S[t];
      if constexpr (RULE == 2) {
        if (M_all) *reinterpret_cast<f32x4*>((M_all + si * mat + roff(t))) = M[t];
        if (V_all) *reinterpret_cast<f32x4*>((V_all + si * mat + roff(t))) = V[t];
      }
    }
    // B operands: -S^T, one per k-block
    typename P::Op Bop[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Bop[kb] = P::pack(-S[2 * kb], -S[2 * kb + 1]);
    const float a = av[si];
    float b = 0.f, m = 0.f, n = 0.f;
    if constexpr (RULE == 2) {
      b = bv[si];
      m = mv[si];
      n = nv[si];
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 g = Ucur[t];  // G^T tile rows c = 16t.., cols = this wave's rows
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) g = P::mma(col_op<P, SwzMat<D>>(kl, 32 * kb, 16 * t), Bop[kb], g);
      if constexpr (RULE == 0) {
        S[t] = a * S[t] + g;
      } else {
        M[t] = m * M[t] + (1.f - m) * g;
        V[t] = n * V[t] + (1.f - n) * g * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) S[t][j] = a * S[t][j] + b * M[t][j] / (sqrtf(V[t][j]) + 1e-6f);
      }
    }
    wait_vmem();
    __syncthreads();
  }
}

// ------------------------------------- forward, 8 waves per 32 rows (bf16x3)
// The same recurrence with one workgroup of 8 waves per 32 rows of S: wave
// (rt, cq) holds rows 32 blk + 16 rt + lc and column quarter cq as D-layout
// tiles of S^T.  The contraction G = U - S K runs over all columns of S, so
// the workgroup's rows are exchanged each chunk as split bf16 planes in LDS;
// K_i is staged once per chunk, as split bf16 planes (double buffered), by
// all 512 threads from fp32 loads issued one chunk ahead.  Every MFMA operand
// is then a plain LDS read.
template <int D>
struct Rows8Lds {
  static constexpr int PLANE = D * D * 2;   // one bf16 plane of K_i (bytes)
  static constexpr int K0 = 0;              // [buffer][hi | lo]
  static constexpr int XSP = 32 * D * 2;    // the workgroup's S rows, one plane
  static constexpr int XS0 = K0 + 4 * PLANE;
  static constexpr int BYTES = XS0 + 2 * XSP;
  static_assert(BYTES <= 160 * 1024, "row scan LDS exceeds the 160 KiB of a CU");
};
constexpr int A8_THREADS = 512;

template <int D, int RULE>
__global__ void __launch_bounds__(A8_THREADS)
scan_fwd_rows8(const float* __restrict__ U, const float* __restrict__ K,
               const float* __restrict__ av, const float* __restrict__ bv,
               const float* __restrict__ mv, const float* __restrict__ nv,
               float* __restrict__ S_all, float* __restrict__ M_all,
               float* __restrict__ V_all, int64_t BH, int N) {
  using L = BSwz<D>;
  using R = Rows8Lds<D>;
  using P = PrecX3;
  constexpr int NKB = D / 32;                // k-blocks over all columns of S
  constexpr int TPW = D / 64;                // column tiles per wave
  constexpr int ROWB = D * 2;                // bytes per row of a plane
  constexpr int PR = D / 4;                  // fp32 pieces per row of K
  constexpr int NQ = D * PR / A8_THREADS;    // pieces of K_i per thread
  constexpr int RSTEP = A8_THREADS / PR;     // rows between a thread's pieces
  static_assert(NQ * A8_THREADS == D * PR && RSTEP % 16 == 0, "K pieces split in swizzle-keeping row steps");
  extern __shared__ __align__(16) float smem[];

  int64_t bh;
  int blk;
  map_rows_block(BH, D / 32, bh, blk);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int rt = w >> 2, cq = w & 3;
  const int row = 32 * blk + 16 * rt + lc;   // this lane's row of S
  const int64_t mat = (int64_t)D * D;
  const float* Ub = U + bh * N * mat;
  const float* Kb = K + bh * N * mat;
  const lds_ptr L0 = lds_base(smem);

  // per-lane LDS offsets (row tiles, k-blocks and planes are immediates)
  uint32_t kcol[TPW], xsw[TPW], xsr[NKB][2];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int ct = cq * TPW + u;
    kcol[u] = swz_off<L>(4 * G + (lc >> 2), 16 * ct + 4 * (lc & 3));
    xsw[u] = swz_off<L>(16 * rt + lc, 16 * ct + 4 * G);
  }
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int h = 0; h < 2; ++h) xsr[kb][h] = swz_off<L>(16 * rt + lc, 32 * kb + 16 * h + 4 * G);
  // K staging: thread j takes pieces (j / PR + q RSTEP, 4 (j % PR))
  const int kr = threadIdx.x / PR, kc = (threadIdx.x % PR) * 4;
  const uint32_t kdst = swz_off<L>(kr, kc);
  const int64_t ksrc = (int64_t)kr * D + kc;
  auto roff = [&](int u) { return (int64_t)row * D + 16 * (cq * TPW + u) + 4 * G; };

  f32x4 Kpre[NQ];
  auto load_k = [&](int i) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) Kpre[q] = *reinterpret_cast<const f32x4*>(Kb + i * mat + ksrc + q * RSTEP * D);
  };
  auto stage_k = [&](int buf) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      bf16x4 hi, lo;
      split4(Kpre[q], hi, lo);
      const uint32_t o = R::K0 + buf * 2 * R::PLANE + kdst + q * RSTEP * ROWB;
      lds_st<bf16x4>(L0 + o, hi);
      lds_st<bf16x4>(L0 + (o + R::PLANE), lo);
    }
  };

  f32x4 S[TPW], M[TPW], V[TPW], Unext[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) S[u] = M[u] = V[u] = Unext[u] = zero4();
  if (N > 0) {
    load_k(0);
    stage_k(0);
#pragma unroll
    for (int u = 0; u < TPW; ++u) Unext[u] = *reinterpret_cast<const f32x4*>(Ub + roff(u));
  }
  if (N > 1) load_k(1);
  __syncthreads();

  for (int i = 0; i < N; ++i) {
    const int buf = i & 1;
    const int64_t si = bh * N + i;
    f32x4 Ucur[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      Ucur[u] = Unext[u];
      // pre-update state (and adam's moments)
      *reinterpret_cast<f32x4*>(S_all + si * mat + roff(u)) = S[u];
      if constexpr (RULE == 2) {
        if (M_all) *reinterpret_cast<f32x4*>(M_all + si * mat + roff(u)) = M[u];
        if (V_all) *reinterpret_cast<f32x4*>(V_all + si * mat + roff(u)) = V[u];
      }
      // this wave's split S tile -> the exchange planes
      bf16x4 hi, lo;
      split4(S[u], hi, lo);
      lds_st<bf16x4>(L0 + (R::XS0 + xsw[u]), hi);
      lds_st<bf16x4>(L0 + (R::XS0 + xsw[u] + R::XSP), lo);
    }
    __syncthreads();  // S rows published (K_i staged by the last barrier)
    // B operands: this lane's row of S over every k-block (pair order)
    P::Op Sop[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      Sop[kb].hi = cat8(lds_ld<bf16x4>(L0 + (R::XS0 + xsr[kb][0])), lds_ld<bf16x4>(L0 + (R::XS0 + xsr[kb][1])));
      Sop[kb].lo = cat8(lds_ld<bf16x4>(L0 + (R::XS0 + R::XSP + xsr[kb][0])),
                        lds_ld<bf16x4>(L0 + (R::XS0 + R::XSP + xsr[kb][1])));
    }
    const float a = av[si];
    float b = 0.f, m = 0.f, n = 0.f;
    if constexpr (RULE == 2) {
      b = bv[si];
      m = mv[si];
      n = nv[si];
    }
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      // (S K)^T tile: A = K^T (column reads of K_i), B = S^T
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const uint32_t o = R::K0 + buf * 2 * R::PLANE + kcol[u] + kb * 32 * ROWB;
        P::Op A;
        A.hi = cat8(lds_tr16(L0 + o), lds_tr16(L0 + (o + 16 * ROWB)));
        A.lo = cat8(lds_tr16(L0 + (o + R::PLANE)), lds_tr16(L0 + (o + R::PLANE + 16 * ROWB)));
        acc = P::mma(A, Sop[kb], acc);
      }
      const f32x4 g = Ucur[u] - acc;  // G^T = U^T - K^T S^T
      if constexpr (RULE == 0) {
        S[u] = a * S[u] + g;
      } else {
        M[u] = m * M[u] + (1.f - m) * g;
        V[u] = n * V[u] + (1.f - n) * g * g;
#pragma unroll
        for (int j = 0; j < 4; ++j) S[u][j] = a * S[u][j] + b * M[u][j] * hw_rcp(hw_sqrt(V[u][j]) + 1e-6f);
      }
    }
    // K_{i+1} into the other buffer (last read in chunk i-1); loads of K_{i+2}, U_{i+1}
    if (i + 1 < N) {
      stage_k(buf ^ 1);
#pragma unroll
      for (int u = 0; u < TPW; ++u) Unext[u] = *reinterpret_cast<const f32x4*>(Ub + (i + 1) * mat + roff(u));
    }
    if (i + 2 < N) load_k(i + 2);
    __syncthreads();  // K_{i+1} staged; the exchange planes free
  }
}

// Reverse scan for the row-separable rules.  Writes dU (= Gb) for every
// chunk, and for adam the per-row-tile partial sums of da, db, dm, dn into
// part[(bh*N + i) * n_tiles + tile][4]; delta's da is formed later from dU
// and S_all.
template <int D, int RULE, int PREC>
__global__ void __launch_bounds__(A_THREADS)
scan_bwd_rows(const float* __restrict__ U, const float* __restrict__ K,
              const float* __restrict__ av, const float* __restrict__ bv,
              const float* __restrict__ mv, const float* __restrict__ nv,
              const float* __restrict__ S_all, const float* __restrict__ M_all,
              const float* __restrict__ V_all, const float* __restrict__ gS,
              float* __restrict__ dU, float* __restrict__ part, int64_t BH, int N) {
  using P = typename PrecSel<PREC>::T;
  constexpr int NT = D / 16;
  constexpr int NKB = D / 32;
  constexpr int NTILES = D / 16;
  extern __shared__ __align__(16) float smem[];

  int64_t bh;
  int blk;
  map_rows_block(BH, D / (16 * A_WAVES), bh, blk);
  const int l = lane_id(), G = l >> 4, rl = l & 15;
  const int tile = blk * A_WAVES + wave_id();
  const int r0 = tile * 16;
  const int64_t mat = (int64_t)D * D;
  const float* Kb = K + bh * N * mat;
  auto roff = [&](int t) { return (int64_t)(r0 + rl) * D + 16 * t + 4 * G; };

  f32x4 Sb[NT], Mb[NT], Vb[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) Sb[t] = Mb[t] = Vb[t] = zero4();

  if (N > 0) lds_dma_matrix<D, A_THREADS>((smem + ((N - 1) & 1) * D * D), Kb + (int64_t)(N - 1) * mat);
  wait_vmem();
  __syncthreads();

  for (int i = N - 1; i >= 0; --i) {
    const float* kl = (smem + (i & 1) * D * D);
    if (i > 0) lds_dma_matrix<D, A_THREADS>((smem + ((i - 1) & 1) * D * D), Kb + (int64_t)(i - 1) * mat);
    const int64_t si = bh * N + i;
    const float a = av[si];
    f32x4 Gb[NT];
    if constexpr (RULE == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t) Gb[t] = Sb[t];
    } else {
      // recompute G^T = U^T - K^T S_i^T from the saved pre-update state
      const float b = bv[si], m = mv[si], n = nv[si];
      f32x4 Si[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) Si[t] = *reinterpret_cast<const f32x4*>((S_all + si * mat + roff(t)));
      typename P::Op Bop[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Bop[kb] = P::pack(-Si[2 * kb], -Si[2 * kb + 1]);
      float pda = 0.f, pdb = 0.f, pdm = 0.f, pdn = 0.f;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4 g = *reinterpret_cast<const f32x4*>((U + si * mat + roff(t)));
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) g = P::mma(col_op<P, SwzMat<D>>(kl, 32 * kb, 16 * t), Bop[kb], g);
        const f32x4 Mp = *reinterpret_cast<const f32x4*>((M_all + si * mat + roff(t)));
        const f32x4 Vp = *reinterpret_cast<const f32x4*>((V_all + si * mat + roff(t)));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float gg = g[j];
          const float Mi = m * Mp[j] + (1.f - m) * gg;
          const float Vi = n * Vp[j] + (1.f - n) * gg * gg;
          const float root = sqrtf(Vi);
          const float den = root + 1e-6f;
          const float sb = Sb[t][j];
          pda += sb * Si[t][j];
          pdb += sb * (Mi / den);
          const float ub = b * sb;
          const float Mtot = Mb[t][j] + ub / den;
          const float Vtot = Vb[t][j] - ub * Mi / (den * den) / (2.f * fmaxf(root, 1e-12f));
          pdm += Mtot * (Mp[j] - gg);
          pdn += Vtot * (Vp[j] - gg * gg);
          Mb[t][j] = m * Mtot;
          Vb[t][j] = n * Vtot;
          Gb[t][j] = (1.f - m) * Mtot + (1.f - n) * 2.f * gg * Vtot;
        }
      }
      pda = wave_sum(pda);
      pdb = wave_sum(pdb);
      pdm = wave_sum(pdm);
      pdn = wave_sum(pdn);
      if (l == 0) {
        float* pp = part + (si * NTILES + tile) * 4;
        pp[0] = pda;
        pp[1] = pdb;
        pp[2] = pdm;
        pp[3] = pdn;
      }
    }
    // dU_i = Gb
#pragma unroll
    for (int t = 0; t < NT; ++t) *reinterpret_cast<f32x4*>((dU + si * mat + roff(t))) = Gb[t];
    // Sb^T <- a Sb^T - K Gb^T + gS^T : output tile rows c' = 16t.., A = K rows, B = -Gb^T
    typename P::Op Bop[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Bop[kb] = P::pack(-Gb[2 * kb], -Gb[2 * kb + 1]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 acc = a * Sb[t] + *reinterpret_cast<const f32x4*>((gS + si * mat + roff(t)));
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) acc = P::mma(row_op<P, SwzMat<D>>(kl, 16 * t, 32 * kb), Bop[kb], acc);
      Sb[t] = acc;
    }
    wait_vmem();
    __syncthreads();
  }
}

// ------------------------------------ reverse scan, 8 waves per 32 rows (bf16x3)
// Wave (rt, cq) holds rows 32 blk + 16 rt + lc and column quarter cq of Sb as
// D-layout tiles of Sb^T (adam: also of its moment adjoints).  Per chunk the
// workgroup's -Gb rows are exchanged as split bf16 planes in LDS, since the
// update Sb <- a Sb - Gb K^T + gS contracts over every column of Gb; K_i is
// staged as split planes (double buffered) by all threads from fp32 loads
// issued one chunk ahead, read by rows for that update and by columns (adam)
// for recomputing G = U - S_i K_i, whose S_i row pieces a lane loads itself in
// the operand's k order.  Every chunk operand (gS, and adam's U, M, V, S_i)
// is loaded one chunk ahead.
template <int D, int RULE>
__global__ void __launch_bounds__(A8_THREADS)
scan_bwd_rows8(const float* __restrict__ U, const float* __restrict__ K,
               const float* __restrict__ av, const float* __restrict__ bv,
               const float* __restrict__ mv, const float* __restrict__ nv,
               const float* __restrict__ S_all, const float* __restrict__ M_all,
               const float* __restrict__ V_all, const float* __restrict__ gS,
               float* __restrict__ dU, float* __restrict__ part, int64_t BH, int N) {
  using L = BSwz<D>;
  using R = Rows8Lds<D>;
  using P = PrecX3;
  constexpr int NKB = D / 32;
  constexpr int TPW = D / 64;
  constexpr int ROWB = D * 2;
  constexpr int PR = D / 4;
  constexpr int NQ = D * PR / A8_THREADS;
  constexpr int RSTEP = A8_THREADS / PR;
  constexpr int NTILES = D / 16;
  constexpr int RED = R::BYTES;  // adam: [rt][cq][4] partial sums after the planes
  static_assert(NQ * A8_THREADS == D * PR && RSTEP % 16 == 0, "K pieces split in swizzle-keeping row steps");
  static_assert(RULE == 0 || R::BYTES + 32 * 4 <= 160 * 1024, "adam partial sums exceed the LDS");
  extern __shared__ __align__(16) float smem[];

  int64_t bh;
  int blk;
  map_rows_block(BH, D / 32, bh, blk);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int rt = w >> 2, cq = w & 3;
  const int row = 32 * blk + 16 * rt + lc;
  const int64_t mat = (int64_t)D * D;
  const float* Kb = K + bh * N * mat;
  const lds_ptr L0 = lds_base(smem);

  // per-lane LDS offsets: K rows 16 ct + lc over k-block kb (both halves of
  // the pair order), K columns (adam), exchange-plane writes and reads
  uint32_t krow[NKB][2], kcol[TPW], xsw[TPW], xsr[NKB][2];
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      krow[kb][h] = swz_off<L>(lc, 32 * kb + 16 * h + 4 * G);
      xsr[kb][h] = swz_off<L>(16 * rt + lc, 32 * kb + 16 * h + 4 * G);
    }
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int ct = cq * TPW + u;
    kcol[u] = swz_off<L>(4 * G + (lc >> 2), 16 * ct + 4 * (lc & 3));
    xsw[u] = swz_off<L>(16 * rt + lc, 16 * ct + 4 * G);
  }
  const int kr = threadIdx.x / PR, kc = (threadIdx.x % PR) * 4;
  const uint32_t kdst = swz_off<L>(kr, kc);
  const int64_t ksrc = (int64_t)kr * D + kc;
  auto roff = [&](int u) { return (int64_t)row * D + 16 * (cq * TPW + u) + 4 * G; };

  f32x4 Kpre[NQ];
  auto load_k = [&](int i) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) Kpre[q] = *reinterpret_cast<const f32x4*>(Kb + i * mat + ksrc + q * RSTEP * D);
  };
  auto stage_k = [&](int buf) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      bf16x4 hi, lo;
      split4(Kpre[q], hi, lo);
      const uint32_t o = R::K0 + buf * 2 * R::PLANE + kdst + q * RSTEP * ROWB;
      lds_st<bf16x4>(L0 + o, hi);
      lds_st<bf16x4>(L0 + (o + R::PLANE), lo);
    }
  };
  // chunk operands of this lane: gS tiles; adam: U, M, V tiles and the S_i row
  // pieces of every k-block (columns 32 kb + 16 h + 4G .. +3)
  f32x4 gsn[TPW], un[TPW], mn[TPW], vn[TPW], sn[NKB][2];
  auto load_chunk = [&](int i) {
    const int64_t base = (bh * N + i) * mat;
#pragma unroll
    for (int u = 0; u < TPW; ++u) gsn[u] = *reinterpret_cast<const f32x4*>(gS + base + roff(u));
    if constexpr (RULE == 2) {
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        un[u] = *reinterpret_cast<const f32x4*>(U + base + roff(u));
        mn[u] = *reinterpret_cast<const f32x4*>(M_all + base + roff(u));
        vn[u] = *reinterpret_cast<const f32x4*>(V_all + base + roff(u));
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          sn[kb][h] = *reinterpret_cast<const f32x4*>(S_all + base + (int64_t)row * D + 32 * kb + 16 * h + 4 * G);
    }
  };

  f32x4 Sb[TPW], Mb[TPW], Vb[TPW];
#pragma unroll
  for (int u = 0; u < TPW; ++u) Sb[u] = Mb[u] = Vb[u] = zero4();
  if (N > 0) {
    load_k(N - 1);
    stage_k((N - 1) & 1);
    load_chunk(N - 1);
  }
  if (N > 1) load_k(N - 2);
  __syncthreads();

  for (int i = N - 1; i >= 0; --i) {
    const int buf = i & 1;
    const int64_t si = bh * N + i;
    const float a = av[si];
    f32x4 gsc[TPW], Gb[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) gsc[u] = gsn[u];
    if constexpr (RULE == 0) {
#pragma unroll
      for (int u = 0; u < TPW; ++u) Gb[u] = Sb[u];
    } else {
      const float b = bv[si], m = mv[si], n = nv[si];
      P::Op Sop[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) Sop[kb] = P::pack(-sn[kb][0], -sn[kb][1]);
      float pda = 0.f, pdb = 0.f, pdm = 0.f, pdn = 0.f;
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        // G^T = U^T - K^T S_i^T : A = K^T (column reads), B = -S_i^T
        f32x4 g = un[u];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          const uint32_t o = R::K0 + buf * 2 * R::PLANE + kcol[u] + kb * 32 * ROWB;
          P::Op A;
          A.hi = cat8(lds_tr16(L0 + o), lds_tr16(L0 + (o + 16 * ROWB)));
          A.lo = cat8(lds_tr16(L0 + (o + R::PLANE)), lds_tr16(L0 + (o + R::PLANE + 16 * ROWB)));
          g = P::mma(A, Sop[kb], g);
        }
        const int ct = cq * TPW + u;  // this tile's S_i pieces, selected with constant indices
        f32x4 Si = sn[0][0];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            if (2 * kb + h == ct) Si = sn[kb][h];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float gg = g[j];
          const float Mi = m * mn[u][j] + (1.f - m) * gg;
          const float Vi = n * vn[u][j] + (1.f - n) * gg * gg;
          const float root = hw_sqrt(Vi);
          const float rden = hw_rcp(root + 1e-6f);
          const float sb = Sb[u][j];
          pda += sb * Si[j];
          pdb += sb * (Mi * rden);
          const float ub = b * sb;
          const float Mtot = Mb[u][j] + ub * rden;
          const float Vtot = Vb[u][j] - ub * Mi * rden * rden * hw_rcp(2.f * fmaxf(root, 1e-12f));
          pdm += Mtot * (mn[u][j] - gg);
          pdn += Vtot * (vn[u][j] - gg * gg);
          Mb[u][j] = m * Mtot;
          Vb[u][j] = n * Vtot;
          Gb[u][j] = (1.f - m) * Mtot + (1.f - n) * 2.f * gg * Vtot;
        }
      }
      pda = wave_sum(pda);
      pdb = wave_sum(pdb);
      pdm = wave_sum(pdm);
      pdn = wave_sum(pdn);
      if (l < 4) {
        const float v = l == 0 ? pda : l == 1 ? pdb : l == 2 ? pdm : pdn;
        lds_st<float>(L0 + (RED + (w * 4 + l) * 4), v);
      }
    }
    // dU_i = Gb ; -Gb (split) -> the exchange planes
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      *reinterpret_cast<f32x4*>(dU + si * mat + roff(u)) = Gb[u];
      bf16x4 hi, lo;
      split4(-Gb[u], hi, lo);
      lds_st<bf16x4>(L0 + (R::XS0 + xsw[u]), hi);
      lds_st<bf16x4>(L0 + (R::XS0 + xsw[u] + R::XSP), lo);
    }
    __syncthreads();  // -Gb rows (and adam's partial sums) published
    if constexpr (RULE == 2) {
      if (cq == 0 && l < 4) {
        float t = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) t += lds_ld<float>(L0 + (RED + ((4 * rt + q) * 4 + l) * 4));
        part[(si * NTILES + 2 * blk + rt) * 4 + l] = t;
      }
    }
    P::Op Gop[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      Gop[kb].hi = cat8(lds_ld<bf16x4>(L0 + (R::XS0 + xsr[kb][0])), lds_ld<bf16x4>(L0 + (R::XS0 + xsr[kb][1])));
      Gop[kb].lo = cat8(lds_ld<bf16x4>(L0 + (R::XS0 + R::XSP + xsr[kb][0])),
                        lds_ld<bf16x4>(L0 + (R::XS0 + R::XSP + xsr[kb][1])));
    }
    // Sb^T <- a Sb^T - K Gb^T + gS^T : A = K rows 16 ct.., B = -Gb^T
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int ct = cq * TPW + u;
      f32x4 acc = a * Sb[u] + gsc[u];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const uint32_t o0 = R::K0 + buf * 2 * R::PLANE + 16 * ct * ROWB;
        P::Op A;
        A.hi = cat8(lds_ld<bf16x4>(L0 + (o0 + krow[kb][0])), lds_ld<bf16x4>(L0 + (o0 + krow[kb][1])));
        A.lo = cat8(lds_ld<bf16x4>(L0 + (o0 + R::PLANE + krow[kb][0])),
                    lds_ld<bf16x4>(L0 + (o0 + R::PLANE + krow[kb][1])));
        acc = P::mma(A, Gop[kb], acc);
      }
      Sb[u] = acc;
    }
    // K_{i-1} into the other buffer (last read in chunk i+1); loads of K_{i-2} and chunk i-1
    if (i > 0) {
      stage_k(buf ^ 1);
      load_chunk(i - 1);
    }
    if (i > 1) load_k(i - 2);
    __syncthreads();  // K_{i-1} staged; the exchange planes free
  }
}

// Chunk-parallel part of the backward: dK_i = -S_i^T Gb_i (contraction over
// the rows of S) and the scalar gradients of chunk i.  One workgroup of
// A_KWAVES waves per (bh, i); S_i and Gb_i are staged in swizzled LDS.
constexpr int A_KWAVES = 4;
constexpr int A_KTHREADS = A_KWAVES * 64;

template <int D, int RULE, int PREC>
__global__ void __launch_bounds__(A_KTHREADS)
scan_bwd_dk(const float* __restrict__ S_all, const float* __restrict__ dU,
            const float* __restrict__ part, float* __restrict__ dK,
            float* __restrict__ da, float* __restrict__ db, float* __restrict__ dm,
            float* __restrict__ dn, int64_t BH, int N) {
  using P = typename PrecSel<PREC>::T;
  constexpr int NT = D / 16;
  constexpr int NKB = D / 32;
  extern __shared__ __align__(16) float smem[];
  float* Sl = smem;
  float* Gl = smem + D * D;
  __shared__ float red[A_KWAVES];
  const int64_t si = blockIdx.x;  // = bh * N + i
  const int64_t mat = (int64_t)D * D;
  lds_dma_matrix<D, A_KTHREADS>(Sl, S_all + si * mat);
  lds_dma_matrix<D, A_KTHREADS>(Gl, dU + si * mat);
  wait_vmem();
  __syncthreads();
  const int w = wave_id(), l = lane_id();
  // dK^T[c][c'] = -sum_r Gb[r][c] S[r][c'] ; tile (tc, tcp) with rows c.
  // Stored as dK[c'][c]: lane (c', G) of the D-layout tile of dK^T^T...
  // Output tile of dK (rows c' = 16 tr, cols c = 16 tc): A = S^T rows c'
  // (k = r, column reads of S), B = Gb (k = r, column reads of Gb).
  for (int tile = w; tile < NT * NT; tile += A_KWAVES) {
    const int tr = tile / NT, tc = tile % NT;
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
      acc = P::mma(col_op<P, SwzMat<D>>(Sl, 32 * kb, 16 * tr), col_op<P, SwzMat<D>>(Gl, 32 * kb, 16 * tc), acc);
    // D-layout: lane (c = l%16, G) holds dK[16tr + 4G + j][16tc + c]
    float* out = dK + si * mat + (int64_t)(16 * tr + 4 * (l >> 4)) * D + 16 * tc + (l & 15);
#pragma unroll
    for (int j = 0; j < 4; ++j) out[(int64_t)j * D] = -acc[j];
  }
  if constexpr (RULE == 0) {
    // da_i = <Sb_{i+1}, S_i> = <dU_i, S_i> for delta
    float s = 0.f;
    for (int e = threadIdx.x; e < D * D; e += A_KTHREADS) {
      const int r = e / D, c = e % D;
      s += Sl[SwzMat<D>::off(r, c)] * Gl[SwzMat<D>::off(r, c)];
    }
    s = wave_sum(s);
    if (l == 0) red[w] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
      float t = 0.f;
      for (int q = 0; q < A_KWAVES; ++q) t += red[q];
      da[si] = t;
      db[si] = 0.f;
      dm[si] = 0.f;
      dn[si] = 0.f;
    }
  } else if constexpr (RULE == 2) {
    if (threadIdx.x < 4) {
      float t = 0.f;
      for (int q = 0; q < D / 16; ++q) t += part[(si * (D / 16) + q) * 4 + threadIdx.x];
      float* dst = threadIdx.x == 0 ? da : threadIdx.x == 1 ? db : threadIdx.x == 2 ? dm : dn;
      dst[si] = t;
    }
  }
  // RULE == 1: the muon backward kernel writes the scalar gradients itself
}

// The chunk-parallel part with 8 waves: S_i and Gb_i staged as split bf16
// planes (loaded as 16-byte fp32 pieces by all threads, which also form
// delta's da = <Gb_i, S_i> in fp32 on the way), every operand a transposing
// LDS read, and each output tile formed transposed, (Gb^T S)[c][c'] =
// -dK[c'][c], so that a lane writes four consecutive columns of dK.
template <int D>
struct Dk8Lds {
  static constexpr int PLANE = D * D * 2;
  static constexpr int S0 = 0;          // S_i hi, lo
  static constexpr int G0 = 2 * PLANE;  // Gb_i hi, lo
  static constexpr int RED = 4 * PLANE; // per-wave partial sums
  static constexpr int BYTES = RED + 8 * 4;
  static_assert(BYTES <= 160 * 1024, "dK LDS exceeds the 160 KiB of a CU");
};

template <int D, int RULE>
__global__ void __launch_bounds__(A8_THREADS)
scan_bwd_dk8(const float* __restrict__ S_all, const float* __restrict__ dU,
             const float* __restrict__ part, float* __restrict__ dK,
             float* __restrict__ da, float* __restrict__ db, float* __restrict__ dm,
             float* __restrict__ dn, int64_t BH, int N) {
  using L = BSwz<D>;
  using R = Dk8Lds<D>;
  using P = PrecX3;
  constexpr int NT = D / 16;
  constexpr int NKB = D / 32;
  constexpr int ROWB = D * 2;
  constexpr int PR = D / 4;
  constexpr int NQ = D * PR / A8_THREADS;
  constexpr int RSTEP = A8_THREADS / PR;
  constexpr int NW = A8_THREADS / 64;
  static_assert(NQ * A8_THREADS == D * PR && RSTEP % 16 == 0, "pieces split in swizzle-keeping row steps");
  static_assert((NT * NT) % NW == 0, "output tiles split evenly over the waves");
  extern __shared__ __align__(16) float smem[];
  const lds_ptr L0 = lds_base(smem);
  const int64_t si = blockIdx.x;  // = bh * N + i
  const int64_t mat = (int64_t)D * D;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = lane_id(), G = l >> 4, lc = l & 15;

  // ---- staging (and delta's da from the fp32 values)
  {
    const int kr = threadIdx.x / PR, kc = (threadIdx.x % PR) * 4;
    const float* sg = S_all + si * mat + (int64_t)kr * D + kc;
    const float* gg = dU + si * mat + (int64_t)kr * D + kc;
    const uint32_t dst = swz_off<L>(kr, kc);
    f32x4 xs[NQ], xg[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      xs[q] = *reinterpret_cast<const f32x4*>(sg + q * RSTEP * D);
      xg[q] = *reinterpret_cast<const f32x4*>(gg + q * RSTEP * D);
    }
    float dot = 0.f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const uint32_t o = dst + q * RSTEP * ROWB;
      bf16x4 hi, lo;
      split4(xs[q], hi, lo);
      lds_st<bf16x4>(L0 + (R::S0 + o), hi);
      lds_st<bf16x4>(L0 + (R::S0 + R::PLANE + o), lo);
      split4(xg[q], hi, lo);
      lds_st<bf16x4>(L0 + (R::G0 + o), hi);
      lds_st<bf16x4>(L0 + (R::G0 + R::PLANE + o), lo);
      if constexpr (RULE == 0) dot += xs[q][0] * xg[q][0] + xs[q][1] * xg[q][1] + xs[q][2] * xg[q][2] + xs[q][3] * xg[q][3];
    }
    if constexpr (RULE == 0) {
      dot = wave_sum(dot);
      if (l == 0) reinterpret_cast<float*>(smem + R::RED / 4)[w] = dot;
    }
  }
  __syncthreads();

  // ---- dK tiles: (Gb^T S) tile (tc, tr) = -dK^T; A = Gb columns, B = S columns
  uint32_t pcol[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) pcol[t] = swz_off<L>(4 * G + (lc >> 2), 16 * t + 4 * (lc & 3));
  auto colop = [&](uint32_t base, int kb, int t) {
    const uint32_t o = base + pcol[t] + kb * 32 * ROWB;
    P::Op x;
    x.hi = cat8(lds_tr16(L0 + o), lds_tr16(L0 + (o + 16 * ROWB)));
    x.lo = cat8(lds_tr16(L0 + (o + R::PLANE)), lds_tr16(L0 + (o + R::PLANE + 16 * ROWB)));
    return x;
  };
  float* const dKi = dK + si * mat;
#pragma unroll
  for (int q = 0; q < NT * NT / NW; ++q) {
    const int tile = w + NW * q, tr = tile / NT, tc = tile % NT;
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) acc = P::mma(colop(R::G0, kb, tc), colop(R::S0, kb, tr), acc);
    // lane (c', G) holds (Gb^T S)[16 tc + 4G + j][16 tr + c'] = -dK[16 tr + c'][16 tc + 4G + j]
    *reinterpret_cast<f32x4*>(dKi + (int64_t)(16 * tr + lc) * D + 16 * tc + 4 * G) = -acc;
  }

  // ---- scalar gradients of the chunk
  if constexpr (RULE == 0) {
    if (threadIdx.x == 0) {
      const float* red = reinterpret_cast<const float*>(smem + R::RED / 4);
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < NW; ++q) t += red[q];
      da[si] = t;
      db[si] = 0.f;
      dm[si] = 0.f;
      dn[si] = 0.f;
    }
  } else if constexpr (RULE == 2) {
    if (threadIdx.x < 4) {
      float t = 0.f;
      for (int q = 0; q < D / 16; ++q) t += part[(si * (D / 16) + q) * 4 + threadIdx.x];
      float* dst = threadIdx.x == 0 ? da : threadIdx.x == 1 ? db : threadIdx.x == 2 ? dm : dn;
      dst[si] = t;
    }
  }
  // RULE == 1: the muon backward kernel writes the scalar gradients itself
}

// ---------------------------------------------------------------- launchers
template <int D, int RULE, int PREC>
static hipError_t launch_fwd_rows(const ScanArgs& s) {
  const int nblk = D / (16 * A_WAVES);
  const size_t lds = 2 * (size_t)D * D * sizeof(float);
  auto kern = scan_fwd_rows<D, RULE, PREC>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)(s.BH * nblk)), dim3(A_THREADS), lds, s.stream, s.U, s.K, s.a,
                     s.b, s.m, s.n, s.S_all, s.M_all, s.V_all, s.BH, (int)s.N);
  return hipGetLastError();
}

template <int D, int RULE, int PREC>
static hipError_t launch_bwd_rows(const ScanArgs& s, float* part) {
  const int nblk = D / (16 * A_WAVES);
  const size_t lds = 2 * (size_t)D * D * sizeof(float);
  auto kern = scan_bwd_rows<D, RULE, PREC>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)(s.BH * nblk)), dim3(A_THREADS), lds, s.stream, s.U, s.K, s.a,
                     s.b, s.m, s.n, s.S_all, s.M_all, s.V_all, s.gS, s.dU, part, s.BH, (int)s.N);
  return hipGetLastError();
}

template <int D, int RULE, int PREC>
static hipError_t launch_bwd_dk(const ScanArgs& s, const float* part) {
  if constexpr (PREC == 0 && D >= 64) {  // bf16x3: the 8-wave kernel
    const int lds = Dk8Lds<D>::BYTES;
    auto k8 = scan_bwd_dk8<D, RULE>;
    hipError_t e = hipFuncSetAttribute((const void*)k8, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k8, dim3((unsigned)(s.BH * s.N)), dim3(A8_THREADS), lds, s.stream, s.S_all, s.dU, part,
                       s.dK, s.da, s.db, s.dm, s.dn, s.BH, (int)s.N);
    return hipGetLastError();
  }
  const size_t lds = 2 * (size_t)D * D * sizeof(float);
  auto k2 = scan_bwd_dk<D, RULE, PREC>;
  hipError_t e = hipFuncSetAttribute((const void*)k2, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k2, dim3((unsigned)(s.BH * s.N)), dim3(A_KTHREADS), lds, s.stream, s.S_all, s.dU, part,
                     s.dK, s.da, s.db, s.dm, s.dn, s.BH, (int)s.N);
  return hipGetLastError();
}

template <int D, int PREC>
static hipError_t dk_rule(const ScanArgs& s, const float* part) {
  switch (s.rule) {
    case 0: return launch_bwd_dk<D, 0, PREC>(s, part);
    case 1: return launch_bwd_dk<D, 1, PREC>(s, part);
    default: return launch_bwd_dk<D, 2, PREC>(s, part);
  }
}

template <int D>
static hipError_t dk_prec(const ScanArgs& s, const float* part) {
  return s.precision == 0 ? dk_rule<D, 0>(s, part) : dk_rule<D, 1>(s, part);
}

hipError_t scan_bwd_dk_launch(const ScanArgs& s, const float* part) {
  switch (s.dh) {
    case 32: return dk_prec<32>(s, part);
    case 64: return dk_prec<64>(s, part);
    case 128: return dk_prec<128>(s, part);
  }
  return hipErrorInvalidValue;
}

template <int D, int RULE>
static hipError_t launch_fwd_rows8(const ScanArgs& s) {
  const int lds = Rows8Lds<D>::BYTES;
  auto kern = scan_fwd_rows8<D, RULE>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)(s.BH * (D / 32))), dim3(A8_THREADS), lds, s.stream, s.U, s.K, s.a,
                     s.b, s.m, s.n, s.S_all, s.M_all, s.V_all, s.BH, (int)s.N);
  return hipGetLastError();
}

template <int D, int PREC>
static hipError_t fwd_rows_rule(const ScanArgs& s) {
  if constexpr (PREC == 0 && D >= 64)  // bf16x3: the 8-wave kernel
    return s.rule == 0 ? launch_fwd_rows8<D, 0>(s) : launch_fwd_rows8<D, 2>(s);
  else
    return s.rule == 0 ? launch_fwd_rows<D, 0, PREC>(s) : launch_fwd_rows<D, 2, PREC>(s);
}
template <int D, int RULE>
static hipError_t launch_bwd_rows8(const ScanArgs& s, float* part) {
  const int lds = Rows8Lds<D>::BYTES + (RULE == 2 ? 32 * 4 : 0);
  auto kern = scan_bwd_rows8<D, RULE>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)(s.BH * (D / 32))), dim3(A8_THREADS), lds, s.stream, s.U, s.K, s.a,
                     s.b, s.m, s.n, s.S_all, s.M_all, s.V_all, s.gS, s.dU, part, s.BH, (int)s.N);
  return hipGetLastError();
}

template <int D, int PREC>
static hipError_t bwd_rows_rule(const ScanArgs& s, float* part) {
  // bf16x3: the 8-wave kernel (adam's at D = 128 would spill: the 2-wave one)
  if constexpr (PREC == 0 && D >= 64) {
    if (s.rule == 0) return launch_bwd_rows8<D, 0>(s, part);
    if constexpr (D == 64) return launch_bwd_rows8<D, 2>(s, part);
  }
  return s.rule == 0 ? launch_bwd_rows<D, 0, PREC>(s, part) : launch_bwd_rows<D, 2, PREC>(s, part);
}

template <int D>
static hipError_t fwd_rows_prec(const ScanArgs& s) {
  return s.precision == 0 ? fwd_rows_rule<D, 0>(s) : fwd_rows_rule<D, 1>(s);
}
template <int D>
static hipError_t bwd_rows_prec(const ScanArgs& s, float* part) {
  return s.precision == 0 ? bwd_rows_rule<D, 0>(s, part) : bwd_rows_rule<D, 1>(s, part);
}

hipError_t scan_fwd_rows_launch(const ScanArgs& s) {
  switch (s.dh) {
    case 32: return fwd_rows_prec<32>(s);
    case 64: return fwd_rows_prec<64>(s);
    case 128: return fwd_rows_prec<128>(s);
  }
  return hipErrorInvalidValue;
}

hipError_t scan_bwd_rows_launch(const ScanArgs& s, float* part) {
  switch (s.dh) {
    case 32: return bwd_rows_prec<32>(s, part);
    case 64: return bwd_rows_prec<64>(s, part);
    case 128: return bwd_rows_prec<128>(s, part);
  }
  return hipErrorInvalidValue;
}

}  // namespace gmdn
