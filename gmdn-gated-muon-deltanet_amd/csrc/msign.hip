// Outer-Muon msign on batched rectangular matrices (reference
// train_ablation.py:60-73, applied per 2-D hidden weight at :284), with its
// extern "C" entry points (include/gmdn_msign.h).
//
// With m = min(rows, cols) and n = max(rows, cols), X is the m x n
// orientation of M.  Every iterate lives in the workspace as "split pieces":
// row r of a matrix with `ld` columns is ld / 4 pieces of 16 bytes, piece q
// holding {hi, lo} bf16 of columns 4q .. 4q+3 (x = hi + lo), in the bytes the
// fp32 values would take.  Matrices are zero-padded to multiples of 128 in
// both dimensions; zero rows and columns stay zero under the iteration, so
// the padding changes nothing.  One quintic Newton-Schulz step is three
// launches of one GEMM kernel:
//
//   A  = X X^T                 (contraction over n, both operands by rows)
//   Bm = b A + c A A           (A is symmetric, so A A = A A^T: by rows)
//   X' = a X + Bm X            (X read by columns: transposing LDS reads)
//
// A and Bm are symmetric: their launches form only the tiles on and above
// the diagonal and write each off-diagonal tile twice, the mirror through an
// LDS transpose.  ns_gemm forms a 128 x 128 output tile per workgroup of four
// waves (64 x 64 each) from 32-wide contraction blocks that arrive by LDS-DMA
// in a 2-stage ring (64 KiB, two workgroups per CU).  The pieces copy to LDS
// unchanged (no conversion on the way), and every MFMA operand is then one
// or two LDS reads.  The products are split (hi hi + hi lo + lo hi); the MFMA
// operands are swapped so that each lane's accumulator is four consecutive
// columns of one output row, which leaves as one 16-byte piece.  The
// normalisation and the final unpacking move tall matrices through 64 x 64
// LDS transposes.
#include "../../include/gmdn_msign.h"
#include "tile.h"

namespace gmdn {
namespace {

constexpr int MS_TILE = 128;                // output tile edge; padding unit
constexpr int MS_KB = 32;                   // contraction per ring stage
constexpr int MS_THREADS = 256;             // 4 waves as 2 x 2 blocks of 64 x 64
constexpr int MS_STAGES = 2;
constexpr int MS_NPART = 64;                // norm partial sums per matrix
constexpr int MS_MAXDIM = 32768;
constexpr float NS_A = 3.4445f, NS_B = -4.7750f, NS_C = 2.0315f;  // train_ablation.py:66

struct MsLds {
  static constexpr int PIECES = MS_TILE * MS_KB / 4;  // 16-byte pieces per operand tile
  static constexpr int OPB = PIECES * 16;             // 16 KiB
  static constexpr int STAGE = 2 * OPB;               // P tile, then Q tile
  static constexpr int NOPS = PIECES / MS_THREADS;    // LDS-DMA copies per thread and tile
  static constexpr int MIRROR_LD = 68;                // words per row of a wave's transposed 64 x 64 tile
  static constexpr int MIRROR = 64 * MIRROR_LD * 4;   // bytes of it, one per wave after the loop
  static constexpr int RING = MS_STAGES * STAGE;
  static constexpr int BYTES = RING > 4 * MIRROR ? RING : 4 * MIRROR;
};

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

template <typename T>
GMDN_DEV float ld_elem(const T* p) { return (float)*p; }

// four consecutive elements (16-byte aligned for float, 8-byte for bf16)
template <typename T>
GMDN_DEV f32x4 ld4(const T* p);
template <>
GMDN_DEV f32x4 ld4<float>(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
template <>
GMDN_DEV f32x4 ld4<bf16>(const bf16* p) {
  const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

// ------------------------------------------------------------------ norm
// Partial sums of squares: workgroup (blk, b) takes elements (VEC: groups of
// four) blk*256 + t, strided by MS_NPART * 256, of matrix b.
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) ns_norm_partial(const T* __restrict__ M, float* __restrict__ part,
                                                       int64_t per) {
  __shared__ float red[4];
  const int64_t b = blockIdx.y;
  const T* Mb = M + b * per;
  float s = 0.f;
  if constexpr (VEC) {
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; 4 * e < per; e += (int64_t)MS_NPART * 256) {
      const f32x4 v = ld4(Mb + 4 * e);
      s += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
    }
  } else {
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < per; e += (int64_t)MS_NPART * 256) {
      const float v = ld_elem(Mb + e);
      s += v * v;
    }
  }
  s = wave_sum(s);
  if (lane_id() == 0) red[wave_id()] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[b * MS_NPART + blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

GMDN_DEV float block_norm(const float* part, int64_t b, float* nrm_s) {
  if (threadIdx.x < 64) {
    const float t = wave_sum(part[b * MS_NPART + threadIdx.x]);
    if (threadIdx.x == 0) *nrm_s = sqrtf(t);
  }
  __syncthreads();
  return *nrm_s;
}

// ------------------------------------------------------------------ pack
// X0 = X / (|X|_F + eps) as split pieces, zero-padded to mp x np, X = M
// (rows <= cols).  One thread per piece; VEC: cols % 4 == 0, so a piece is
// one aligned load of M.
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) ns_pack(const T* __restrict__ M, const float* __restrict__ part,
                                               char* __restrict__ X, int64_t x_bs, int m, int n, int mp,
                                               int np, float eps) {
  __shared__ float nrm_s;
  const int64_t b = blockIdx.y;
  const float den = block_norm(part, b, &nrm_s) + eps;
  const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nq = np / 4;
  if (p >= (int64_t)mp * nq) return;
  const int r = (int)(p / nq), q = (int)(p % nq);
  const T* Mb = M + b * (int64_t)m * n;
  f32x4 v = zero4();
  if constexpr (VEC) {
    if (r < m && 4 * q < n) v = ld4(Mb + (int64_t)r * n + 4 * q);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (r < m && 4 * q + e < n) v[e] = ld_elem(Mb + (int64_t)r * n + 4 * q + e);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = v[e] / den;  // the reference divides (train_ablation.py:65)
  *reinterpret_cast<bf16x8*>(X + b * x_bs + ((int64_t)r * np + 4 * q) * 4) = split_piece(v);
}

// Transposing pack, X = M^T (M is n x m with n > m): workgroup (tile, b)
// moves a 64 x 64 block through LDS; rows of M are read and rows of X
// written 256 contiguous bytes per wave instruction.
template <typename T>
__global__ void __launch_bounds__(256) ns_pack_tr(const T* __restrict__ M, const float* __restrict__ part,
                                                  char* __restrict__ X, int64_t x_bs, int m, int n, int mp,
                                                  int np, float eps) {
  __shared__ float nrm_s;
  __shared__ float tile[64][65];  // [row of M][column of M]
  const int64_t b = blockIdx.y;
  const float den = block_norm(part, b, &nrm_s) + eps;
  const int tx = mp / 64;
  const int r0 = (int)(blockIdx.x % tx) * 64;  // first row of X (= column of M)
  const int c0 = (int)(blockIdx.x / tx) * 64;  // first column of X (= row of M)
  const T* Mb = M + b * (int64_t)m * n;
  const int t = threadIdx.x, lr = t >> 6, lcol = t & 63;
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int mr = c0 + 4 * it + lr, mc = r0 + lcol;
    tile[4 * it + lr][lcol] = (mr < n && mc < m) ? ld_elem(Mb + (int64_t)mr * m + mc) : 0.f;
  }
  __syncthreads();
  const int q = t & 15;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int rl = (t >> 4) + 16 * it;
    f32x4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = tile[4 * q + e][rl] / den;
    *reinterpret_cast<bf16x8*>(X + b * x_bs + ((int64_t)(r0 + rl) * np + c0 + 4 * q) * 4) = split_piece(v);
  }
}

// ---------------------------------------------------------------- unpack
// out (rows x cols, dtype T) = X from the padded pieces.
template <typename T>
__global__ void __launch_bounds__(256) ns_unpack(const char* __restrict__ X, T* __restrict__ out, int64_t x_bs,
                                                 int rows, int cols, int np) {
  const int64_t b = blockIdx.y;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)rows * cols) return;
  const int orow = (int)(e / cols), ocol = (int)(e % cols);
  const bf16* pc = reinterpret_cast<const bf16*>(X + b * x_bs + ((int64_t)orow * np + (ocol & ~3)) * 4);
  const float v = (float)pc[ocol & 3] + (float)pc[4 + (ocol & 3)];
  out[b * (int64_t)rows * cols + e] = (T)v;
}

// Transposing unpack, out = X^T (out is rows x cols with rows > cols, X is
// cols x rows): 64 x 64 blocks through LDS, both sides row-contiguous.
template <typename T>
__global__ void __launch_bounds__(256) ns_unpack_tr(const char* __restrict__ X, T* __restrict__ out, int64_t x_bs,
                                                    int rows, int cols, int mp, int np) {
  __shared__ float tile[64][65];  // [row of X][column of X]
  const int64_t b = blockIdx.y;
  const int tx = mp / 64;
  const int xr0 = (int)(blockIdx.x % tx) * 64;  // first row of X (= column of out)
  const int xc0 = (int)(blockIdx.x / tx) * 64;  // first column of X (= row of out)
  const int t = threadIdx.x, q = t & 15;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int rl = (t >> 4) + 16 * it;
    const f32x4 v = unsplit_piece(*reinterpret_cast<const bf16x8*>(X + b * x_bs + ((int64_t)(xr0 + rl) * np + xc0 + 4 * q) * 4));
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[rl][4 * q + e] = v[e];
  }
  __syncthreads();
  const int lr = t >> 6, lcol = t & 63;
  T* ob = out + b * (int64_t)rows * cols;
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const int orow = xc0 + 4 * it + lr, ocol = xr0 + lcol;
    if (orow < rows && ocol < cols) ob[(int64_t)orow * cols + ocol] = (T)tile[lcol][4 * it + lr];
  }
}

// ------------------------------------------------------------------ GEMM
// C[i][j] = sum_k P[i][k] Q(k, j)   (EPI: alpha * that + beta * D[i][j])
// P: rows i, k contiguous.  Q: NN -- rows k, j contiguous (read by columns);
// otherwise rows j, k contiguous (Q(k, j) = Q[j][k], read by rows).  All
// are split-piece matrices of one batch entry each; C and D share a layout.
//
// LDS tiles: P (and Q by rows) 128 rows x 8 pieces, piece q of row r at slot
// 8 r + (q ^ (r & 7)); Q by columns 32 rows x 32 pieces, piece q of row k at
// 32 k + (q ^ 4 (k & 3)).  Wave (wi, wj) owns output rows 64 wi .. and
// columns 64 wj .. of the tile.
struct PieceOp {
  bf16x8 hi, lo;
};

GMDN_DEV PieceOp row_op(lds_cptr p0, lds_cptr p1) {
  const bf16x8 a = lds_ld<bf16x8>(p0), b = lds_ld<bf16x8>(p1);
  PieceOp r;
  r.hi = __builtin_shufflevector(a, b, 0, 1, 2, 3, 8, 9, 10, 11);
  r.lo = __builtin_shufflevector(a, b, 4, 5, 6, 7, 12, 13, 14, 15);
  return r;
}

GMDN_DEV f32x4 mma3(const PieceOp& a, const PieceOp& b, f32x4 acc) {
  acc = mfma(a.hi, b.hi, acc);
  acc = mfma(a.hi, b.lo, acc);
  acc = mfma(a.lo, b.hi, acc);
  return acc;
}

template <bool NN, bool EPI, bool SYM>
__global__ void __launch_bounds__(MS_THREADS)
ns_gemm(const char* __restrict__ P, const char* __restrict__ Q, const char* __restrict__ Dm,
        char* __restrict__ Cm, int64_t p_bs, int64_t q_bs, int64_t c_bs, int p_ld, int q_ld, int c_ld, int mt,
        int nt, int K, float alpha, float beta) {
  extern __shared__ __align__(16) char ms_smem[];
  using Lp = MsLds;
  const lds_ptr L0 = lds_base(ms_smem);
  // XCD-aware order: the 8 XCDs take contiguous ranges of the (b, ti, tj)
  // tile order, so the workgroups of one P row panel share an L2.
  const int64_t total = gridDim.x, x = blockIdx.x;
  const int64_t t = (total % 8 == 0) ? (x % 8) * (total / 8) + x / 8 : x;
  // SYM (square symmetric C, mt == nt): only the tiles ti <= tj, in row order
  const int tiles = SYM ? mt * (mt + 1) / 2 : mt * nt;
  const int64_t b = t / tiles;
  int rem = (int)(t % tiles), ti, tj;
  if constexpr (SYM) {
    ti = 0;
    while (rem >= mt - ti) {
      rem -= mt - ti;
      ++ti;
    }
    tj = ti + rem;
  } else {
    ti = rem / nt;
    tj = rem % nt;
  }
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  const int l = lane_id(), G = l >> 4, lc = l & 15;
  const int wi = w >> 1, wj = w & 1;

  const char* Pb = P + b * p_bs + (int64_t)ti * MS_TILE * p_ld * 4;
  const char* Qb = NN ? Q + b * q_bs + (int64_t)tj * MS_TILE * 4 : Q + b * q_bs + (int64_t)tj * MS_TILE * q_ld * 4;
  const int64_t q_step = NN ? (int64_t)MS_KB * q_ld * 4 : MS_KB * 4;  // bytes per contraction block

  // DMA: copy k of thread (w, l) fills LDS slot s = 256 k + 64 w + l and
  // fetches the piece stored there.
  uint32_t poff[Lp::NOPS], qoff[Lp::NOPS];
#pragma unroll
  for (int k = 0; k < Lp::NOPS; ++k) {
    const int s = k * MS_THREADS + w * 64 + l;
    {
      const int r = s >> 3, q = (s & 7) ^ (r & 7);
      poff[k] = (uint32_t)((r * p_ld + 4 * q) * 4);
    }
    if constexpr (NN) {
      const int kk = s >> 5, q = (s & 31) ^ ((kk & 3) << 2);
      qoff[k] = (uint32_t)((kk * q_ld + 4 * q) * 4);
    } else {
      const int r = s >> 3, q = (s & 7) ^ (r & 7);
      qoff[k] = (uint32_t)((r * q_ld + 4 * q) * 4);
    }
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)L0;
  auto issue = [&](int kb, int stage) {
    const char* pb = Pb + (int64_t)kb * MS_KB * 4;
    const char* qb = Qb + (int64_t)kb * q_step;
    const uint32_t st = lds0 + stage * Lp::STAGE + w * 64 * 16;
#pragma unroll
    for (int k = 0; k < Lp::NOPS; ++k) lds_dma16_s(pb, poff[k], st + k * MS_THREADS * 16);
#pragma unroll
    for (int k = 0; k < Lp::NOPS; ++k) lds_dma16_s(qb, qoff[k], st + Lp::OPB + k * MS_THREADS * 16);
  };

  // per-lane LDS byte offsets of the operand reads (within a stage)
  uint32_t pr[4][2], qr[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int r = 64 * wi + 16 * u + lc;
    pr[u][0] = (uint32_t)((8 * r + (G ^ (r & 7))) * 16);
    pr[u][1] = (uint32_t)((8 * r + ((4 + G) ^ (r & 7))) * 16);
    if constexpr (NN) {
      // transposing reads: lane (lc, G) addresses row 4G + lc/4 (+16) and
      // piece 16 wj + 4u + lc%4; hi at byte 0 of the piece, lo at byte 8
      const int q = 16 * wj + 4 * u + (lc & 3);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kk = 16 * h + 4 * G + (lc >> 2);
        qr[u][h] = (uint32_t)(Lp::OPB + (32 * kk + (q ^ ((kk & 3) << 2))) * 16);
      }
    } else {
      const int rq = 64 * wj + 16 * u + lc;
      qr[u][0] = (uint32_t)(Lp::OPB + (8 * rq + (G ^ (rq & 7))) * 16);
      qr[u][1] = (uint32_t)(Lp::OPB + (8 * rq + ((4 + G) ^ (rq & 7))) * 16);
    }
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int v = 0; v < 4; ++v) acc[u][v] = zero4();

  // blocks are copied MS_STAGES - 1 ahead; block kb + MS_STAGES - 1 reuses
  // the stage of block kb - 1
  constexpr int AHEAD = MS_STAGES - 1;
  static_assert(AHEAD == 1 || AHEAD == 2, "ring of 2 or 3 stages");
  const int nkb = K / MS_KB;
#pragma unroll
  for (int s = 0; s < AHEAD; ++s)
    if (s < nkb) issue(s, s);
  for (int kb = 0; kb < nkb; ++kb) {
    const int stage = kb % MS_STAGES;
    if (AHEAD == 2 && kb + 1 < nkb)
      wait_vmem_le<2 * Lp::NOPS>();  // this wave's copies of block kb landed; kb+1's may still fly
    else
      wait_vmem();
    __syncthreads();  // every wave's copies of block kb visible; block kb-1's stage free
    if (kb + AHEAD < nkb) issue(kb + AHEAD, (kb + AHEAD) % MS_STAGES);
    const lds_cptr Ls = L0 + stage * Lp::STAGE;
    PieceOp po[4], qo[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) po[u] = row_op(Ls + pr[u][0], Ls + pr[u][1]);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if constexpr (NN) {
        qo[v].hi = cat8(lds_tr16(Ls + qr[v][0]), lds_tr16(Ls + qr[v][1]));
        qo[v].lo = cat8(lds_tr16(Ls + (qr[v][0] + 8)), lds_tr16(Ls + (qr[v][1] + 8)));
      } else {
        qo[v] = row_op(Ls + qr[v][0], Ls + qr[v][1]);
      }
    }
    // swapped operands: A = Q^T rows (output columns), B = P^T columns
    // (output rows); lane (lc, G) accumulates row 16u + lc, columns
    // 16v + 4G .. +3
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[u][v] = mma3(qo[v], po[u], acc[u][v]);
  }

  // epilogue: one 16-byte piece per lane and tile
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t i = (int64_t)ti * MS_TILE + 64 * wi + 16 * u + lc;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t j = (int64_t)tj * MS_TILE + 64 * wj + 16 * v + 4 * G;
      const int64_t off = b * c_bs + (i * c_ld + j) * 4;
      f32x4 r = acc[u][v];
      if constexpr (EPI) {
        const f32x4 d = unsplit_piece(*reinterpret_cast<const bf16x8*>(Dm + off));
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = alpha * r[e] + beta * d[e];
      }
      *reinterpret_cast<bf16x8*>(Cm + off) = split_piece(r);
      acc[u][v] = r;
    }
  }
  if constexpr (SYM) {
    // the mirror tile (tj, ti): each wave transposes its 64 x 64 block
    // through its own LDS rows, T[j][i] at word 68 j + i
    if (ti != tj) {
      __syncthreads();  // every wave is done with the ring
      const lds_ptr Tw = L0 + w * Lp::MIRROR;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            lds_st<float>(Tw + ((16 * v + 4 * G + e) * Lp::MIRROR_LD + 16 * u + lc) * 4, acc[u][v][e]);
      __syncthreads();
      const int i4 = l & 15, jj = l >> 4;
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        const int j = 4 * it + jj;
        const f32x4 r = lds_ld<f32x4>(Tw + (j * Lp::MIRROR_LD + 4 * i4) * 4);
        const int64_t row = (int64_t)tj * MS_TILE + 64 * wj + j, col = (int64_t)ti * MS_TILE + 64 * wi + 4 * i4;
        *reinterpret_cast<bf16x8*>(Cm + b * c_bs + (row * c_ld + col) * 4) = split_piece(r);
      }
    }
  }
}

struct MsPlan {
  int64_t m, n, mp, np;
  size_t x_bytes, a_bytes, part_off, total;  // per-batch sizes and section layout
};

bool plan(int64_t batch, int64_t rows, int64_t cols, MsPlan& p) {
  if (batch <= 0 || rows <= 0 || cols <= 0 || rows > MS_MAXDIM || cols > MS_MAXDIM) return false;
  p.m = rows < cols ? rows : cols;
  p.n = rows < cols ? cols : rows;
  p.mp = round_up(p.m, MS_TILE);
  p.np = round_up(p.n, MS_TILE);
  p.x_bytes = (size_t)(p.mp * p.np * 4);
  p.a_bytes = (size_t)(p.mp * p.mp * 4);
  // sections: X0, X1 (batch x x_bytes each), A, Bm (batch x a_bytes each), norm partials
  const size_t xs = (size_t)round_up((int64_t)(batch * p.x_bytes), 256);
  const size_t as = (size_t)round_up((int64_t)(batch * p.a_bytes), 256);
  p.part_off = 2 * xs + 2 * as;
  p.total = p.part_off + (size_t)round_up(batch * MS_NPART * 4, 256);
  return true;
}

template <bool NN, bool EPI, bool SYM = false>
hipError_t launch_gemm(const char* P, const char* Q, const char* D, char* C, int64_t batch, int64_t p_bs,
                       int64_t q_bs, int64_t c_bs, int p_ld, int q_ld, int c_ld, int M, int N, int K, float alpha,
                       float beta, hipStream_t st) {
  auto kern = ns_gemm<NN, EPI, SYM>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, MsLds::BYTES);
  if (e != hipSuccess) return e;
  const int mt = M / MS_TILE, nt = N / MS_TILE;
  const int64_t tiles = SYM ? (int64_t)mt * (mt + 1) / 2 : (int64_t)mt * nt;
  hipLaunchKernelGGL(kern, dim3((unsigned)(batch * tiles)), dim3(MS_THREADS), MsLds::BYTES, st, P, Q, D, C, p_bs,
                     q_bs, c_bs, p_ld, q_ld, c_ld, mt, nt, K, alpha, beta);
  return hipGetLastError();
}

template <typename T>
hipError_t run_msign(const T* M, T* out, int64_t batch, int64_t rows, int64_t cols, int steps, float eps,
                     char* ws, const MsPlan& p, hipStream_t st) {
  const bool tr = rows > cols;
  const int64_t xs = (int64_t)round_up((int64_t)(batch * p.x_bytes), 256);
  const int64_t as = (int64_t)round_up((int64_t)(batch * p.a_bytes), 256);
  char* X[2] = {ws, ws + xs};
  char* A = ws + 2 * xs;
  char* Bm = A + as;
  float* part = reinterpret_cast<float*>(ws + p.part_off);
  const int64_t xb = (int64_t)p.x_bytes, ab = (int64_t)p.a_bytes;
  const int mp = (int)p.mp, np = (int)p.np;

  const bool vec = (rows * cols) % 4 == 0 && ((uintptr_t)M % (4 * sizeof(T))) == 0;
  if (vec)
    hipLaunchKernelGGL((ns_norm_partial<T, true>), dim3(MS_NPART, (unsigned)batch), dim3(256), 0, st, M, part,
                       rows * cols);
  else
    hipLaunchKernelGGL((ns_norm_partial<T, false>), dim3(MS_NPART, (unsigned)batch), dim3(256), 0, st, M, part,
                       rows * cols);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (tr) {
    const unsigned blocks = (unsigned)((p.mp / 64) * (p.np / 64));
    hipLaunchKernelGGL(ns_pack_tr<T>, dim3(blocks, (unsigned)batch), dim3(256), 0, st, M, part, X[0], xb, (int)p.m,
                       (int)p.n, mp, np, eps);
  } else {
    const unsigned blocks = (unsigned)((p.mp * (p.np / 4) + 255) / 256);
    if (vec && cols % 4 == 0)
      hipLaunchKernelGGL((ns_pack<T, true>), dim3(blocks, (unsigned)batch), dim3(256), 0, st, M, part, X[0], xb,
                         (int)p.m, (int)p.n, mp, np, eps);
    else
      hipLaunchKernelGGL((ns_pack<T, false>), dim3(blocks, (unsigned)batch), dim3(256), 0, st, M, part, X[0], xb,
                         (int)p.m, (int)p.n, mp, np, eps);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  int cur = 0;
  for (int s = 0; s < steps; ++s) {
    // A = X X^T
    e = launch_gemm<false, false, true>(X[cur], X[cur], nullptr, A, batch, xb, xb, ab, np, np, mp, mp, mp, np, 1.f, 0.f,
                                  st);
    if (e != hipSuccess) return e;
    // Bm = b A + c A A
    e = launch_gemm<false, true, true>(A, A, A, Bm, batch, ab, ab, ab, mp, mp, mp, mp, mp, mp, NS_C, NS_B, st);
    if (e != hipSuccess) return e;
    // X' = a X + Bm X
    e = launch_gemm<true, true>(Bm, X[cur], X[cur], X[cur ^ 1], batch, ab, xb, xb, mp, np, np, mp, np, mp, 1.f,
                                NS_A, st);
    if (e != hipSuccess) return e;
    cur ^= 1;
  }
  if (tr) {
    const unsigned blocks = (unsigned)((p.mp / 64) * (p.np / 64));
    hipLaunchKernelGGL(ns_unpack_tr<T>, dim3(blocks, (unsigned)batch), dim3(256), 0, st, X[cur], out, xb, (int)rows,
                       (int)cols, mp, np);
  } else {
    const unsigned blocks = (unsigned)((rows * cols + 255) / 256);
    hipLaunchKernelGGL(ns_unpack<T>, dim3(blocks, (unsigned)batch), dim3(256), 0, st, X[cur], out, xb, (int)rows,
                       (int)cols, np);
  }
  return hipGetLastError();
}

}  // namespace
}  // namespace gmdn

using namespace gmdn;

extern "C" {

size_t gmdn_msign_workspace_bytes(int64_t batch, int64_t rows, int64_t cols) {
  MsPlan p;
  return plan(batch, rows, cols, p) ? p.total : 0;
}

int gmdn_msign(const void* M, void* out, int64_t batch, int64_t rows, int64_t cols, int32_t steps, float eps,
               int32_t dtype, void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || rows < 0 || cols < 0 || steps < 0 || steps > 64) return GMDN_ERR_ARG;
  if (dtype != GMDN_DTYPE_F32 && dtype != GMDN_DTYPE_BF16) return GMDN_ERR_UNSUPPORTED;
  if (rows > MS_MAXDIM || cols > MS_MAXDIM) return GMDN_ERR_UNSUPPORTED;
  if (!(eps >= 0.f)) return GMDN_ERR_ARG;
  if (batch == 0 || rows == 0 || cols == 0) return GMDN_OK;
  if (batch > 65535) return GMDN_ERR_ARG;  // the batch is the grid's y dimension
  if (!M || !out) return GMDN_ERR_ARG;
  MsPlan p;
  if (!plan(batch, rows, cols, p)) return GMDN_ERR_ARG;
  if (!workspace || workspace_bytes < p.total || ((uintptr_t)workspace & 255)) return GMDN_ERR_WORKSPACE;
  const int64_t tiles = batch * (p.mp / MS_TILE) * (p.np / MS_TILE);
  if (tiles > ((int64_t)1 << 31) - 1) return GMDN_ERR_ARG;
  const hipStream_t st = (hipStream_t)stream;
  char* ws = static_cast<char*>(workspace);
  hipError_t e;
  if (dtype == GMDN_DTYPE_F32)
    e = run_msign<float>(static_cast<const float*>(M), static_cast<float*>(out), batch, rows, cols, steps, eps, ws,
                         p, st);
  else
    e = run_msign<bf16>(static_cast<const bf16*>(M), static_cast<bf16*>(out), batch, rows, cols, steps, eps, ws, p,
                        st);
  return e == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

}  // extern "C"
