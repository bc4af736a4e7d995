// Level B backward, delta rule: token gradients of chunk pairs.
//
// The forward keeps the state checkpoint S_i of the even chunks only, and
// the reverse scan (chunk_bwd_dscan) writes the state cotangent
// Gb_i = Sb_{i+1} of the odd chunks only: half of the checkpoint's HBM
// writes and reads and of Gb's.  One workgroup per (b, h, pair i0 = 2p,
// i1 = 2p + 1) rebuilds what it lacks on chip:
//   S_{i1} = a_{i0} S_{i0} + E_{i0}^T diag(beta) K_{i0}       (forward step)
//   Gb_{i0} = Sb_{i1} = a_{i1} Gb_{i1} + dO^T Q - dE^T K      (reverse step,
//             from chunk i1's own dE, formed while its gradients are)
// and forms the gradients of chunk i1, then of chunk i0, each exactly as the
// per-chunk kernel does (reference train_ablation.py:142-187 differentiated
// through fast_scan.py:72-95): with A = tril(Q K^T) diag(beta),
// E = V - K S^T,
//   dE = A^T dO + diag(beta) K Gb^T,  dA = tril(dO E^T),
//   dQ = dO S + (dA diag(beta)) K,  dK = (dA diag(beta))^T Q - dE S + diag(beta) E Gb,
//   dV = dE,  dbeta, dg from the A terms, (E Gb) k and <Gb, S> a.
// State rows stay in registers as split pieces (16 bytes = hi, lo of four
// consecutive columns); a pair with no odd partner (N odd) has Gb = 0.
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

namespace gmdn {

template <int D>
struct PairLds {
  static constexpr int NW = D / 16;
  static constexpr int NTHR = 64 * NW;
  static constexpr int TILE = CB_C * D * 2;
  static constexpr int Q0 = 0, K0 = TILE, V0 = 2 * TILE, O0 = 3 * TILE;
  static constexpr int EH0 = 4 * TILE, EL0 = 5 * TILE;    // E (rows s, columns r), hi / lo
  static constexpr int DH0 = 6 * TILE, DL0 = 7 * TILE;    // dE
  static constexpr int AP = CB_C * CB_C * 2;
  static constexpr int AH0 = 8 * TILE, AL0 = AH0 + AP;    // A^T, then dA diag(beta) (rows s)
  // floats: per-wave dbeta partials [NW][64], two gate slots {beta, g}
  // (chunk i0's stays published while chunk i1's is in use), per-wave da
  // partials [NW]
  static constexpr int R0 = AL0 + AP;
  static constexpr int BYTES = R0 + (NW * CB_C + 4 * CB_C + NW) * 4;
  static_assert(BYTES <= 160 * 1024, "pair backward LDS exceeds the 160 KiB of a CU");
};

template <int D>
struct PairCtx {
  static constexpr int NKB = D / 32;
  using LQ = PairSwz<D>;
  using LA = PairSwz<CB_C>;
  using L = PairLds<D>;
  char* smem;
  const ChunkArgs* p;
  int64_t bh, bb, hh;
  int w, l, G, lc, r0;
  int gs = 0;  // the gate slot in use

  GMDN_DEV const bf16* Qs() const { return reinterpret_cast<const bf16*>(smem + L::Q0); }
  GMDN_DEV const bf16* Ks() const { return reinterpret_cast<const bf16*>(smem + L::K0); }
  GMDN_DEV const bf16* Vs() const { return reinterpret_cast<const bf16*>(smem + L::V0); }
  GMDN_DEV const bf16* Os() const { return reinterpret_cast<const bf16*>(smem + L::O0); }
  GMDN_DEV bf16* Eh() const { return reinterpret_cast<bf16*>(smem + L::EH0); }
  GMDN_DEV bf16* El() const { return reinterpret_cast<bf16*>(smem + L::EL0); }
  GMDN_DEV bf16* Dh() const { return reinterpret_cast<bf16*>(smem + L::DH0); }
  GMDN_DEV bf16* Dl() const { return reinterpret_cast<bf16*>(smem + L::DL0); }
  GMDN_DEV bf16* Ah() const { return reinterpret_cast<bf16*>(smem + L::AH0); }
  GMDN_DEV bf16* Al() const { return reinterpret_cast<bf16*>(smem + L::AL0); }
  // dbeta and da are summed per wave into the wave's own slots, then over
  // the waves in a fixed order: the gradients are bitwise reproducible
  GMDN_DEV float* pdbeta() const { return reinterpret_cast<float*>(smem + L::R0); }  // [NW][64]
  GMDN_DEV float* rbeta() const { return pdbeta() + L::NW * CB_C + gs * 2 * CB_C; }
  GMDN_DEV float* rg() const { return rbeta() + CB_C; }
  GMDN_DEV float* pda() const { return pdbeta() + L::NW * CB_C + 4 * CB_C; }  // [NW]

  // Chunk i's gate rows {beta, g} into gate slot `slot` by one LDS-DMA
  // operation of wave 0 (lanes 0-15 beta, 16-31 g; the caller waits and
  // synchronises).  No register holds them, so the compiler places no wait
  // of its own for them (such a wait drains every copy in flight).
  GMDN_DEV void dma_gates(int i, int slot) const {
    if (w == 0 && l < 32) {
      const float* src = (G == 0 ? p->beta : p->g) + bh * p->T + (int64_t)i * CB_C + 4 * lc;
      lds_dma16(src, smem + L::R0 + (L::NW * CB_C + slot * 2 * CB_C) * 4);
    }
  }
  // Asynchronous copy of one of chunk i's token tiles (rows of `x`, row
  // stride `sx`) into the LDS tile at byte offset `dst` (2 operations per wave)
  GMDN_DEV void issue_tile(const bf16* x, const int64_t (&sx)[3], int i, int dst) const {
    // the plan's lane offsets are recomputed at every copy (a few VALU
    // operations) rather than held live across the kernel: held, they spill,
    // and every reload of a spilled offset waits for all vector memory
    int wv = w;
    asm volatile("" : "+s"(wv));
    DmaPlan<LQ, CB_C, L::NTHR> pl;
    pl.init(wv, sx[2]);
    pl.issue(x + bb * sx[0] + hh * sx[1] + (int64_t)i * CB_C * sx[2], lds_addr(smem) + dst, w);
  }
  // a = exp(sum over the chunk of max(g, log 1e-6)) (every lane)
  GMDN_DEV float chunk_decay() const { return expf(wave_sum(fmaxf(rg()[l], LOG_FLOOR))); }

  // E^T tiles of the wave's 16 state rows: lane (s, G) of tile st holds
  // E^T[r0 + 4G + jj][16 st + s], from the split operands Sa of the rows
  GMDN_DEV void e_tiles(const Op<2> (&Sa)[NKB], const bf16* Kt, const bf16* Vt, f32x4 (&Et)[4]) const {
    f32x4 Ets[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const bf16x4 vv = *reinterpret_cast<const bf16x4*>(Vt + LQ::off(16 * st + lc, r0 + 4 * G));
      Ets[st] = f32x4{-(float)vv[0], -(float)vv[1], -(float)vv[2], -(float)vv[3]};
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int st = 0; st < 4; ++st) Ets[st] = mma<2, 1>(Sa[kb], Op<1>{{row8<LQ>(Kt, 16 * st + lc, 32 * kb)}}, Ets[st]);
#pragma unroll
    for (int st = 0; st < 4; ++st) Et[st] = -Ets[st];
  }

  // the D-layout tile t of a [s][r] matrix -> split planes at (s = 16 st + lc, r = r0 + 4G ..)
  GMDN_DEV void put_sr(bf16* hi, bf16* lo, int st, const f32x4& t) const {
    bf16x4 h, o;
    split4(t, h, o);
    const int off = LQ::off(16 * st + lc, r0 + 4 * G);
    *reinterpret_cast<bf16x4*>(hi + off) = h;
    *reinterpret_cast<bf16x4*>(lo + off) = o;
  }

  // acc += (sign) sum_t X[t][c] Y[t][r] over the 64 tokens, in piece order:
  // acc[kb][u] lane (r, G) holds columns 32 kb + 8G + 4u .. +3 of row r0 + lc
  template <int PB, bool NEG>
  GMDN_DEV void rows_product(const bf16* X, const bf16* Yh, const bf16* Yl, f32x4 (&acc)[NKB][2]) const {
    Op<PB> Y[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      Y[kt].v[0] = col8<LQ>(Yh, 32 * kt, r0);
      if constexpr (PB == 2) Y[kt].v[1] = col8<LQ>(Yl, 32 * kt, r0);
    }
    // the X operands software-pipelined two ahead of their MFMAs (left to
    // itself the compiler waits for each read right before its MFMA)
    constexpr int NJ = NKB * 4, PIPE = 2;
    auto xop = [&](int j) { return col8p<LQ>(X, 32 * (j & 1), 32 * (j >> 2) + 4 * ((j >> 1) & 1)); };
    bf16x8 xs[PIPE];
#pragma unroll
    for (int j = 0; j < PIPE; ++j) xs[j] = xop(j);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      bf16x8 x = xs[j % PIPE];
      if (j + PIPE < NJ) xs[j % PIPE] = xop(j + PIPE);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (NEG) x = neg8(x);
      const int kb = j >> 2, u = (j >> 1) & 1, kt = j & 1;
      acc[kb][u] = mma<1, PB>(Op<1>{{x}}, Y[kt], acc[kb][u]);
    }
  }

  // The gradients of chunk i, whose q, k tiles and gates are in LDS (the v,
  // dO tiles and the state rows may still be arriving: they are waited for
  // after phase I'), given its state rows S (pieces) and Gb (pieces).  With
  // want_sb, also Sb_i = a_i Gb + dO^T Q - dE^T K (pieces) into sb.
  // `rows_free()` runs once every wave has staged its S and Gb rows for
  // phase IIb (srow and grow are not read after it), two blocks before
  // the end of its products; `qk_free()` once the q and k tiles (phase IIb's
  // first staging buffer) are read for the last time, before the last
  // block's products; `next()` once the dO tile is free, after the dq, dk
  // stores are issued.  The V tile and the A planes stay in use until the
  // return.
  template <class RowsFree, class QkFree, class Next>
  GMDN_DEV void chunk_grads(int i, const bf16x8 (&srow)[NKB][2], const bf16x8 (&grow)[NKB][2], bool want_sb,
                            bf16x8 (&sb)[NKB][2], RowsFree&& rows_free, QkFree&& qk_free, Next&& next) const {
    const int64_t t0 = (int64_t)i * CB_C;
    const bf16* Qs_ = Qs();
    const bf16* Ks_ = Ks();
    const bf16* Os_ = Os();
    bf16* Eh_ = Eh();
    bf16* El_ = El();
    bf16* Dh_ = Dh();
    bf16* Dl_ = Dl();
    bf16* Ah_ = Ah();
    bf16* Al_ = Al();
    float* pdb = pdbeta() + w * CB_C;  // this wave's dbeta slots
    const float* rbeta_ = rbeta();
    constexpr int NW = L::NW;
    static_assert(NW % 4 == 0, "a wave's phase IIa tiles share one token tile");

    // ---- A^T = (tril(Q K^T) diag(beta))^T split into the A planes (rows s)
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
          X = mfma(row8<LQ>(Qs_, 16 * tt + lc, 32 * kb), row8<LQ>(Ks_, 16 * st + lc, 32 * kb), X);
        const float bs = rbeta_[16 * st + lc];
        f32x4 xv;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) xv[jj] = (tt > st || 4 * G + jj >= lc) ? X[jj] * bs : 0.f;
        split4(xv, ah, al);
      }
      const int ao = LA::off(16 * st + lc, 16 * tt + 4 * G);
      *reinterpret_cast<bf16x4*>(Ah_ + ao) = ah;
      *reinterpret_cast<bf16x4*>(Al_ + ao) = al;
    }
    wait_vmem();
    __syncthreads();  // the A planes published, every tile landed

    // ---- E^T, (Gb K^T) and dE^T for this wave's 16 state rows
    Op<2> Sa[NKB], Ga[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      Sa[kb] = join_pieces(srow[kb][0], srow[kb][1]);
      Ga[kb] = join_pieces(grow[kb][0], grow[kb][1]);
    }
    {
      float dbp[4];
      f32x4 Et[4], GKs[4];
      e_tiles(Sa, Ks_, Vs(), Et);
#pragma unroll
      for (int st = 0; st < 4; ++st) GKs[st] = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int st = 0; st < 4; ++st) GKs[st] = mma<2, 1>(Ga[kb], Op<1>{{row8<LQ>(Ks_, 16 * st + lc, 32 * kb)}}, GKs[st]);
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const f32x4 GK = GKs[st];
        dbp[st] = dot4(Et[st], GK);
        f32x4 dEt = GK * rbeta_[16 * st + lc];
#pragma unroll
        for (int kbt = 0; kbt < 2; ++kbt) {
          if (32 * kbt + 31 < 16 * st) continue;
          const Op<1> dOt{{col8<LQ>(Os_, 32 * kbt, r0)}};
          const Op<2> At{{row8<LA>(Ah_, 16 * st + lc, 32 * kbt), row8<LA>(Al_, 16 * st + lc, 32 * kbt)}};
          dEt = mma<1, 2>(dOt, At, dEt);
        }
        put_sr(Eh_, El_, st, Et[st]);
        put_sr(Dh_, Dl_, st, dEt);
      }
#pragma unroll
      for (int st = 0; st < 4; ++st) dbp[st] = group_sum(dbp[st]);
      if (G == 0) {
#pragma unroll
        for (int st = 0; st < 4; ++st) pdb[16 * st + lc] = dbp[st];  // every token slot
      }
      // da_i = <Gb, S>: the trace of the wave's diagonal block of Gb S^T
      f32x4 T = zero4();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) T = mma<2, 2>(Ga[kb], Sa[kb], T);
      const float dpart = (lc >> 2) == G ? T[lc & 3] : 0.f;
      const float da_w = wave_sum(dpart);
      if (l == 0) pda()[w] = da_w;
    }
    __syncthreads();

    // ---- Sb_i = a_i Gb + dO^T Q - dE^T K for the other chunk of the pair
    if (want_sb) {
      f32x4 acc[NKB][2];
      const float a = chunk_decay();
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) acc[kb][u] = a * unsplit_piece(grow[kb][u]);
      rows_product<1, false>(Qs_, Os_, Os_, acc);
      rows_product<2, true>(Ks_, Dh_, Dl_, acc);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int u = 0; u < 2; ++u) sb[kb][u] = split_piece(acc[kb][u]);
    }

    // ---- dA = tril(dO E^T), dbeta's A term, dA diag(beta) -> the A planes
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
          const Op<1> dOr{{row8<LQ>(Os_, 16 * tt + lc, 32 * kb)}};
          const Op<2> Er{{row8<LQ>(Eh_, 16 * st + lc, 32 * kb), row8<LQ>(El_, 16 * st + lc, 32 * kb)}};
          P = mma<1, 2>(dOr, Er, P);
          QK = mfma(row8<LQ>(Qs_, 16 * tt + lc, 32 * kb), row8<LQ>(Ks_, 16 * st + lc, 32 * kb), QK);
        }
        const float bs = rbeta_[16 * st + lc];
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
      *reinterpret_cast<bf16x4*>(Ah_ + ao) = ah;
      *reinterpret_cast<bf16x4*>(Al_ + ao) = al;
    }
    {
      // the wave's tiles k = w + NW kk all have st = w % 4
      float db = 0.f;
#pragma unroll
      for (int kk = 0; kk < 16 / NW; ++kk) {
        const int k = w + NW * kk, tt = k >> 2, st = k & 3;
        const float v = group_sum(dbk[kk]);
        if (tt >= st) db += v;
      }
      if (G == 0) pdb[16 * (w & 3) + lc] += db;
    }
    __syncthreads();

    // ---- gate gradients and dV
    if (w == 0) {
      const int64_t o = bh * p->T + t0 + l;
      const float a = chunk_decay();
      float db = 0.f, da = 0.f;
#pragma unroll
      for (int q = 0; q < NW; ++q) {
        db += pdbeta()[q * CB_C + l];
        da += pda()[q];
      }
      p->dbeta[o] = db;
      p->dg[o] = rg()[l] >= LOG_FLOOR ? da * a : 0.f;
    }
    {
      bf16* dvg = p->dv + bb * p->sv[0] + hh * p->sv[1] + t0 * p->sv[2];
      for (int e = threadIdx.x; e < CB_C * D / 8; e += L::NTHR) {
        const int r = e / (D / 8), c8 = (e % (D / 8)) * 8;
        *reinterpret_cast<bf16x8*>(dvg + r * p->sv[2] + c8) = *reinterpret_cast<const bf16x8*>(Dh_ + LQ::off(r, c8));
      }
    }

    // ---- dQ and dK for this wave's two state-column tiles 2 cp, 2 cp + 1
    // and two token tiles 2 th, 2 th + 1 (operands swapped: lane <-> token,
    // registers <-> 4 consecutive state columns).  Per 32-row block a wave
    // reads 18 KiB of operands, where one column tile by four token tiles
    // would read 24 KiB for the same products.
    constexpr int NCP = NW / 2;
    const int cp = w % NCP, th = w / NCP;
    const int jb = 32 * cp;
    bf16* dqg = p->dq + bb * p->sq[0] + hh * p->sq[1] + t0 * p->sq[2];
    bf16* dkg = p->dk + bb * p->sk[0] + hh * p->sk[1] + t0 * p->sk[2];
    f32x4 dqa[2][2], dka[2][2], des[2][2], eg[2][2];  // [column tile][token tile]
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      const int tt = 2 * th + ti;
#pragma unroll
      for (int ci = 0; ci < 2; ++ci) dqa[ci][ti] = zero4();
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        if (32 * ks > 16 * tt + 15) continue;
        const Op<2> dA{{col8<LA>(Ah_, 32 * ks, 16 * tt), col8<LA>(Al_, 32 * ks, 16 * tt)}};
#pragma unroll
        for (int ci = 0; ci < 2; ++ci)
          dqa[ci][ti] = mma<1, 2>(Op<1>{{col8<LQ>(Ks_, 32 * ks, jb + 16 * ci)}}, dA, dqa[ci][ti]);
      }
    }
#pragma unroll
    for (int si = 0; si < 2; ++si) {
      const int st = 2 * th + si;
#pragma unroll
      for (int ci = 0; ci < 2; ++ci) dka[ci][si] = des[ci][si] = eg[ci][si] = zero4();
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        if (32 * kt + 31 < 16 * st) continue;
        const Op<2> dAT{{row8<LA>(Ah_, 16 * st + lc, 32 * kt), row8<LA>(Al_, 16 * st + lc, 32 * kt)}};
#pragma unroll
        for (int ci = 0; ci < 2; ++ci)
          dka[ci][si] = mma<1, 2>(Op<1>{{col8<LQ>(Qs_, 32 * kt, jb + 16 * ci)}}, dAT, dka[ci][si]);
      }
    }
    // S and Gb by columns: the rows pass through free tiles one 32-row block
    // at a time as split planes, double-buffered (the Q and K tiles; the V
    // tile, free since phase I, and the A planes, free since dQ, dK's first
    // products): block kb + 1 is written while block kb is read
    bf16* const Sbuf[2] = {reinterpret_cast<bf16*>(smem + L::Q0), reinterpret_cast<bf16*>(smem + L::V0)};
    bf16* const Gbuf[2] = {reinterpret_cast<bf16*>(smem + L::K0), Ah_};
    auto put_rows = [&](int kb) {
      if ((w >> 1) == kb) {
        bf16* Sh = Sbuf[kb & 1];
        bf16* Sl = Sh + 32 * D;
        bf16* Gh = Gbuf[kb & 1];
        bf16* Gl = Gh + 32 * D;
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
    };
    __syncthreads();  // Q and K tiles free
    put_rows(0);
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      if (kb + 1 == NKB) qk_free();  // block NKB - 2 (buffer 0) read by every wave
      if (kb + 1 < NKB) put_rows(kb + 1);
      if (kb + 2 == NKB) rows_free();  // every wave's rows staged
      const bf16* Sh = Sbuf[kb & 1];
      const bf16* Sl = Sh + 32 * D;
      const bf16* Gh = Gbuf[kb & 1];
      const bf16* Gl = Gh + 32 * D;
      Op<2> sc[2], gc[2];
#pragma unroll
      for (int ci = 0; ci < 2; ++ci) {
        sc[ci] = Op<2>{{col8<LQ>(Sh, 0, jb + 16 * ci), col8<LQ>(Sl, 0, jb + 16 * ci)}};
        gc[ci] = Op<2>{{col8<LQ>(Gh, 0, jb + 16 * ci), col8<LQ>(Gl, 0, jb + 16 * ci)}};
      }
#pragma unroll
      for (int ti = 0; ti < 2; ++ti) {
        const Op<1> Or{{row8<LQ>(Os_, 16 * (2 * th + ti) + lc, 32 * kb)}};
#pragma unroll
        for (int ci = 0; ci < 2; ++ci) dqa[ci][ti] = mma<2, 1>(sc[ci], Or, dqa[ci][ti]);
      }
#pragma unroll
      for (int si = 0; si < 2; ++si) {
        const int st = 2 * th + si;
        const Op<2> Er{{row8<LQ>(Eh_, 16 * st + lc, 32 * kb), row8<LQ>(El_, 16 * st + lc, 32 * kb)}};
        const Op<2> Dr{{row8<LQ>(Dh_, 16 * st + lc, 32 * kb), row8<LQ>(Dl_, 16 * st + lc, 32 * kb)}};
#pragma unroll
        for (int ci = 0; ci < 2; ++ci) {
          eg[ci][si] = mma<2, 2>(gc[ci], Er, eg[ci][si]);
          des[ci][si] = mma<2, 2>(sc[ci], Dr, des[ci][si]);
        }
      }
      __syncthreads();  // block kb read, block kb + 1 written
    }
    bf16* dqs = reinterpret_cast<bf16*>(smem + L::V0);
    bf16* dks = Ah_;
#pragma unroll
    for (int ti = 0; ti < 2; ++ti) {
      const int t = 16 * (2 * th + ti) + lc;
      const float rb = rbeta_[t];
#pragma unroll
      for (int ci = 0; ci < 2; ++ci) {
        const int c = jb + 16 * ci + 4 * G;
        *reinterpret_cast<bf16x4*>(dqs + LQ::off(t, c)) = to_bf16x4(dqa[ci][ti]);
        const f32x4 acc = dka[ci][ti] - des[ci][ti] + eg[ci][ti] * rb;
        *reinterpret_cast<bf16x4*>(dks + LQ::off(t, c)) = to_bf16x4(acc);
      }
    }
    __syncthreads();
    // the stores go out before next()'s copies and loads: vector-memory
    // instructions leave a CU in issue order, so stores issued behind 100+
    // KiB of loads wait for them
    for (int e = threadIdx.x; e < CB_C * D / 8; e += L::NTHR) {
      const int r = e / (D / 8), c8 = (e % (D / 8)) * 8;
      *reinterpret_cast<bf16x8*>(dqg + r * p->sq[2] + c8) = *reinterpret_cast<const bf16x8*>(dqs + LQ::off(r, c8));
      *reinterpret_cast<bf16x8*>(dkg + r * p->sk[2] + c8) = *reinterpret_cast<const bf16x8*>(dks + LQ::off(r, c8));
    }
    next();
    __syncthreads();  // the staging tiles are read before the next chunk's copies land
  }

  // S_{i+1} rows = a_i S_i + E_i^T diag(beta) K_i (pieces), for the wave's
  // rows, from chunk i's k and v tiles at Kt, Vt and its gates in LDS
  GMDN_DEV void state_step(const bf16* Kt, const bf16* Vt, const bf16x8 (&srow)[NKB][2],
                           bf16x8 (&snext)[NKB][2]) const {
    Op<2> Sa[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) Sa[kb] = join_pieces(srow[kb][0], srow[kb][1]);
    f32x4 Et[4];
    e_tiles(Sa, Kt, Vt, Et);
    const float* rbeta_ = rbeta();
    // beta E into the E planes as [s][r]
#pragma unroll
    for (int st = 0; st < 4; ++st) put_sr(Eh(), El(), st, Et[st] * rbeta_[16 * st + lc]);
    __syncthreads();
    f32x4 acc[NKB][2];
    const float a = chunk_decay();
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) acc[kb][u] = a * unsplit_piece(srow[kb][u]);
    rows_product<2, false>(Kt, Eh(), El(), acc);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int u = 0; u < 2; ++u) snext[kb][u] = split_piece(acc[kb][u]);
    __syncthreads();  // the k, v tiles and the E planes are read before they are reused
  }
};

// Marks register pieces as used: the compiler completes their loads here.
template <int NKB>
GMDN_DEV void held(const bf16x8 (&x)[NKB][2]) {
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
    for (int u = 0; u < 2; ++u) asm volatile("" ::"v"(x[kb][u]));
}

template <int D>
__global__ void __launch_bounds__(PairLds<D>::NTHR) chunk_bwd_pair(ChunkArgs p) {
  constexpr int NKB = D / 32;
  extern __shared__ __align__(16) char smem[];
  const int NP = (p.N + 1) / 2, NO = p.N / 2;
  PairCtx<D> c;
  c.smem = smem;
  c.p = &p;
  c.bh = blockIdx.x / NP;
  const int pi = (int)(blockIdx.x % NP);
  c.bb = c.bh / p.H;
  c.hh = c.bh % p.H;
  c.w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  c.l = lane_id();
  c.G = c.l >> 4;
  c.lc = c.l & 15;
  c.r0 = 16 * c.w;
  const int i0 = 2 * pi, i1 = i0 + 1;

  // rows r0 + lc of a d x d plane, as split pieces (columns 32 kb + 8G ..)
  auto load_rows = [&](const float* plane, bf16x8(&rows)[NKB][2]) {
    const float* r = plane + (c.r0 + c.lc) * (int64_t)D + 8 * c.G;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      rows[kb][0] = *reinterpret_cast<const bf16x8*>(r + 32 * kb);
      rows[kb][1] = *reinterpret_cast<const bf16x8*>(r + 32 * kb + 4);
    }
  };
  using L = PairLds<D>;
  const float* S0 = p.states + (c.bh * NP + pi) * (int64_t)D * D;  // S_{i0}: even checkpoint pi
  bf16x8 sr[NKB][2], gr[NKB][2], gn[NKB][2];
  c.dma_gates(i0, 0);
  if (i1 < p.N) {
    // Vector-memory operations complete in issue order.  Chunk i0's k, v go
    // to the dE planes (free until chunk i1's phase I) for the state step,
    // then chunk i1's four tiles stream into their slots meanwhile.
    {
      bf16x8 s0[NKB][2];
      load_rows(S0, s0);
      c.issue_tile(p.k, p.sk, i0, L::DH0);
      c.issue_tile(p.v, p.sv, i0, L::DL0);
      wait_vmem();
      // the compiler's own wait for the S rows goes here, not after the
      // copies below (it does not count them): they stay in flight
      held(s0);
      __syncthreads();
      c.issue_tile(p.q, p.sq, i1, L::Q0);
      c.issue_tile(p.k, p.sk, i1, L::K0);
      c.issue_tile(p.v, p.sv, i1, L::V0);
      c.issue_tile(p.o, p.so, i1, L::O0);
      c.dma_gates(i1, 1);
      load_rows(p.gb + (c.bh * NO + pi) * (int64_t)D * D, gr);  // Gb_{i1}: odd plane pi
      c.state_step(reinterpret_cast<const bf16*>(smem + L::DH0), reinterpret_cast<const bf16*>(smem + L::DL0),
                   s0, sr);  // S_{i1}
    }
    wait_vmem_le<2 * NKB>();  // chunk i1's tiles and gates landed; the Gb rows may be in flight
    c.gs = 1;  // chunk i0's gates stay in slot 0
    __syncthreads();
    // chunk i1, and Gb_{i0} = Sb_{i1}.  Chunk i0's S rows are requested once
    // chunk i1's rows are staged for phase IIb (its last two blocks' products
    // run meanwhile), its q, k tiles before the last block's products, its
    // dO tile once chunk i1's dq, dk stores are issued.
    c.chunk_grads(
        i1, sr, gr, true, gn, [&] { load_rows(S0, sr); },
        [&] {
          c.issue_tile(p.q, p.sq, i0, L::Q0);
          c.issue_tile(p.k, p.sk, i0, L::K0);
        },
        [&] { c.issue_tile(p.o, p.so, i0, L::O0); });
    c.issue_tile(p.v, p.sv, i0, L::V0);
    // chunk i0's S rows and q, k, dO tiles landed (issued among them: the dq,
    // dk stores); in flight at most: the v tile
    wait_vmem_le<2>();
    c.gs = 0;
  } else {
    const bf16x8 z8 = bf16x8{(bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f, (bf16)0.f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) gn[kb][0] = gn[kb][1] = z8;  // the last chunk: Sb_N = 0
    c.issue_tile(p.q, p.sq, i0, L::Q0);
    c.issue_tile(p.k, p.sk, i0, L::K0);
    c.issue_tile(p.o, p.so, i0, L::O0);
    load_rows(S0, sr);
    c.issue_tile(p.v, p.sv, i0, L::V0);
    // (a lone last chunk: no overlap sought) the compiler's wait for the S
    // registers is placed here, where it is already met
    wait_vmem();
    held(sr);
  }
  __syncthreads();
  c.chunk_grads(i0, sr, gn, false, gr, [] {}, [] {}, [] {});
}

hipError_t chunk_bwd_pair_launch(const ChunkArgs& a, int d, hipStream_t s) {
  const int64_t grid = a.B * a.H * ((a.N + 1) / 2);
  if (d == 128) {
    auto k = chunk_bwd_pair<128>;
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, PairLds<128>::BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(PairLds<128>::NTHR), PairLds<128>::BYTES, s, a);
  } else {
    auto k = chunk_bwd_pair<64>;
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, PairLds<64>::BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(PairLds<64>::NTHR), PairLds<64>::BYTES, s, a);
  }
  return hipGetLastError();
}

}  // namespace gmdn
