// Wave64 MFMA tile primitives for gfx950 (CDNA4).
//
// Every product in the scan kernels is built from 16x16 output tiles of
// v_mfma_f32_16x16x32_bf16 (or v_mfma_f32_16x16x4_f32 for the exact-fp32
// mode).  Lane layouts, checked on MI355X hardware:
//
//   16x16x32 bf16   A: lane l holds A[l%16][8(l/16)+i], i=0..7
//                   B: lane l holds B[8(l/16)+i][l%16]
//                   D: lane l holds D[4(l/16)+j][l%16], j=0..3
//   16x16x4  f32    A: A[l%16][l/16]  B: B[l/16][l%16]  D as above
//
// "D layout": a 16x16 fp32 tile with lane <-> column (l%16) and the four
// accumulator registers <-> rows 4G+j (G = l/16).
//
// Chaining without a shuffle.  The contraction index of an MFMA may be
// permuted freely as long as both operands use the same permutation.  All
// 32-wide k-blocks here use the "pair order": lane group G holds the k
// indices {4G..4G+3} in slots 0..3 and {16+4G..16+4G+3} in slots 4..7.  Then
// two D-layout tiles stacked along k (rows 0..15 and 16..31) ARE an operand
// whose free index is the tile column: no LDS round trip is needed to feed
// one product's result into the next as the k side.  Operands read from
// memory use the same pair order (two 8-byte reads per lane, or two
// ds_read_b64_tr_b16 transposing reads for a k-major source).
//
// ds_read_b64_tr_b16 (checked on hardware): within each 16-lane group,
// output lane i element j is element i%4 of the 8-byte vector addressed by
// lane 4j+i/4.  So if lane (i, G) passes &X[r0 + i/4][c0 + 4(i%4)], it
// receives X[r0 + j][c0 + i] for j = 0..3: a column of a row-major tile.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gmdn {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define GMDN_DEV __device__ __forceinline__

GMDN_DEV int lane_id() { return threadIdx.x & 63; }
GMDN_DEV int wave_id() { return threadIdx.x >> 6; }

GMDN_DEV f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

GMDN_DEV f32x4 mfma(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
GMDN_DEV f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- operands
// An operand in split precision: value ~= hi + lo, both bf16.  P = 1 keeps
// only hi (inputs that are exact bf16); P = 2 keeps both.
template <int P>
struct Op {
  bf16x8 v[P];
};

// acc += a * b with split operands; the lo*lo term (2^-16 relative) is dropped.
template <int PA, int PB>
GMDN_DEV f32x4 mma(const Op<PA>& a, const Op<PB>& b, f32x4 acc) {
  acc = mfma(a.v[0], b.v[0], acc);
  if constexpr (PB == 2) acc = mfma(a.v[0], b.v[1], acc);
  if constexpr (PA == 2) acc = mfma(a.v[1], b.v[0], acc);
  return acc;
}

GMDN_DEV bf16 to_bf16(float x) { return (bf16)x; }
GMDN_DEV float from_bf16(bf16 x) { return (float)x; }

// Split x into hi + lo (both bf16).
GMDN_DEV void split2(float x, bf16& hi, bf16& lo) {
  hi = (bf16)x;
  lo = (bf16)(x - (float)hi);
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats rounded to bf16 (to nearest even) by one v_cvt_pk_bf16_f32.
GMDN_DEV bf16x2 to_bf16x2(float a, float b) { return __builtin_convertvector(f32x2{a, b}, bf16x2); }
GMDN_DEV bf16x4 to_bf16x4(const f32x4& x) {
  return __builtin_shufflevector(to_bf16x2(x[0], x[1]), to_bf16x2(x[2], x[3]), 0, 1, 2, 3);
}

// split2 of four values, two per conversion (hi's value as a float is its
// bits shifted into the upper half): the same bits in about three
// instructions per value instead of five.
GMDN_DEV void split4(const f32x4& x, bf16x4& hi, bf16x4& lo) {
  const bf16x2 h01 = to_bf16x2(x[0], x[1]), h23 = to_bf16x2(x[2], x[3]);
  const uint32_t a = __builtin_bit_cast(uint32_t, h01), b = __builtin_bit_cast(uint32_t, h23);
  const bf16x2 l01 = to_bf16x2(x[0] - __builtin_bit_cast(float, a << 16), x[1] - __builtin_bit_cast(float, a & 0xffff0000u));
  const bf16x2 l23 = to_bf16x2(x[2] - __builtin_bit_cast(float, b << 16), x[3] - __builtin_bit_cast(float, b & 0xffff0000u));
  hi = __builtin_shufflevector(h01, h23, 0, 1, 2, 3);
  lo = __builtin_shufflevector(l01, l23, 0, 1, 2, 3);
}

// Two D-layout tiles stacked along k (t0: k rows 0..15, t1: rows 16..31)
// -> pair-order operand.
template <int P>
GMDN_DEV Op<P> pack_tiles(const f32x4& t0, const f32x4& t1) {
  Op<P> r;
  if constexpr (P == 1) {
    r.v[0] = __builtin_shufflevector(to_bf16x4(t0), to_bf16x4(t1), 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    bf16x4 h0, l0, h1, l1;
    split4(t0, h0, l0);
    split4(t1, h1, l1);
    r.v[0] = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
    r.v[1] = __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7);
  }
  return r;
}

// ------------------------------------------------- swizzled bf16 LDS tiles
// Row-major bf16 tile with COLS elements per row, stored without padding; the
// 16-byte group q of row r sits at group q ^ (r & MASK).  Row reads (16
// rows, one 8-byte piece each) and transposing column reads (4 rows x 32
// bytes per lane group) then spread over the LDS banks.
template <int COLS>
struct BSwz {
  static constexpr int GPR = COLS / 8;  // 16-byte groups per row
  static constexpr int MASK = (GPR < 16 ? GPR : 16) - 1;
  static GMDN_DEV int xr(int r) { return r & MASK; }  // the row's XOR pattern
  static GMDN_DEV int off(int r, int c) { return r * COLS + ((((c >> 3) ^ xr(r)) << 3) | (c & 7)); }
};

// Row swizzle for tiles read by columns: the 16-byte group q of row r sits
// at q ^ f(r), with f a bijection of r mod 16.  The transposing column reads
// touch, per 16 lanes, four consecutive rows x four consecutive groups; under
// q ^ (r mod 16) the low bits of row and group cancel and those 16 reads land
// in four groups (a 4-way bank conflict, measured at half of the LDS-active
// cycles).  Here f moves the row's low two bits above the group's: for
// 256-byte rows (D = 128) f swaps the two 2-bit halves of r mod 16, giving 16
// distinct groups; for 128-byte rows (D = 64, two rows per 256-byte bank
// sweep) f(r) = 4 ((r >> 1) & 1) + ((r >> 2) & 3), giving 16 distinct (bank
// half, group) pairs.  Row reads and publishes (16 rows, one group) stay
// conflict-free since f is a bijection.
template <int COLS>
struct NSwz {
  static constexpr int GPR = COLS / 8;  // 16-byte groups per row
  static constexpr int MASK = 15;       // the pattern repeats every 16 rows
  static GMDN_DEV int f(int r) {
    if constexpr (COLS == 128)
      return ((r & 3) << 2) | ((r >> 2) & 3);
    else if constexpr (COLS == 64)
      return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else
      return r & (GPR < 16 ? GPR - 1 : 15);
  }
  static GMDN_DEV int xr(int r) { return f(r); }  // the row's XOR pattern
  static GMDN_DEV int off(int r, int c) { return r * COLS + ((((c >> 3) ^ f(r)) << 3) | (c & 7)); }
};

// LDS bank model (measured on gfx950 with SQ_LDS_BANK_CONFLICT): 64 banks of
// 4 bytes; a 16-byte access is served in cycles of 16 lanes -- within each
// half of the wave, the four-lane quads q = 0..7 of equal parity of
// popcount(q) -- and an 8-byte access (ds_read_b64, ds_read_b64_tr_b16) in
// cycles of 32 consecutive lanes.  The swizzles below are the XOR patterns
// linear in the row bits that do best under it for the access patterns named.
//
// RowSwz: 16-byte row reads (16 rows x one group per lane group) are
// conflict-free; the transposing reads that take four rows x 8-byte pieces
// of four groups (the Newton-Schulz planes' column operands in their stored
// column order; the K^T operands of the delta forward and reverse scans,
// columns 8 (i % 4) + 4u) are two-way, the least those patterns allow.
template <int COLS>
struct RowSwz {
  static constexpr int GPR = COLS / 8;  // 16-byte groups per row
  static constexpr int MASK = 15;       // the pattern repeats every 16 rows
  static GMDN_DEV int f(int r) {
    if constexpr (COLS >= 128)
      return ((r & 1) << 3) | ((r & 2) << 1) | ((r & 4) >> 1);
    else if constexpr (COLS == 64)
      return ((r & 2) << 1) | ((r & 4) >> 1);
    else
      return (r & 4) >> 1;
  }
  static GMDN_DEV int xr(int r) { return f(r); }
  static GMDN_DEV int off(int r, int c) { return r * COLS + ((((c >> 3) ^ f(r)) << 3) | (c & 7)); }
};

// PairSwz: 16-byte row reads, natural-order transposing column reads (col8:
// rows 8G + i/4, columns 4 (i % 4)) and 8-byte row pieces are conflict-free;
// the permuted transposing reads (col8p: columns 8 (i % 4)) two-way.  For the
// token-gradient kernels, which use all four.
template <int COLS>
struct PairSwz {
  static constexpr int GPR = COLS / 8;  // 16-byte groups per row
  static constexpr int MASK = 15;       // the pattern repeats every 16 rows
  static GMDN_DEV int f(int r) {
    if constexpr (COLS >= 128)
      return ((r & 1) << 3) ^ ((r & 2) << 1) ^ (((r >> 2) & 1) * 3) ^ (((r >> 3) & 1) * 2);
    else
      return ((r & 2) << 1) ^ (((r >> 2) & 1) * 3) ^ (((r >> 3) & 1) * 2);
  }
  static GMDN_DEV int xr(int r) { return f(r); }
  static GMDN_DEV int off(int r, int c) { return r * COLS + ((((c >> 3) ^ f(r)) << 3) | (c & 7)); }
};

// Byte offset of element (r, c) of a swizzled bf16 tile (c % 4 == 0 for the
// 8-byte pieces the kernels read).
template <class L>
GMDN_DEV uint32_t swz_off(int r, int c) {
  return (uint32_t)(2 * L::off(r, c));
}

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// lane (r, G) takes X[r0 + r][k0 + pair(G, s)], s = 0..7
template <class L>
GMDN_DEV bf16x8 b_row(const bf16* X, int r0, int k0) {
  const int l = lane_id(), r = r0 + (l & 15), G = l >> 4;
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(X + L::off(r, k0 + 4 * G));
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(X + L::off(r, k0 + 16 + 4 * G));
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// lane (c, G) takes X[k0 + pair(G, s)][c0 + c] (two transposing reads)
template <class L>
GMDN_DEV bf16x8 b_col(const bf16* X, int k0, int c0) {
  const int l = lane_id(), i = l & 15, G = l >> 4;
  const int rr = k0 + 4 * G + (i >> 2), cc = c0 + 4 * (i & 3);
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + L::off(rr, cc)));
  s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + L::off(rr + 16, cc)));
  const bf16x4 ab = __builtin_bit_cast(bf16x4, a), bb = __builtin_bit_cast(bf16x4, b);
  return bf16x8{ab[0], ab[1], ab[2], ab[3], bb[0], bb[1], bb[2], bb[3]};
}

// D-layout tile of X: lane (c, G) gets X[r0 + 4G + j][c0 + c], j = 0..3
template <class L>
GMDN_DEV f32x4 b_dtile(const bf16* X, int r0, int c0) {
  const int l = lane_id(), i = l & 15, G = l >> 4;
  s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + L::off(r0 + 4 * G + (i >> 2), c0 + 4 * (i & 3))));
  const bf16x4 ab = __builtin_bit_cast(bf16x4, a);
  return f32x4{(float)ab[0], (float)ab[1], (float)ab[2], (float)ab[3]};
}

// One 16-byte-per-lane LDS-DMA load (global_load_lds_dwordx4): lane l's 16
// bytes at gptr land at lds + 16 l.  `lds` must be the same for the whole
// wave.  Issued through inline asm on purpose: the compiler cannot tell the
// ring-buffer stage being filled from the stage being read and would
// otherwise wait for every in-flight copy before each LDS read; completion is
// tracked explicitly by the callers (wait_vmem / wait_vmem_le + barrier).
GMDN_DEV void lds_dma16(const void* gptr, void* lds) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)lds));
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(gptr), "{m0}"(m0v)
      : "memory");
}

// Same copy with a wave-uniform 64-bit base (SGPRs) and a per-lane 32-bit
// byte offset: the form the chunk loops use, with lane offsets computed once.
GMDN_DEV void lds_dma16_s(const void* sbase, uint32_t voff, uint32_t m0v) {
  asm volatile(
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %1"
      :
      : "v"(voff), "s"(sbase), "{m0}"(m0v)
      : "memory");
}

// LDS byte pointers.  Precomputed per-lane bases are kept as LDS pointers so
// that base + compile-time offset is an in-bounds address computation, which
// the compiler folds into the ds_read / ds_write immediate offset.
typedef __attribute__((address_space(3))) char* lds_ptr;
typedef const __attribute__((address_space(3))) char* lds_cptr;

template <class T>
GMDN_DEV T lds_ld(lds_cptr p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(p);
}
template <class T>
GMDN_DEV void lds_st(lds_ptr p, const T& v) {
  *reinterpret_cast<__attribute__((address_space(3))) T*>(p) = v;
}
GMDN_DEV bf16x4 lds_tr16(lds_cptr p) {
  const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(bf16x4, x);
}
GMDN_DEV bf16x8 cat8(const bf16x4& a, const bf16x4& b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Split-state pieces: the chunk kernels keep fp32 state matrices in memory
// as 16-byte pieces {hi[0..3], lo[0..3]} of four consecutive columns
// (x = hi + lo, hi = bf16(x), lo = bf16(x - hi)), the form their MFMA
// operands take, in the bytes the fp32 values would occupy.
GMDN_DEV bf16x8 split_piece(const f32x4& x) {
  bf16x4 hi, lo;
  split4(x, hi, lo);
  return cat8(hi, lo);
}
GMDN_DEV bf16x8 split_piece(const bf16x4& hi, const bf16x4& lo) { return cat8(hi, lo); }
GMDN_DEV f32x4 unsplit_piece(const bf16x8& p) {
  return f32x4{(float)p[0] + (float)p[4], (float)p[1] + (float)p[5], (float)p[2] + (float)p[6],
               (float)p[3] + (float)p[7]};
}
// -x of eight bf16 values (sign bits flipped)
GMDN_DEV bf16x8 neg8(const bf16x8& x) {
  using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, x) ^ 0x80008000u);
}
// Pieces of columns k0 .. k0+3 and k0+4 .. k0+7 -> split operand, natural k order
GMDN_DEV Op<2> join_pieces(const bf16x8& a, const bf16x8& b) {
  Op<2> r;
  r.v[0] = __builtin_shufflevector(a, b, 0, 1, 2, 3, 8, 9, 10, 11);
  r.v[1] = __builtin_shufflevector(a, b, 4, 5, 6, 7, 12, 13, 14, 15);
  return r;
}

// LDS byte address of a pointer into LDS (wave-uniform when `p` is).
GMDN_DEV uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) char*)p);
}
GMDN_DEV lds_ptr lds_base(void* p) { return (lds_ptr)p; }

// Plan of an asynchronous copy of a ROWS x COLS bf16 tile (global rows
// `gstride` elements apart, 16-byte aligned) into a swizzled LDS tile:
// NOPS = ROWS * COLS / 8 / NTHREADS LDS-DMA instructions per wave; lane l of
// instruction k fills physical 16-byte group k NTHREADS + 64 w + l and
// fetches the logical group stored there.  off[k] is that lane's byte offset
// from the tile's first global row.
template <class L, int ROWS, int NTHREADS>
struct DmaPlan {
  static constexpr int GROUPS = ROWS * L::GPR;
  static_assert(GROUPS % NTHREADS == 0, "tile must split evenly over the block");
  static constexpr int NOPS = GROUPS / NTHREADS;
  uint32_t off[NOPS];
  GMDN_DEV void init(int w, int64_t gstride) {
    const int l = lane_id();
#pragma unroll
    for (int k = 0; k < NOPS; ++k) {
      const int p = k * NTHREADS + w * 64 + l;
      const int r = p / L::GPR;
      const int q = (p % L::GPR) ^ L::xr(r);
      off[k] = (uint32_t)((r * gstride + q * 8) * 2);
    }
  }
  // issue the copy of the tile whose first global row starts at `g`
  GMDN_DEV void issue(const bf16* g, uint32_t lds_tile, int w) const {
#pragma unroll
    for (int k = 0; k < NOPS; ++k) lds_dma16_s(g, off[k], lds_tile + (k * NTHREADS + w * 64) * 16);
  }
};

// Wait for this wave's outstanding vector-memory operations, including the
// LDS-DMA loads above (the caller then synchronises the block).
GMDN_DEV void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Wait until at most N vector-memory operations of this wave are in flight.
template <int N>
GMDN_DEV void wait_vmem_le() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Hardware square root and reciprocal (v_sqrt_f32, v_rcp_f32: 1 ulp) in
// place of the correctly rounded library sequences (about ten instructions
// each), for the bf16x3 paths' elementwise state updates.
GMDN_DEV float hw_sqrt(float x) { return __builtin_amdgcn_sqrtf(x); }
GMDN_DEV float hw_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// ------------------------------------------------------------ reductions
// DPP move of a float within the wave (CTRL: quad_perm 0x00-0xff, row_ror:n
// 0x120 + n); every lane must be active.
template <int CTRL>
GMDN_DEV float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// Sum over the 64 lanes, wave-uniform result: two quad-permute and two
// row-rotate steps leave every lane of a 16-lane row holding the row's sum,
// then the four row sums are read into scalar registers.  No LDS traffic
// (a shuffle-based reduction costs six dependent LDS permutes).
GMDN_DEV float wave_sum(float x) {
  x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_mov<0x124>(x);  // row_ror:4
  x += dpp_mov<0x128>(x);  // row_ror:8
  const int xi = __builtin_bit_cast(int, x);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(xi, 48));
  return (r0 + r1) + (r2 + r3);
}

// wave_sum of two values at once: two independent DPP chains interleaved,
// half the dependent latency of two calls.
GMDN_DEV f32x2 wave_sum2(float x, float y) {
  x += dpp_mov<0xB1>(x);
  y += dpp_mov<0xB1>(y);
  x += dpp_mov<0x4E>(x);
  y += dpp_mov<0x4E>(y);
  x += dpp_mov<0x124>(x);
  y += dpp_mov<0x124>(y);
  x += dpp_mov<0x128>(x);
  y += dpp_mov<0x128>(y);
  const int xi = __builtin_bit_cast(int, x), yi = __builtin_bit_cast(int, y);
  auto rl = [](int v, int lane) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, lane)); };
  return f32x2{(rl(xi, 0) + rl(xi, 16)) + (rl(xi, 32) + rl(xi, 48)),
               (rl(yi, 0) + rl(yi, 16)) + (rl(yi, 32) + rl(yi, 48))};
}

// Sum over the 4 lane groups (G) of a value held per lane: result equal in
// all lanes sharing l%16.
GMDN_DEV float group_sum(float x) {
  x += __shfl_xor(x, 16, 64);
  x += __shfl_xor(x, 32, 64);
  return x;
}

}  // namespace gmdn
