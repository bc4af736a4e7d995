// Shared definitions of the fused chunk (Level B) kernels: problem arguments,
// workgroup geometry and the launch interface between translation units.
#pragma once
#include "tile.h"

namespace gmdn {

constexpr int CB_C = 64;  // chunk length
constexpr int CB_WAVES = 4;
constexpr int CB_THREADS = CB_WAVES * 64;
constexpr float LOG_FLOOR = -13.815510557964274f;  // log(1e-6)
// LDS ring depth of the serial chunk loops: tiles arrive RING - 1 chunks ahead
constexpr int RING = 3;

struct ChunkArgs {
  const bf16 *q, *k, *v;
  const float *beta, *g, *gmu, *gnu;
  bf16* o;         // forward output (backward: dO, read only)
  float* states;   // per-chunk pre-update S_i [, M_i, V_i] planes (backward: read only)
  int64_t B, H, T;
  int N;
  float eps;
  int64_t sq[3], sk[3], sv[3], so[3];
  // backward only
  float* gb;       // per-chunk state cotangents Gb_i (B, H, N, d, d)
  float* part;     // per (chunk, row block): partial da, db, dm, dn
  bf16 *dq, *dk, *dv;
  float *dbeta, *dg, *dgmu, *dgnu;
};

// blockIdx -> ((b, h), row block).  Workgroups are dispatched round-robin
// over the 8 XCDs; all row blocks of one (b, h) go to one XCD so that they
// share its token stream through that XCD's L2.
GMDN_DEV void map_block(int64_t BH, int nblk, int64_t& bh, int& blk) {
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

// ------------------------------------------------- LDS operand helpers
// lane (m, G) takes X[r][k0 + 8G .. k0 + 8G + 7] (natural k order, 16 bytes).
// The helpers take the lane index (lane_id() by default): a caller in a loop
// passes its own copy so that the addresses are not hoisted out of the loop.
template <class L>
GMDN_DEV bf16x8 row8(const bf16* X, int r, int k0, int l = lane_id()) {
  return *reinterpret_cast<const bf16x8*>(X + L::off(r, k0 + 8 * (l >> 4)));
}

// lane (i, G) takes X[k0 + 8G + j][c0 + i], j = 0..7 (two transposing reads)
template <class L>
GMDN_DEV bf16x8 col8(const bf16* X, int k0, int c0, int l = lane_id()) {
  const int i = l & 15, G = l >> 4;
  const int rr = k0 + 8 * G + (i >> 2), cc = c0 + 4 * (i & 3);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + L::off(rr, cc)));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + L::off(rr + 4, cc)));
  return cat8(__builtin_bit_cast(bf16x4, a), __builtin_bit_cast(bf16x4, b));
}

GMDN_DEV float dot4(const f32x4& a, const f32x4& b) {
  return a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
}

// Column operand whose output lane i stands for column cb + 8 (i / 4) + i % 4:
// lane (i, G) takes X[k0 + 8G + j][cb + 8 (i / 4) + i % 4], j = 0..7.  With
// cb = 32 kb + 4u, output row 4G' + jj of the product is column
// 32 kb + 8 G' + 4u + jj, so tiles u = 0, 1 hold, per lane group G', the
// eight consecutive columns 32 kb + 8 G' .. +7 of one pair of state-row
// pieces (the order the checkpoints keep).
template <class L>
GMDN_DEV bf16x8 col8p(const bf16* X, int k0, int cb, int l = lane_id()) {
  const int i = l & 15, G = l >> 4;
  const int rr = k0 + 8 * G + (i >> 2), cc = cb + 8 * (i & 3);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + L::off(rr, cc)));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(X + L::off(rr + 4, cc)));
  return cat8(__builtin_bit_cast(bf16x4, a), __builtin_bit_cast(bf16x4, b));
}

hipError_t chunk_fwd_launch(const ChunkArgs& a, int d, int rule, hipStream_t s);
// delta rule and adam: row-owned state waves, one barrier per chunk
hipError_t chunk_fwd_rows_launch(const ChunkArgs& a, int d, int rule, hipStream_t s);
// adam at d = 64: 16-row workgroups, four state waves per row block
hipError_t chunk_fwd_adam16_launch(const ChunkArgs& a, int d, hipStream_t s);
// rule 1: the serial muon scan (S_i, M_i of every chunk to S_out, M_out;
// M_out may be null) and the chunk-parallel output kernel
hipError_t chunk_fwd_muon_launch(const ChunkArgs& a, int d, float* S_out, float* M_out, int ns, hipStream_t s);
// exact WY/UT mode: prep kernel, the delta scan, output kernel (workspace in floats)
size_t wy_workspace_floats(int64_t B, int64_t H, int64_t T, int d);
hipError_t wy_fwd_launch(const ChunkArgs& a, int d, float* ws, hipStream_t s);
// its backward from the forward's workspace (the checkpoint) and dO (strides a.so)
size_t wy_bwd_workspace_floats(int64_t B, int64_t H, int64_t T, int d);
hipError_t wy_bwd_launch(const ChunkArgs& a, int d, float* ckpt, const void* dO, void* dq, void* dk, void* dv,
                         float* dbeta, float* dg, float* ws, hipStream_t s);
// ascan_carry (adam at d = 64, B H d d * 3 floats, or null): the carry of
// the reverse scan's segments; with it the scan runs in segments beside the
// token gradients of the segment before, on a second stream
hipError_t chunk_bwd_launch(const ChunkArgs& a, int d, int rule, float* ascan_carry, hipStream_t s);
// delta rule: the reverse scan of the state cotangent (Gb of the odd chunks)
hipError_t chunk_bwd_dscan_launch(const ChunkArgs& a, int d, hipStream_t s);
// adam at d = 64: the reverse scan of the state and moment cotangents (Gb of
// every chunk; partial sums of da, db, dm, dn per chunk and 16-row block)
// over chunks c1 - 1 .. c0; the cotangents of chunk c1 enter from `carry`
// (B H d d * 3 floats) unless c1 = N, and leave into it unless c0 = 0
hipError_t chunk_bwd_ascan_launch(const ChunkArgs& a, int d, float* carry, int c0, int c1, hipStream_t s);
// the matrix form's per-chunk Kw, Uv (fwd) and gS (bwd) as (B, H, N, d, d)
// float32, and a, b, m, n (four B H N arrays): muon (fwd and bwd together,
// for its backward) and adam at d = 128 (fwd: training forward, bwd: backward)
hipError_t chunk_prep_launch(const ChunkArgs& a, int d, int rule, bool fwd, bool bwd, float* Kw, float* Uv,
                             float* gS, float* abm, hipStream_t s);
// o = Q S_i^T + A E from float32 S_i planes (chunk-parallel)
hipError_t chunk_out_launch(const ChunkArgs& a, int d, const float* S_all, hipStream_t s);
// muon backward (workspace floats; states = S_i then M_i planes of every chunk)
size_t chunk_bwd_muon_ws_floats(int64_t BH, int64_t N, int d, int ns);
// the smallest workspace the 'tf32' muon backward runs with (one-chunk segments)
size_t chunk_bwd_muon_min_ws_floats(int64_t BH, int64_t N, int d, int ns);
hipError_t chunk_bwd_muon_launch(const ChunkArgs& a, int d, int ns, int precision, float* ws, size_t ws_floats,
                                 hipStream_t s);
// adam at d = 128, exact float32 scan: training forward (states = S, M, V,
// Kw, Uv planes and the four scalar arrays) and backward
size_t chunk_adam_mat_states_floats(int64_t BH, int64_t N, int d);
hipError_t chunk_fwd_adam_mat_launch(const ChunkArgs& a, int d, float* states, hipStream_t s);
size_t chunk_bwd_adam_mat_ws_floats(int64_t BH, int64_t N, int d);
hipError_t chunk_bwd_adam_mat_launch(const ChunkArgs& a, int d, float* ws, hipStream_t s);
// delta rule: token gradients of chunk pairs (i0 = 2p from the forward's
// checkpoint, i1 = 2p + 1 from the reverse scan's Gb)
hipError_t chunk_bwd_pair_launch(const ChunkArgs& a, int d, hipStream_t s);
// float32 token streams (every rule, d = 32, 64, 128): the matrix form with
// exact float32 products around the drop-in scan in 'ieee'.  The token
// pointers of ChunkArgs hold float32 data.  states = S [, M] [, V] planes of
// every chunk, Kw, Uv planes, then a, b, m, n (floats below); the backward
// workspace holds gS, dU, dK, the scalar gradients and the drop-in
// backward's own workspace.
size_t chunk_f32_states_floats(int64_t BH, int64_t N, int d, int rule);
size_t chunk_f32_bwd_ws_floats(int64_t BH, int64_t N, int d, int rule, int ns);
hipError_t chunk_fwd_f32_launch(const ChunkArgs& a, int d, int rule, int ns, float* states, hipStream_t s);
hipError_t chunk_bwd_f32_launch(const ChunkArgs& a, int d, int rule, int ns, const float* states, float* ws,
                                size_t ws_floats, hipStream_t s);

}  // namespace gmdn
