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

hipError_t chunk_fwd_launch(const ChunkArgs& a, int d, int rule, hipStream_t s);
// rule 1: the serial muon scan (S_i, M_i of every chunk to S_out, M_out;
// M_out may be null) and the chunk-parallel output kernel
hipError_t chunk_fwd_muon_launch(const ChunkArgs& a, int d, float* S_out, float* M_out, int ns, hipStream_t s);
// exact WY/UT mode: prep kernel, the delta scan, output kernel (workspace in floats)
size_t wy_workspace_floats(int64_t B, int64_t H, int64_t T, int d);
hipError_t wy_fwd_launch(const ChunkArgs& a, int d, float* ws, hipStream_t s);
hipError_t chunk_bwd_launch(const ChunkArgs& a, int d, int rule, hipStream_t s);

}  // namespace gmdn
