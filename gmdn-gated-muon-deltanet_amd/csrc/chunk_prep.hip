// Level B: launches of the chunk-parallel matrix-form stage (chunk_prep.h)
// for muon's backward and adam's training at d = 128.
#include "../../include/gmdn_scan.h"
#include "chunk_prep.h"

namespace gmdn {

template <int D, int RULE, bool FWD, bool BWD>
__global__ void __launch_bounds__(PrepLds<D>::NTHR) chunk_prep(ChunkArgs p, float* __restrict__ Kw,
                                                              float* __restrict__ Uv, float* __restrict__ gS,
                                                              float* __restrict__ abm) {
  chunk_prep_body<D, RULE, FWD, BWD>(p, Kw, Uv, gS, abm, blockIdx.x / p.N, (int)(blockIdx.x % p.N));
}

template <int D, int RULE, bool FWD, bool BWD>
static hipError_t launch_prep(const ChunkArgs& a, float* Kw, float* Uv, float* gS, float* abm, hipStream_t s) {
  auto k = chunk_prep<D, RULE, FWD, BWD>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, PrepLds<D>::BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, dim3((unsigned)(a.B * a.H * a.N)), dim3(PrepLds<D>::NTHR), PrepLds<D>::BYTES, s, a, Kw, Uv,
                     gS, abm);
  return hipGetLastError();
}

hipError_t chunk_prep_launch(const ChunkArgs& a, int d, int rule, bool fwd, bool bwd, float* Kw, float* Uv,
                             float* gS, float* abm, hipStream_t s) {
  // muon's backward: Kw, Uv and gS; adam: Kw, Uv (training forward), gS (backward)
  if (d == 128) {
    if (rule == 1 && fwd && bwd) return launch_prep<128, 1, true, true>(a, Kw, Uv, gS, abm, s);
    if (rule == 2 && fwd && !bwd) return launch_prep<128, 2, true, false>(a, Kw, Uv, gS, abm, s);
    if (rule == 2 && !fwd && bwd) return launch_prep<128, 2, false, true>(a, Kw, Uv, gS, abm, s);
  } else if (d == 64) {
    if (rule == 1 && fwd && bwd) return launch_prep<64, 1, true, true>(a, Kw, Uv, gS, abm, s);
  }
  return hipErrorNotSupported;
}

// Adam at d = 128, training forward: Kw, Uv and the chunk scalars, the
// drop-in adam scan in exact float32 (S, M, V of every chunk), then
// o = Q S_i^T + A E from S_i.  states = [S | M | V | Kw | Uv | a b m n].
size_t chunk_adam_mat_states_floats(int64_t BH, int64_t N, int d) {
  return (size_t)(5 * BH * N * (int64_t)d * d + 4 * BH * N);
}

hipError_t chunk_fwd_adam_mat_launch(const ChunkArgs& a, int d, float* states, hipStream_t s) {
  if (d != 128) return hipErrorNotSupported;
  const int64_t BH = a.B * a.H, BHN = BH * a.N, mat = (int64_t)d * d;
  float* S = states;
  float* Kw = S + 3 * BHN * mat;
  float* Uv = S + 4 * BHN * mat;
  float* abm = S + 5 * BHN * mat;
  hipError_t e = chunk_prep_launch(a, d, 2, true, false, Kw, Uv, nullptr, abm, s);
  if (e != hipSuccess) return e;
  ScanArgs sa{};
  sa.U = Uv; sa.K = Kw; sa.a = abm; sa.b = abm + BHN; sa.m = abm + 2 * BHN; sa.n = abm + 3 * BHN;
  sa.S_all = S; sa.M_all = S + BHN * mat; sa.V_all = S + 2 * BHN * mat;
  sa.BH = BH; sa.N = a.N; sa.dh = d; sa.rule = 2; sa.ns = 0; sa.precision = GMDN_PREC_IEEE;
  sa.stream = s;
  e = scan_fwd_rows_launch(sa);
  if (e != hipSuccess) return e;
  return chunk_out_launch(a, d, S, s);
}

}  // namespace gmdn
