// Internal launch interface of the drop-in chunk state scan kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gmdn {

struct ScanArgs {
  const float *U, *K, *a, *b, *m, *n;
  float *S_all, *M_all, *V_all;  // forward outputs / backward inputs
  const float* gS;
  float *dU, *dK, *da, *db, *dm, *dn;
  int64_t BH, N;
  int dh, rule, ns, precision;
  hipStream_t stream;
};

// delta / adam (rows of the state are independent)
hipError_t scan_fwd_rows_launch(const ScanArgs& s);
hipError_t scan_bwd_rows_launch(const ScanArgs& s, float* part);
// chunk-parallel dK_i = -S_i^T dU_i plus scalar gradients (all rules)
hipError_t scan_bwd_dk_launch(const ScanArgs& s, const float* part);
// muon (msign couples the whole state)
hipError_t scan_fwd_muon_launch(const ScanArgs& s);
hipError_t scan_bwd_muon_launch(const ScanArgs& s, float* ws, int64_t ws_floats);

// workspace floats per (b, h) of the fp32 ('ieee') muon backward: 4 + ns matrices
__host__ __device__ inline int64_t muon_bwd_ws_floats(int dh, int ns) { return (int64_t)(4 + ns) * dh * dh; }
// The bf16x3 muon backward keeps, per chunk of a segment, the iterates
// X_0 .. X_ns, the products Z_0 .. Z_{ns-1}, P_0 .. P_{ns-1} and M_i
// (3 ns + 2 matrices) and |M_i|, in nbuf buffers (two let one segment's
// iterates be formed while the previous segment's reverse pass runs); per
// (b, h) the carried Mbar and Sb.  Workspace floats for segments of nseg
// chunks:
inline int64_t muon_bwd_ws_segment_floats(int64_t BH, int64_t nseg, int dh, int ns, int nbuf = 1) {
  const int64_t mat = (int64_t)dh * dh;
  return nbuf * BH * nseg * ((3 * ns + 2) * mat + 1) + 2 * BH * mat;
}
// Segment length and buffer count for a workspace of ws_floats: one segment
// of all N chunks if one buffer holds them, else two buffers of as many
// chunks as fit, else one buffer of as many (nseg 0: too small).
struct MuonBwdPlan {
  int64_t nseg;
  int nbuf;
};
inline MuonBwdPlan muon_bwd_plan(int64_t BH, int64_t N, int dh, int ns, int64_t ws_floats) {
  const int64_t mat = (int64_t)dh * dh;
  const int64_t per = BH * ((3 * ns + 2) * mat + 1), fixed = 2 * BH * mat;
  if (ws_floats < fixed + per) return {0, 1};
  const int64_t n1 = (ws_floats - fixed) / per, n2 = (ws_floats - fixed) / (2 * per);
  if (n1 >= N) return {N, 1};
  if (n2 >= 1) return {n2, 2};
  return {n1, 1};
}
// The default workspace: two buffers of segments of as many chunks as fit in
// MUON_BWD_WS_BUDGET bytes each (at least one chunk; one buffer of all N
// chunks if they fit), or the fp32 kernel's per-(b, h) matrices if larger.
constexpr int64_t MUON_BWD_WS_BUDGET = (int64_t)512 << 20;
inline int64_t muon_bwd_ws_total(int64_t BH, int64_t N, int dh, int ns) {
  const int64_t mat = (int64_t)dh * dh;
  const int64_t per = BH * ((3 * ns + 2) * mat + 1);
  int64_t nseg = (MUON_BWD_WS_BUDGET / 4 - 2 * BH * mat) / per;
  if (nseg < 1) nseg = 1;
  if (nseg > N) nseg = N;
  const int64_t x3 = muon_bwd_ws_segment_floats(BH, nseg, dh, ns, nseg < N ? 2 : 1);
  const int64_t f32 = BH * muon_bwd_ws_floats(dh, ns);
  return x3 > f32 ? x3 : f32;
}

}  // namespace gmdn
