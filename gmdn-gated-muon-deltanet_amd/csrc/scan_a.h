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
hipError_t scan_bwd_muon_launch(const ScanArgs& s, float* ws);

// workspace floats per (b, h) of the fp32 ('ieee') muon backward: 4 + ns matrices
__host__ __device__ inline int64_t muon_bwd_ws_floats(int dh, int ns) { return (int64_t)(4 + ns) * dh * dh; }
// workspace floats of the whole muon backward, either precision: the bf16x3
// kernels keep per chunk the iterates X_0 .. X_ns, the products Z_0 .. Z_{ns-1}
// and M_i (2 ns + 2 matrices), per (b, h) the carried Mbar, per chunk |M_i|
inline int64_t muon_bwd_ws_total(int64_t BH, int64_t N, int dh, int ns) {
  const int64_t mat = (int64_t)dh * dh;
  const int64_t x3 = BH * N * (2 * ns + 2) * mat + BH * mat + BH * N;
  const int64_t f32 = BH * muon_bwd_ws_floats(dh, ns);
  return x3 > f32 ? x3 : f32;
}

}  // namespace gmdn
