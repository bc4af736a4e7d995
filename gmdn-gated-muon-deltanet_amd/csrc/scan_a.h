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

// workspace floats per (b, h) for the muon backward: the bf16x3 kernel keeps
// 2 ns + 2 matrices (iterates X_k, products Z_k, M_i, Mbar), the fp32 one 4 + ns
__host__ __device__ inline int64_t muon_bwd_ws_floats(int dh, int ns) {
  return (int64_t)(2 * ns + 2 > 4 + ns ? 2 * ns + 2 : 4 + ns) * dh * dh;
}

}  // namespace gmdn
