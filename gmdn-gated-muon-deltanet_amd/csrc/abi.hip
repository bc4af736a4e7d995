// extern "C" entry points of libgmdn_scan.so (declared in include/gmdn_scan.h).
// Argument validation happens here, on the host, before any launch: a call
// that returns an error has launched nothing.
#include "../../include/gmdn_scan.h"
#include "scan_a.h"
#include "chunk_b.h"

#include <mutex>

using namespace gmdn;

// Scratch of gmdn_scan_bwd_noalloc: the backward's workspace (adam's
// partial sums, muon's iterates) in a file-scope device array, one copy per
// GPU, held until the process ends.  Host code never passes `scratch` itself
// to a kernel (in host code the name is a stand-in, not a device address):
// it uses the address hipGetSymbolAddress returns for the current device.
static_assert(GMDN_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
static __device__ __align__(256) char scratch[GMDN_NOALLOC_SCRATCH_BYTES];

namespace {

int launch_status(hipError_t e) { return e == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH; }

bool dh_ok(int32_t dh) { return dh == 32 || dh == 64 || dh == 128; }

// Smallest workspace the backward runs with: the muon backward's segments
// shrink to one chunk; the other rules need their full partial sums.
size_t scan_bwd_min_workspace(int64_t BH, int64_t N, int32_t dh, int32_t rule, int32_t ns, int32_t precision) {
  if (rule != 1) return gmdn_scan_bwd_workspace_bytes(BH, N, dh, rule, ns);
  if (precision == GMDN_PREC_IEEE) return (size_t)(BH * muon_bwd_ws_floats(dh, ns)) * sizeof(float);
  return (size_t)muon_bwd_ws_segment_floats(BH, 1, dh, ns) * sizeof(float);
}

int check_scan_common(const float* U, const float* K, const float* a, const float* b,
                      const float* m, const float* n, int64_t BH, int64_t N, int32_t dh,
                      int32_t rule, int32_t ns, int32_t precision) {
  if (BH < 0 || N < 0 || ns < 0 || ns > 8) return GMDN_ERR_ARG;
  if (rule < 0 || rule > 2) return GMDN_ERR_ARG;
  if (precision != GMDN_PREC_TF32 && precision != GMDN_PREC_IEEE) return GMDN_ERR_ARG;
  if (!dh_ok(dh)) return GMDN_ERR_UNSUPPORTED;
  if (BH * N == 0) return GMDN_OK;
  if (BH > (int64_t)1 << 31 || N > (int64_t)1 << 30) return GMDN_ERR_ARG;
  if (!U || !K || !a) return GMDN_ERR_ARG;
  if (rule >= 1 && (!b || !m)) return GMDN_ERR_ARG;
  if (rule == 2 && !n) return GMDN_ERR_ARG;
  return GMDN_OK;
}

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[MAX_DEVICES] = {};

// The device address of the current device's scratch (looked up once per
// device, with that device current); GMDN_ERR_LAUNCH when the runtime fails.
int scratch_of_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return GMDN_ERR_LAUNCH;
  std::lock_guard<std::mutex> g(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return GMDN_ERR_LAUNCH;
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return GMDN_OK;
}

}  // namespace

extern "C" {

const char* gmdn_error_string(int code) {
  switch (code) {
    case GMDN_OK: return "ok";
    case GMDN_ERR_ARG: return "invalid argument (null pointer, size, rule, ns or precision)";
    case GMDN_ERR_UNSUPPORTED: return "unsupported configuration (head dim, chunk length or dtype)";
    case GMDN_ERR_WORKSPACE: return "workspace missing or too small";
    case GMDN_ERR_LAUNCH: return "kernel launch failed";
  }
  return "unknown error";
}

int gmdn_scan_supported(int32_t dh) { return dh_ok(dh) ? 1 : 0; }

int gmdn_scan_fwd(const float* U, const float* K, const float* a, const float* b, const float* m,
                  const float* n, float* S_all, float* M_all, float* V_all, int64_t BH, int64_t N,
                  int32_t dh, int32_t rule, int32_t ns, int32_t precision, void* stream) {
  int rc = check_scan_common(U, K, a, b, m, n, BH, N, dh, rule, ns, precision);
  if (rc != GMDN_OK || BH * N == 0) return rc;
  if (!S_all) return GMDN_ERR_ARG;
  ScanArgs s{};
  s.U = U; s.K = K; s.a = a; s.b = b; s.m = m; s.n = n;
  s.S_all = S_all; s.M_all = M_all; s.V_all = V_all;
  s.BH = BH; s.N = N; s.dh = dh; s.rule = rule; s.ns = ns; s.precision = precision;
  // adam's backward amplifies the rounding of the moments it is handed:
  // with split-bf16 products in the forward, dK is 0.29 (Frobenius) from
  // float64 at BH = 64, N = 64, dh = 128 where exact float32 products give
  // 3e-3.  When the moments are kept for a backward, the forward runs in
  // exact float32.
  if (rule == 2 && (M_all || V_all)) s.precision = GMDN_PREC_IEEE;
  s.stream = (hipStream_t)stream;
  return launch_status(rule == 1 ? scan_fwd_muon_launch(s) : scan_fwd_rows_launch(s));
}

size_t gmdn_scan_bwd_workspace_bytes(int64_t BH, int64_t N, int32_t dh, int32_t rule, int32_t ns) {
  if (BH <= 0 || N <= 0 || !dh_ok(dh) || ns < 0) return 0;
  if (rule == 2) return (size_t)(BH * N * (dh / 16) * 4) * sizeof(float);
  if (rule == 1) return (size_t)muon_bwd_ws_total(BH, N, dh, ns) * sizeof(float);
  return 0;
}

int gmdn_scan_bwd(const float* U, const float* K, const float* a, const float* b, const float* m,
                  const float* n, const float* S_all, const float* M_all, const float* V_all,
                  const float* gS, float* dU, float* dK, float* da, float* db, float* dm, float* dn,
                  void* workspace, size_t workspace_bytes, int64_t BH, int64_t N, int32_t dh,
                  int32_t rule, int32_t ns, int32_t precision, void* stream) {
  int rc = check_scan_common(U, K, a, b, m, n, BH, N, dh, rule, ns, precision);
  if (rc != GMDN_OK || BH * N == 0) return rc;
  if (!S_all || !gS || !dU || !dK || !da || !db || !dm || !dn) return GMDN_ERR_ARG;
  if (rule >= 1 && !M_all) return GMDN_ERR_ARG;
  if (rule == 2 && !V_all) return GMDN_ERR_ARG;
  // muon: any workspace from the one-chunk segment up (the segments use what
  // is given); gmdn_scan_bwd_workspace_bytes is the default size
  const size_t need = scan_bwd_min_workspace(BH, N, dh, rule, ns, precision);
  if (need > 0 && (!workspace || workspace_bytes < need)) return GMDN_ERR_WORKSPACE;
  ScanArgs s{};
  s.U = U; s.K = K; s.a = a; s.b = b; s.m = m; s.n = n;
  s.S_all = const_cast<float*>(S_all); s.M_all = const_cast<float*>(M_all);
  s.V_all = const_cast<float*>(V_all); s.gS = gS;
  s.dU = dU; s.dK = dK; s.da = da; s.db = db; s.dm = dm; s.dn = dn;
  s.BH = BH; s.N = N; s.dh = dh; s.rule = rule; s.ns = ns; s.precision = precision;
  s.stream = (hipStream_t)stream;
  hipError_t e;
  float* part = static_cast<float*>(workspace);
  if (rule == 1) {
    e = scan_bwd_muon_launch(s, part, (int64_t)(workspace_bytes / sizeof(float)));
  } else {
    e = scan_bwd_rows_launch(s, part);
  }
  if (e != hipSuccess) return GMDN_ERR_LAUNCH;
  return launch_status(scan_bwd_dk_launch(s, part));
}

int gmdn_scan_bwd_noalloc(const float* U, const float* K, const float* a, const float* b,
                          const float* m, const float* n, const float* S_all, const float* M_all,
                          const float* V_all, const float* gS, float* dU, float* dK, float* da,
                          float* db, float* dm, float* dn, int64_t BH, int64_t N, int32_t dh,
                          int32_t rule, int32_t ns, int32_t precision, void* stream) {
  int rc = check_scan_common(U, K, a, b, m, n, BH, N, dh, rule, ns, precision);
  if (rc != GMDN_OK || BH * N == 0) return rc;
  if (scan_bwd_min_workspace(BH, N, dh, rule, ns, precision) > GMDN_NOALLOC_SCRATCH_BYTES) return GMDN_ERR_WORKSPACE;
  void* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc != GMDN_OK) return rc;
  return gmdn_scan_bwd(U, K, a, b, m, n, S_all, M_all, V_all, gS, dU, dK, da, db, dm, dn, ws,
                       GMDN_NOALLOC_SCRATCH_BYTES, BH, N, dh, rule, ns, precision, stream);
}

}  // extern "C"
