// Level B: the fused mixer core (stub until the kernels land).
#include "../../include/gmdn_scan.h"
#include "chunk_b.h"

extern "C" {

size_t gmdn_chunk_states_bytes(const gmdn_chunk_desc* desc) { return 0; }

int gmdn_chunk_fwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v,
                   const float* beta, const float* g, const float* gmu, const float* gnu, void* o,
                   void* states, void* stream) {
  return GMDN_ERR_UNSUPPORTED;
}

size_t gmdn_chunk_bwd_workspace_bytes(const gmdn_chunk_desc* desc) { return 0; }

int gmdn_chunk_bwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v,
                   const float* beta, const float* g, const float* gmu, const float* gnu,
                   const void* states, const void* dO, void* dq, void* dk, void* dv, float* dbeta,
                   float* dg, float* dgmu, float* dgnu, void* workspace, size_t workspace_bytes,
                   void* stream) {
  return GMDN_ERR_UNSUPPORTED;
}

}  // extern "C"
