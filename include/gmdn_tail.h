/* C-ABI of the mixer's gate activations and per-head output norm in
 * libgmdn_scan.so (MI355X, gfx950).
 *
 * Gates (reference train_ablation.py:131-134 with the clamped logs of
 * :155, :169-175): the gate projection's output y (B, T, nG H) -- channel
 * g H + h is gate g of head h -- becomes per gate a (B, H, T) float32 row:
 *   g = 1 (beta):              sigmoid(y)
 *   g = 0, 2, 3 (alpha, mu, nu): max(log sigmoid(y), log 1e-6)
 * (log of the gate clamped at 1e-6, the form the fused core takes), in one
 * (nG, B, H, T) float32 output.
 *
 * Head norm (reference :188, nn.RMSNorm(dh) applied to each head's output):
 *   out = x / sqrt(mean(x^2) + eps) * weight   over each row of d elements,
 * on x (rows, d) in the mixer's (B, T, H, d) layout, so the output is
 * already the (B, T, D) input of the output projection.
 *
 * dtype (GMDN_DTYPE_BF16 or GMDN_DTYPE_F32) is that of y / dy and x / out /
 * dx; everything else is float32.  Pointers are 16-byte aligned, tensors
 * contiguous.  Error codes are those of gmdn_scan.h; calls are asynchronous
 * on `stream` and allocate nothing.
 */
#ifndef GMDN_TAIL_H
#define GMDN_TAIL_H

#include <stddef.h>
#include <stdint.h>

#include "gmdn_scan.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces torch.sigmoid(self.gates(x)) and the gate logs
 * (train_ablation.py:131-134, :152-175).  nG is 3 or 4, nG H <= 128. */
int gmdn_gates_fwd(const void* y, float* out, int64_t B, int64_t T, int32_t H, int32_t nG, int32_t dtype,
                   void* stream);

/* dy from the cotangent `dout` of gmdn_gates_fwd's output ((nG, B, H, T),
 * zeros for gates nothing reads): sigmoid'(y) for beta; for the log gates
 * 1 - sigmoid(y) where the log is above the floor, else 0. */
int gmdn_gates_bwd(const void* y, const float* dout, void* dy, int64_t B, int64_t T, int32_t H, int32_t nG,
                   int32_t dtype, void* stream);

/* Replaces self.norm(o) (train_ablation.py:188).  d is 16, 32, 64 or 128; rstd
 * receives 1 / sqrt(mean(x^2) + eps) per row for the backward. */
int gmdn_head_norm_fwd(const void* x, const float* weight, void* out, float* rstd, int64_t rows, int32_t d,
                       float eps, int32_t dtype, void* stream);

/* Floats of the backward's workspace (per-workgroup partial sums of the
 * weight gradient). */
size_t gmdn_head_norm_bwd_workspace_floats(int64_t rows, int32_t d);

/* dx and dweight (float32, d) of gmdn_head_norm_fwd given dout. */
int gmdn_head_norm_bwd(const void* x, const float* weight, const float* rstd, const void* dout, void* dx,
                       float* dweight, float* workspace, size_t workspace_floats, int64_t rows, int32_t d,
                       int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GMDN_TAIL_H */
