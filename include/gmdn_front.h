/* C-ABI of the mixer front-end kernels in libgmdn_scan.so (MI355X, gfx950).
 *
 * The front-end of the reference's FastWeightMixer.forward between the qkv
 * projection and the state scan (train_ablation.py:124-128): a causal
 * depthwise Conv1d over time (kernel K, left padding K - 1, bias), SiLU,
 * the split into q, k, v and F.normalize of q and k over each head's dh
 * channels (eps 1e-12).  Error codes are those of gmdn_scan.h; the calls are
 * asynchronous on `stream` and allocate nothing.
 *
 * Layouts: y is the projection output (B, T, 3 D) with D = H dh, contiguous;
 * q, k, v are (B, T, D) contiguous (the (B, H, T, dh) operands of the scan
 * are their transposed views); weight is (3 D, K) float32 (the Conv1d weight
 * (3 D, 1, K) squeezed), bias (3 D) float32.  Every pointer is 16-byte
 * aligned.  dtype is GMDN_DTYPE_BF16 or
 * GMDN_DTYPE_F32 for y, q, k, v and their gradients.
 */
#ifndef GMDN_FRONT_H
#define GMDN_FRONT_H

#include <stddef.h>
#include <stdint.h>

#include "gmdn_scan.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Forward: q, k, v from y (replaces train_ablation.py:124-128).  dh is 16,
 * 32, 64 or 128, K at most 4. */
int gmdn_front_fwd(const void* y, const float* weight, const float* bias, void* q, void* k, void* v,
                   int64_t B, int64_t T, int32_t D, int32_t dh, int32_t K, int32_t dtype, void* stream);

/* Floats of the backward's partial-sum workspace: per (b, 64-token tile) and
 * channel, the K weight-gradient sums and the bias-gradient sum. */
size_t gmdn_front_bwd_workspace_floats(int64_t B, int64_t T, int32_t D, int32_t K);

/* Backward (autograd of the same lines): dy from dq, dk, dv ((B, T, D),
 * contiguous), and into `partial` ((B * ceil(T / 64), 3 D, K + 1) float32)
 * the per-tile sums whose sum over the first axis is (dweight, dbias). */
int gmdn_front_bwd(const void* y, const float* weight, const float* bias, const void* dq, const void* dk,
                   const void* dv, void* dy, float* partial, int64_t B, int64_t T, int32_t D, int32_t dh,
                   int32_t K, int32_t dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GMDN_FRONT_H */
