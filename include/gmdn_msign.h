/* C-ABI of the outer-Muon msign kernels in libgmdn_scan.so (MI355X, gfx950).
 *
 * msign of a batch of rectangular matrices, as the reference's Muon optimizer
 * applies it to every 2-D hidden weight's update (train_ablation.py:60-73,
 * called at :284): X = M (or M^T when rows > cols), X <- X / (|X|_F + eps),
 * then `steps` quintic Newton-Schulz steps
 *
 *     A = X X^T ;  X <- 3.4445 X + (-4.7750 A + 2.0315 A A) X
 *
 * and the result transposed back.  The products run on bf16 MFMA with split
 * operands (x = hi + lo, three products, about 2^-16 relative per product);
 * the iterates live in a caller-provided workspace as split pieces, each
 * matrix zero-padded to multiples of 128 (padding leaves the iteration
 * exact).  Error codes are those of gmdn_scan.h; the call is asynchronous on
 * `stream` and allocates nothing.
 */
#ifndef GMDN_MSIGN_H
#define GMDN_MSIGN_H

#include <stddef.h>
#include <stdint.h>

#include "gmdn_scan.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes of the workspace gmdn_msign needs for `batch` matrices of
 * rows x cols (0 for an empty batch or an unsupported size). */
size_t gmdn_msign_workspace_bytes(int64_t batch, int64_t rows, int64_t cols);

/* out[b] = msign(M[b], steps, eps) for b < batch (replaces
 * train_ablation.py:60-73, msign(M, steps, eps), for M of shape
 * (batch, rows, cols)).  M and out are contiguous (batch, rows, cols) of
 * dtype GMDN_DTYPE_F32 or GMDN_DTYPE_BF16 (the result is cast back to the
 * input dtype, as the reference's X.to(dt)); they must not overlap the
 * workspace, which is 256-byte aligned and at least
 * gmdn_msign_workspace_bytes(batch, rows, cols) long (GMDN_ERR_WORKSPACE
 * otherwise).  batch <= 65535; rows, cols <= 32768; steps in [0, 64]. */
int gmdn_msign(const void* M, void* out, int64_t batch, int64_t rows, int64_t cols, int32_t steps, float eps,
               int32_t dtype, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GMDN_MSIGN_H */
