/*
 * gmdn_scan.h -- C ABI of the MI355X (gfx950) fast-weight state scan.
 *
 * Plain C: no HIP or torch types.  `stream` is a hipStream_t passed as
 * void* (NULL = the default stream).  All pointers are device pointers to
 * caller-owned memory; the library never allocates and never synchronises
 * the host.  Every entry point returns GMDN_OK (0) or one of the error codes
 * below; gmdn_error_string() describes a code.  Calls are stateless and
 * reentrant; calls on different streams may run concurrently.
 *
 * Layout conventions
 *   Level A (the drop-in fast_state_scan): U, K, S_all, M_all, V_all, gS,
 *     dU, dK are contiguous (BH, N, dh, dh) float32; scalar streams a, b, m,
 *     n and their gradients are contiguous (BH, N) float32.  S is stored
 *     with rows = d_v, columns = d_k, as the reference's S_all.
 *   Level B (fused mixer core): q, k, v, o, dO, dq, dk, dv are (B, H, T, d)
 *     with element strides given per tensor for the B, H and T dimensions
 *     (d must be the unit-stride dimension); gate streams beta, g, gmu, gnu
 *     and their gradients are contiguous (B, H, T) float32.
 */
#ifndef GMDN_SCAN_H
#define GMDN_SCAN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* return codes */
#define GMDN_OK 0
#define GMDN_ERR_ARG 1         /* null pointer, bad size, bad rule/ns */
#define GMDN_ERR_UNSUPPORTED 2 /* head dim / chunk / dtype combination not built */
#define GMDN_ERR_WORKSPACE 3   /* workspace missing or too small */
#define GMDN_ERR_LAUNCH 4      /* hipGetLastError() reported a launch failure */

/* inner rules (reference train_ablation.py:179) */
#define GMDN_RULE_DELTA 0
#define GMDN_RULE_MUON 1
#define GMDN_RULE_ADAM 2

/* product precision of the state GEMMs (reference fast_scan.py:44, :196-199).
 * gfx950 has no TF32 MFMA: 'tf32' maps to bf16x3 split products
 * (hi*hi + hi*lo + lo*hi, fp32 accumulate, about 2^-16 relative error per
 * product), 'ieee' to fp32 MFMA (v_mfma_f32_16x16x4_f32). */
#define GMDN_PREC_TF32 0
#define GMDN_PREC_IEEE 1

/* element type of the Level-B token streams.  bf16 streams run the fused
 * E-form kernels (d = 64, 128).  float32 streams (d = 32, 64, 128, every
 * rule) run the reference's matrix form with exact float32 products, as the
 * reference computes when autocast is off (train_ablation.py:424, 465):
 * chunk-parallel kernels form Kw, Uv and the chunk scalars, the drop-in
 * scan kernels run in GMDN_PREC_IEEE, chunk-parallel kernels form o and,
 * backward, dL/dS_i and the token and gate gradients. */
#define GMDN_DTYPE_BF16 0
#define GMDN_DTYPE_F32 1

const char* gmdn_error_string(int code);

/* Supported head dims of the Level-A kernels (the reference dispatches its
 * kernels for power-of-two dh >= 16, fast_scan.py:406-408; this library
 * has 32, 64 and 128, and the Python host serves dh = 16 by zero-padding
 * U and K to 32, which is exact for every rule).  Returns 1 if dh is
 * supported, else 0. */
int gmdn_scan_supported(int32_t dh);

/* ------------------------------------------------------------------ Level A */

/* Forward of the chunk state scan; replaces _TritonScan.forward and
 * _scan_fwd_kernel (reference fast_scan.py:359-377, :206-248).
 *
 *   S_all[bh, i] = pre-update S_i, with S_0 = 0 and
 *   G_i = U_i - S_i K_i;  delta: S_{i+1} = a_i S_i + G_i
 *   muon: M_{i+1} = m_i M_i + G_i;  S_{i+1} = a_i S_i + b_i msign_ns(M_{i+1})
 *   adam: M_{i+1} = m_i M_i + (1-m_i) G_i;  V_{i+1} = n_i V_i + (1-n_i) G_i^2;
 *         S_{i+1} = a_i S_i + b_i M_{i+1} / (sqrt(V_{i+1}) + 1e-6)
 *
 * M_all (rules 1, 2) and V_all (rule 2) receive the pre-update moments that
 * gmdn_scan_bwd needs; either may be NULL when no backward will follow.
 * Adam with M_all or V_all requested runs in exact float32 (GMDN_PREC_IEEE)
 * whatever `precision` says: its backward amplifies the rounding of the
 * saved moments past the gradient tolerance under split-bf16 products.
 * ns: Newton-Schulz steps for rule 1 (0..8).  b, m, n may be NULL for rule 0;
 * n may be NULL for rule 1. */
int gmdn_scan_fwd(const float* U, const float* K, const float* a, const float* b,
                  const float* m, const float* n, float* S_all, float* M_all,
                  float* V_all, int64_t BH, int64_t N, int32_t dh, int32_t rule,
                  int32_t ns, int32_t precision, void* stream);

/* Workspace bytes gmdn_scan_bwd needs for these sizes (0 if none): adam
 * keeps per-row-tile partial sums of its scalar gradients.  Muon ('tf32')
 * runs the chunks in segments from the end and keeps, per chunk of a segment
 * and (b, h), the Newton-Schulz iterates X_0 .. X_ns, the products
 * Z_0 .. Z_{ns-1}, P_0 .. P_{ns-1} and M_i (3 ns + 2 dh^2 floats) and |M_i|,
 * plus two carried
 * dh^2 matrices per (b, h); the size returned here has as many chunks per
 * segment as fit in 512 MiB (at least one, at most N), and gmdn_scan_bwd also
 * accepts any smaller workspace down to one-chunk segments, using as many
 * chunks per segment as it holds.  Muon ('ieee'): 4 + ns dh^2 matrices per
 * (b, h). */
size_t gmdn_scan_bwd_workspace_bytes(int64_t BH, int64_t N, int32_t dh, int32_t rule,
                                     int32_t ns);

/* Backward of the chunk state scan; replaces _TritonScan.backward and
 * _scan_bwd_kernel (reference fast_scan.py:379-396, :269-331, derivation
 * :134-186).  Inputs are the forward's inputs and saved S_all / M_all /
 * V_all plus the cotangent gS of S_all.  Writes dU, dK (BH, N, dh, dh) and
 * da, db, dm, dn (BH, N).  Gradients of scalars the rule does not use are
 * written as zeros (the reference's Triton backward leaves them
 * uninitialised, fast_scan.py:387-389). */
int gmdn_scan_bwd(const float* U, const float* K, const float* a, const float* b,
                  const float* m, const float* n, const float* S_all,
                  const float* M_all, const float* V_all, const float* gS, float* dU,
                  float* dK, float* da, float* db, float* dm, float* dn,
                  void* workspace, size_t workspace_bytes, int64_t BH, int64_t N,
                  int32_t dh, int32_t rule, int32_t ns, int32_t precision,
                  void* stream);

/* Size of the library's own device scratch for gmdn_scan_bwd_noalloc. */
#define GMDN_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* gmdn_scan_bwd without a workspace argument.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * workspace lives in a file-scope device array of GMDN_NOALLOC_SCRATCH_BYTES
 * (64 MiB), one per GPU the library runs on, held until the process ends;
 * the call allocates nothing.  Problems whose smallest workspace (for muon
 * in 'tf32', one-chunk segments; otherwise gmdn_scan_bwd_workspace_bytes)
 * exceeds that size are refused with GMDN_ERR_WORKSPACE before any launch.  Every call on one GPU shares that
 * GPU's scratch: calls that overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.  Nothing a previous
 * call left in the scratch is read.  Same arguments, results and error codes
 * as gmdn_scan_bwd otherwise. */
int gmdn_scan_bwd_noalloc(const float* U, const float* K, const float* a, const float* b,
                          const float* m, const float* n, const float* S_all,
                          const float* M_all, const float* V_all, const float* gS,
                          float* dU, float* dK, float* da, float* db, float* dm, float* dn,
                          int64_t BH, int64_t N, int32_t dh, int32_t rule, int32_t ns,
                          int32_t precision, void* stream);

/* ------------------------------------------------------------------ Level B */

/* Problem description of the fused chunk op (phases 1-3 of the reference
 * mixer, train_ablation.py:142-187, in the E-form: per chunk
 * E = V - K S^T, o = Q S^T + A E with A = tril(Q K^T) diag(beta),
 * G = E^T diag(w) K, then the rule's state update). */
typedef struct gmdn_chunk_desc {
  int64_t B, H, T;      /* batch, heads, tokens (T % C == 0) */
  int32_t d;            /* head dim (d_k = d_v) */
  int32_t C;            /* chunk length (64) */
  int32_t rule;         /* GMDN_RULE_* */
  int32_t ns;           /* Newton-Schulz steps (rule 1) */
  int32_t dtype;        /* GMDN_DTYPE_* of q, k, v, o, dO, dq, dk, dv */
  int32_t precision;    /* GMDN_PREC_* of rule 1's Newton-Schulz VJP (backward) */
  float eps;            /* adam denominator epsilon (reference: 1e-6) */
  /* element strides (B, H, T) of each token stream; d is unit-stride */
  int64_t sq[3], sk[3], sv[3], so[3];
} gmdn_chunk_desc;

/* Bytes of the state checkpoint gmdn_chunk_fwd writes when `states` is
 * non-NULL (what gmdn_chunk_bwd consumes; for rules 0 and 2 its layout is
 * private to the library: rule 0 keeps the even chunks' states only, d x d
 * float32 each).  float32 streams: S_i [, M_i] [, V_i] of every chunk, the
 * chunks' Kw_i, Uv_i and their four scalars. */
size_t gmdn_chunk_states_bytes(const gmdn_chunk_desc* desc);

/* Forward: o = mixer core(q, k, v, beta, g[, gmu][, gnu]).  g, gmu, gnu are
 * log-gates; each is clamped at log(1e-6) as the reference clamps the gate
 * at 1e-6 before its log (train_ablation.py:155, :170-175).  gmu is needed
 * for rules 1 and 2, gnu for rule 2.  `states` receives the chunk states the
 * backward needs (gmdn_chunk_states_bytes); it may be NULL for rules 0 and 2 when no
 * backward follows.  Rule 1 (muon) always needs it: its output kernel reads
 * the chunk states (S_i, M_i float32 (B, H, N, d, d) planes, the layout
 * gmdn_scan_bwd takes as S_all, M_all), which its backward reads too.
 * float32 streams (every rule) always need it for the same reason, and
 * adam's eps must then be the drop-in scan's 1e-6 (fast_scan.py:94). */
int gmdn_chunk_fwd(const gmdn_chunk_desc* desc, const void* q, const void* k,
                   const void* v, const float* beta, const float* g,
                   const float* gmu, const float* gnu, void* o, void* states,
                   void* stream);

/* Exact WY/UT mode (no counterpart in the reference, which trains the
 * chunk-frozen form above and leaves this transform out,
 * train_ablation.py:12-18): o of the token-exact gated delta rule
 *   S_t = alpha_t S_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T,  o_t = S_t q_t,
 * alpha_t = exp(max(g_t, log 1e-6)), chunked by the WY/UT transform
 * (T = (I + strict_lower(diag(beta) (K K^T * Gamma)))^-1, U = T diag(beta) V,
 * W = T diag(beta gamma) K): T by forward substitution in float32, every
 * product split-bf16 (bf16 q, k, v exact, float32 intermediates as hi + lo,
 * about 2^-16 relative error per product).  desc->rule, ns and
 * eps are ignored; q, k, v, o bf16 (desc->dtype GMDN_DTYPE_BF16) with the
 * strides of desc. */
size_t gmdn_wy_fwd_workspace_bytes(const gmdn_chunk_desc* desc);
int gmdn_wy_fwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v,
                const float* beta, const float* g, void* o, void* workspace,
                size_t workspace_bytes, void* stream);

/* Backward of gmdn_wy_fwd (no counterpart in the reference, like the mode
 * itself).  `ckpt` is the workspace of the forward call on the same inputs,
 * kept unchanged since (the chunks' U_A, K_A, states S_i, Qt, Ov and decay a
 * that the forward formed).  Given dO (bf16, strides desc->so), writes dq,
 * dk, dv (bf16, strides desc->sq, sk, sv) and dbeta, dg (contiguous
 * (B, H, T) float32): the reverse delta scan (split-bf16) gives each chunk's
 * state cotangent, then chunk-parallel kernels differentiate the WY/UT chunk
 * algebra (T = (I + A)^-1, U, W, the decay masks) with split-bf16
 * products.  The workspace (gmdn_wy_bwd_workspace_bytes) holds gS and the
 * state cotangents (d x d per chunk), T, dM, dT (C x C per chunk), the
 * chunk intermediates X, Z, dX and partial dq, dk (B H T d each) and
 * per-token partial sums of the gate gradients. */
size_t gmdn_wy_bwd_workspace_bytes(const gmdn_chunk_desc* desc);
int gmdn_wy_bwd(const gmdn_chunk_desc* desc, const void* q, const void* k, const void* v,
                const float* beta, const float* g, const void* ckpt, const void* dO,
                void* dq, void* dk, void* dv, float* dbeta, float* dg, void* workspace,
                size_t workspace_bytes, void* stream);

/* Workspace bytes gmdn_chunk_bwd needs.  Muon (rule 1) on bfloat16 streams
 * in 'tf32' also runs with any smaller workspace down to one-chunk segments
 * of its reverse scan (the results do not depend on the segment length);
 * this size gives segments of up to 512 MiB of iterates, in two buffers
 * when they do not hold every chunk.  Adam (rule 2) at d = 64 on bfloat16
 * streams: this size ends with a carry of the reverse scan's cotangents
 * (B H d d * 3 floats), with which the scan runs in chunk segments and each
 * segment's token gradients run on a second stream of the library's (one
 * per device, default priority) beside the next segment's scan, joined back
 * before the call returns; a workspace smaller by that carry runs one scan
 * pass on the caller's stream.  Both give the same results bit for bit. */
size_t gmdn_chunk_bwd_workspace_bytes(const gmdn_chunk_desc* desc);

/* Backward given dO (strides desc->so) and the forward's `states`.  Writes
 * dq, dk, dv (strides desc->sq, sk, sv) and dbeta, dg[, dgmu][, dgnu]
 * (contiguous (B, H, T) float32).  Matches torch autograd through the
 * reference's phases 1-3 and scan_eager.  Rule 1 (muon) forms each chunk's
 * Kw, Uv and dL/dS_i, runs the drop-in muon reverse scan (Newton-Schulz VJP
 * in desc->precision) on the forward's S_i, M_i, then the token gradients;
 * in 'tf32' with two iterate buffers, the chunk-parallel stages of later
 * and earlier segments run in the launches of the serial reverse scan.
 * Adam (rule 2) at d = 128 runs the drop-in adam scan in exact float32
 * between chunk-parallel kernels, forward (when `states` is requested) and
 * backward; its epsilon must then be the reference's 1e-6. */
int gmdn_chunk_bwd(const gmdn_chunk_desc* desc, const void* q, const void* k,
                   const void* v, const float* beta, const float* g,
                   const float* gmu, const float* gnu, const void* states,
                   const void* dO, void* dq, void* dk, void* dv, float* dbeta,
                   float* dg, float* dgmu, float* dgnu, void* workspace,
                   size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GMDN_SCAN_H */
