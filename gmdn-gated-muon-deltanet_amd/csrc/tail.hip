// The mixer's gate activations and per-head output norm, forward and
// backward, with their extern "C" entry points (include/gmdn_tail.h).
//
// Gates: one workgroup per (b, 64-token tile).  The tile of the projection
// output (64 tokens x nG H channels, rows contiguous) is read coalesced,
// activated, and written through an LDS transpose as nG H contiguous
// 64-token runs of the (nG, B, H, T) output; the backward reads the
// cotangent the same way round.
//
// Head norm: a row of d elements is d / 8 lanes holding 8 consecutive
// elements each (one 16-byte load in bf16); the sum of squares is a
// butterfly within those lanes.  The backward also needs
// mean(dout * weight * xhat) per row (same reduction) and the weight
// gradient, summed per workgroup over its rows in LDS and then over the
// workgroups by a second kernel (no atomics: the sum order is fixed).
#include "../../include/gmdn_tail.h"
#include <type_traits>
#include "tile.h"

namespace gmdn {
namespace {

constexpr int GT_TOK = 64;      // tokens per gate tile
constexpr int GT_THREADS = 256;
constexpr int GT_MAXC = 128;    // nG H channels at most
constexpr float GATE_FLOOR = -13.815510557964274f;  // log(1e-6)

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename T>
GMDN_DEV float ld1(const T* p) { return (float)*p; }
template <typename T>
GMDN_DEV void st1(T* p, float x) { *p = (T)x; }

GMDN_DEV float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }
// log sigmoid(x) = min(x, 0) - log(1 + exp(-|x|)), without overflow
GMDN_DEV float log_sigmoidf(float x) { return fminf(x, 0.f) - log1pf(expf(-fabsf(x))); }

template <typename T>
__global__ void __launch_bounds__(GT_THREADS)
gates_fwd(const T* __restrict__ y, float* __restrict__ out, int64_t B, int64_t Tn, int H, int nG) {
  __shared__ float tile[GT_MAXC * (GT_TOK + 1)];
  const int C = nG * H;
  const int64_t tiles = (Tn + GT_TOK - 1) / GT_TOK;
  const int64_t b = blockIdx.x / tiles, t0 = (blockIdx.x % tiles) * GT_TOK;
  const int nt = (int)(Tn - t0 < GT_TOK ? Tn - t0 : GT_TOK);
  for (int e = threadIdx.x; e < nt * C; e += GT_THREADS) {
    const int t = e / C, ch = e % C;
    const float x = ld1(y + (b * Tn + t0 + t) * C + ch);
    tile[ch * (GT_TOK + 1) + t] = ch / H == 1 ? sigmoidf(x) : fmaxf(log_sigmoidf(x), GATE_FLOOR);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < C * GT_TOK; e += GT_THREADS) {
    const int ch = e / GT_TOK, t = e % GT_TOK;
    if (t >= nt) continue;
    const int g = ch / H, h = ch % H;
    out[((g * B + b) * H + h) * Tn + t0 + t] = tile[ch * (GT_TOK + 1) + t];
  }
}

template <typename T>
__global__ void __launch_bounds__(GT_THREADS)
gates_bwd(const T* __restrict__ y, const float* __restrict__ dout, T* __restrict__ dy, int64_t B, int64_t Tn,
          int H, int nG) {
  __shared__ float tile[GT_MAXC * (GT_TOK + 1)];
  const int C = nG * H;
  const int64_t tiles = (Tn + GT_TOK - 1) / GT_TOK;
  const int64_t b = blockIdx.x / tiles, t0 = (blockIdx.x % tiles) * GT_TOK;
  const int nt = (int)(Tn - t0 < GT_TOK ? Tn - t0 : GT_TOK);
  for (int e = threadIdx.x; e < C * GT_TOK; e += GT_THREADS) {
    const int ch = e / GT_TOK, t = e % GT_TOK;
    if (t >= nt) continue;
    const int g = ch / H, h = ch % H;
    tile[ch * (GT_TOK + 1) + t] = dout[((g * B + b) * H + h) * Tn + t0 + t];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nt * C; e += GT_THREADS) {
    const int t = e / C, ch = e % C;
    const int64_t o = (b * Tn + t0 + t) * C + ch;
    const float x = ld1(y + o), s = sigmoidf(x), d = tile[ch * (GT_TOK + 1) + t];
    float dx;
    if (ch / H == 1)
      dx = d * s * (1.f - s);
    else
      dx = log_sigmoidf(x) >= GATE_FLOOR ? d * (1.f - s) : 0.f;
    st1(dy + o, dx);
  }
}

// ------------------------------------------------------------- head norm
constexpr int HN_THREADS = 256;
constexpr int HN_MAXBLK = 1024;  // workgroups of the backward (partial sums)

template <typename T>
struct Vec8;
template <>
struct Vec8<bf16> {
  static GMDN_DEV void load(const bf16* p, float (&x)[8]) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (float)v[j];
  }
  static GMDN_DEV void store(bf16* p, const float (&x)[8]) {
    const bf16x8 v = cat8(to_bf16x4(f32x4{x[0], x[1], x[2], x[3]}), to_bf16x4(f32x4{x[4], x[5], x[6], x[7]}));
    *reinterpret_cast<bf16x8*>(p) = v;
  }
};
template <>
struct Vec8<float> {
  static GMDN_DEV void load(const float* p, float (&x)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), c = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = a[j];
      x[4 + j] = c[j];
    }
  }
  static GMDN_DEV void store(float* p, const float (&x)[8]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
  }
};

// sum over the LPR lanes of a row (aligned groups of LPR lanes)
template <int LPR>
GMDN_DEV float row_sum(float x) {
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) x += __shfl_xor(x, o, 64);
  return x;
}

template <typename T, int D>
__global__ void __launch_bounds__(HN_THREADS)
head_norm_fwd(const T* __restrict__ x, const float* __restrict__ w, T* __restrict__ out, float* __restrict__ rstd,
              int64_t rows, float eps) {
  constexpr int LPR = D / 8, RPB = HN_THREADS / LPR;
  const int lr = threadIdx.x / LPR, q = threadIdx.x % LPR;
  float wv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) wv[j] = w[8 * q + j];
  for (int64_t r = (int64_t)blockIdx.x * RPB + lr; r - lr < rows; r += (int64_t)gridDim.x * RPB) {
    const bool live = r < rows;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) Vec8<T>::load(x + r * D + 8 * q, v);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += v[j] * v[j];
    ss = row_sum<LPR>(ss);
    const float rs = 1.f / sqrtf(ss * (1.f / D) + eps);
    if (!live) continue;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = v[j] * rs * wv[j];
    Vec8<T>::store(out + r * D + 8 * q, v);
    if (q == 0) rstd[r] = rs;
  }
}

template <typename T, int D>
__global__ void __launch_bounds__(HN_THREADS)
head_norm_bwd(const T* __restrict__ x, const float* __restrict__ w, const float* __restrict__ rstd,
              const T* __restrict__ dout, T* __restrict__ dx, float* __restrict__ part, int64_t rows) {
  constexpr int LPR = D / 8, RPB = HN_THREADS / LPR;
  __shared__ float red[RPB][D];
  const int lr = threadIdx.x / LPR, q = threadIdx.x % LPR;
  float wv[8], dw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    wv[j] = w[8 * q + j];
    dw[j] = 0.f;
  }
  for (int64_t r = (int64_t)blockIdx.x * RPB + lr; r - lr < rows; r += (int64_t)gridDim.x * RPB) {
    const bool live = r < rows;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, g[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float rs = 0.f;
    if (live) {
      Vec8<T>::load(x + r * D + 8 * q, v);
      Vec8<T>::load(dout + r * D + 8 * q, g);
      rs = rstd[r];
    }
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] *= rs;                 // xhat
      dw[j] += g[j] * v[j];
      g[j] *= wv[j];              // dout * weight
      dot += g[j] * v[j];
    }
    const float mean = row_sum<LPR>(dot) * (1.f / D);
    if (!live) continue;
#pragma unroll
    for (int j = 0; j < 8; ++j) g[j] = rs * (g[j] - v[j] * mean);
    Vec8<T>::store(dx + r * D + 8 * q, g);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) red[lr][8 * q + j] = dw[j];
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += HN_THREADS) {
    float s = 0.f;
    for (int i = 0; i < RPB; ++i) s += red[i][c];
    part[(int64_t)blockIdx.x * D + c] = s;
  }
}

// dweight[c] = sum over the backward's workgroups of their partial sums.
// Workgroup g sums columns 16 g .. 16 g + 15: 16 threads per column take every
// 16th partial row, four independent sums each (the loads of a round are in
// flight together), combined in a fixed order, then the 16 threads' sums in
// a fixed order: the same bits on every run.
constexpr int HN_DW_COLS = 16;
constexpr int HN_DW_SPLIT = HN_THREADS / HN_DW_COLS;
__global__ void __launch_bounds__(HN_THREADS) head_norm_dw(const float* __restrict__ part, float* __restrict__ dw,
                                                           int d, int nblk) {
  __shared__ float red[HN_DW_SPLIT][HN_DW_COLS];
  const int cl = threadIdx.x % HN_DW_COLS, s = threadIdx.x / HN_DW_COLS;
  const int c = blockIdx.x * HN_DW_COLS + cl;
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
  int i = s;
  for (; i + 3 * HN_DW_SPLIT < nblk; i += 4 * HN_DW_SPLIT) {
    a0 += part[(int64_t)i * d + c];
    a1 += part[(int64_t)(i + HN_DW_SPLIT) * d + c];
    a2 += part[(int64_t)(i + 2 * HN_DW_SPLIT) * d + c];
    a3 += part[(int64_t)(i + 3 * HN_DW_SPLIT) * d + c];
  }
  for (; i < nblk; i += HN_DW_SPLIT) a0 += part[(int64_t)i * d + c];
  red[s][cl] = (a0 + a1) + (a2 + a3);
  __syncthreads();
  if (s == 0) {
    float acc = red[0][cl];
    for (int k = 1; k < HN_DW_SPLIT; ++k) acc += red[k][cl];
    dw[c] = acc;
  }
}

int hn_blocks(int64_t rows, int d) {
  const int64_t rpb = HN_THREADS / (d / 8);
  const int64_t nb = (rows + rpb - 1) / rpb;
  return (int)(nb < HN_MAXBLK ? nb : HN_MAXBLK);
}

int check_gates(const void* y, int64_t B, int64_t T, int32_t H, int32_t nG, int32_t dtype) {
  if (B < 0 || T < 0 || H <= 0 || (nG != 3 && nG != 4) || nG * H > GT_MAXC) return GMDN_ERR_ARG;
  if (dtype != GMDN_DTYPE_BF16 && dtype != GMDN_DTYPE_F32) return GMDN_ERR_UNSUPPORTED;
  if (B * T > ((int64_t)1 << 40)) return GMDN_ERR_ARG;
  if (B * T > 0 && !y) return GMDN_ERR_ARG;
  return GMDN_OK;
}

// head dims of the per-head norm: one row is d / 8 lanes of 8 elements
bool norm_dim(int d) { return d == 16 || d == 32 || d == 64 || d == 128; }

// f(std::integral_constant<int, D>{}) for the built head dims
template <class F>
void with_d(int d, F&& f) {
  switch (d) {
    case 16: f(std::integral_constant<int, 16>{}); break;
    case 32: f(std::integral_constant<int, 32>{}); break;
    case 64: f(std::integral_constant<int, 64>{}); break;
    default: f(std::integral_constant<int, 128>{}); break;
  }
}

int check_norm(const void* x, const float* w, int64_t rows, int32_t d, int32_t dtype) {
  if (rows < 0 || !norm_dim(d)) return rows < 0 ? GMDN_ERR_ARG : GMDN_ERR_UNSUPPORTED;
  if (dtype != GMDN_DTYPE_BF16 && dtype != GMDN_DTYPE_F32) return GMDN_ERR_UNSUPPORTED;
  if (rows > 0 && (!x || !w || !aligned16(x))) return GMDN_ERR_ARG;
  return GMDN_OK;
}

}  // namespace
}  // namespace gmdn

using namespace gmdn;

extern "C" {

int gmdn_gates_fwd(const void* y, float* out, int64_t B, int64_t T, int32_t H, int32_t nG, int32_t dtype,
                   void* stream) {
  int rc = check_gates(y, B, T, H, nG, dtype);
  if (rc != GMDN_OK || B * T == 0) return rc;
  if (!out) return GMDN_ERR_ARG;
  const dim3 grid((unsigned)(B * ((T + GT_TOK - 1) / GT_TOK)));
  const hipStream_t st = (hipStream_t)stream;
  if (dtype == GMDN_DTYPE_BF16)
    hipLaunchKernelGGL(gates_fwd<bf16>, grid, dim3(GT_THREADS), 0, st, (const bf16*)y, out, B, T, H, nG);
  else
    hipLaunchKernelGGL(gates_fwd<float>, grid, dim3(GT_THREADS), 0, st, (const float*)y, out, B, T, H, nG);
  return hipGetLastError() == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

int gmdn_gates_bwd(const void* y, const float* dout, void* dy, int64_t B, int64_t T, int32_t H, int32_t nG,
                   int32_t dtype, void* stream) {
  int rc = check_gates(y, B, T, H, nG, dtype);
  if (rc != GMDN_OK || B * T == 0) return rc;
  if (!dout || !dy) return GMDN_ERR_ARG;
  const dim3 grid((unsigned)(B * ((T + GT_TOK - 1) / GT_TOK)));
  const hipStream_t st = (hipStream_t)stream;
  if (dtype == GMDN_DTYPE_BF16)
    hipLaunchKernelGGL(gates_bwd<bf16>, grid, dim3(GT_THREADS), 0, st, (const bf16*)y, dout, (bf16*)dy, B, T, H,
                       nG);
  else
    hipLaunchKernelGGL(gates_bwd<float>, grid, dim3(GT_THREADS), 0, st, (const float*)y, dout, (float*)dy, B, T,
                       H, nG);
  return hipGetLastError() == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

int gmdn_head_norm_fwd(const void* x, const float* weight, void* out, float* rstd, int64_t rows, int32_t d,
                       float eps, int32_t dtype, void* stream) {
  int rc = check_norm(x, weight, rows, d, dtype);
  if (rc != GMDN_OK || rows == 0) return rc;
  if (!out || !rstd || !aligned16(out) || !(eps >= 0.f)) return GMDN_ERR_ARG;
  const dim3 grid((unsigned)hn_blocks(rows, d));
  const hipStream_t st = (hipStream_t)stream;
  with_d(d, [&](auto c) {
    constexpr int D = decltype(c)::value;
    if (dtype == GMDN_DTYPE_BF16)
      hipLaunchKernelGGL((head_norm_fwd<bf16, D>), grid, dim3(HN_THREADS), 0, st, (const bf16*)x, weight,
                         (bf16*)out, rstd, rows, eps);
    else
      hipLaunchKernelGGL((head_norm_fwd<float, D>), grid, dim3(HN_THREADS), 0, st, (const float*)x, weight,
                         (float*)out, rstd, rows, eps);
  });
  return hipGetLastError() == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

size_t gmdn_head_norm_bwd_workspace_floats(int64_t rows, int32_t d) {
  if (rows <= 0 || !norm_dim(d)) return 0;
  return (size_t)hn_blocks(rows, d) * d;
}

int gmdn_head_norm_bwd(const void* x, const float* weight, const float* rstd, const void* dout, void* dx,
                       float* dweight, float* workspace, size_t workspace_floats, int64_t rows, int32_t d,
                       int32_t dtype, void* stream) {
  int rc = check_norm(x, weight, rows, d, dtype);
  if (rc != GMDN_OK || rows == 0) return rc;
  if (!rstd || !dout || !dx || !dweight || !aligned16(dout) || !aligned16(dx)) return GMDN_ERR_ARG;
  const int nb = hn_blocks(rows, d);
  if (!workspace || workspace_floats < (size_t)nb * d) return GMDN_ERR_WORKSPACE;
  const hipStream_t st = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  with_d(d, [&](auto c) {
    constexpr int D = decltype(c)::value;
    if (dtype == GMDN_DTYPE_BF16)
      hipLaunchKernelGGL((head_norm_bwd<bf16, D>), dim3(nb), dim3(HN_THREADS), 0, st, (const bf16*)x, weight,
                         rstd, (const bf16*)dout, (bf16*)dx, workspace, rows);
    else
      hipLaunchKernelGGL((head_norm_bwd<float, D>), dim3(nb), dim3(HN_THREADS), 0, st, (const float*)x, weight,
                         rstd, (const float*)dout, (float*)dx, workspace, rows);
    e = hipGetLastError();
    if (e == hipSuccess) {
      hipLaunchKernelGGL(head_norm_dw, dim3(D / HN_DW_COLS), dim3(HN_THREADS), 0, st, workspace, dweight, D, nb);
      e = hipGetLastError();
    }
  });
  return e == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

}  // extern "C"
