// Mixer front-end: causal depthwise conv over time + SiLU + per-head L2 norm
// of q and k (reference train_ablation.py:93-94, 124-128), forward and
// backward, with their extern "C" entry points (include/gmdn_front.h).
//
// One wave owns 512 channels of the (B, T, 3 D) projection output -- 8
// consecutive channels per lane, so a row is one 16-byte (bf16) load per
// lane -- over a run of 64 tokens.  The conv's K input rows per output sit
// in a register window that slides one token per step, so every row of y is
// read once; a head's dh channels are dh / 8 consecutive lanes, and its norm
// is a shuffle reduction within them.  The backward recomputes the forward
// from y, carries dz in a 4-token window and emits dy three tokens behind;
// each wave writes its weight- and bias-gradient sums for its tile to a
// partial-sum buffer (no atomics) that the caller reduces.
#include "../../include/gmdn_front.h"
#include "tile.h"

#include <type_traits>

namespace gmdn {
namespace {

constexpr int FT_TOK = 64;                // tokens per wave
constexpr int FT_LC = 8;                  // channels per lane
constexpr int FT_WC = 64 * FT_LC;         // channels per wave
constexpr int FT_WAVES = 4;               // waves per workgroup
constexpr int FT_KMAX = 4;                // conv taps held in the window
constexpr float FT_EPS = 1e-12f;          // F.normalize's eps
constexpr int FT_GF = 8;                  // forward: rows loaded ahead per group
constexpr int FT_GB = 4;                  // backward: tokens (2 rows each) per group

template <typename T>
struct Row8;
template <>
struct Row8<bf16> {
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
struct Row8<float> {
  static GMDN_DEV void load(const float* p, float (&x)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = a[j];
      x[4 + j] = b[j];
    }
  }
  static GMDN_DEV void store(float* p, const float (&x)[8]) {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
  }
};

// A lane's 8 channels of one row as loaded (converted when used), so that
// a group of rows can be in flight at once
template <typename T>
struct Raw8;
template <>
struct Raw8<bf16> {
  bf16x8 v;
  GMDN_DEV void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  GMDN_DEV void zero() { v = bf16x8{}; }
  GMDN_DEV void get(float (&x)[8]) const {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (float)v[j];
  }
};
template <>
struct Raw8<float> {
  f32x4 a, b;
  GMDN_DEV void load(const float* p) {
    a = *reinterpret_cast<const f32x4*>(p);
    b = *reinterpret_cast<const f32x4*>(p + 4);
  }
  GMDN_DEV void zero() { a = b = f32x4{0.f, 0.f, 0.f, 0.f}; }
  GMDN_DEV void get(float (&x)[8]) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = a[j];
      x[4 + j] = b[j];
    }
  }
};

// sum over the dh / 8 lanes of one head, in DPP moves (all lanes of the
// wave take part; a head's lanes are an aligned group since D is a multiple
// of dh): the first quad-permute step sums lane pairs (a 16-wide head), the
// second each quad (32); a 128-wide head is a 16-lane row (row_ror 4 and 8
// add the other quads), a 64-wide head a half-row (row_half_mirror adds the
// other quad of the 8)
template <int DH>
GMDN_DEV float head_sum(float s) {
  static_assert(DH == 16 || DH == 32 || DH == 64 || DH == 128, "head dims 16, 32, 64 and 128");
  s += dpp_mov<0xB1>(s);  // quad_perm [1,0,3,2]
  if constexpr (DH >= 32) s += dpp_mov<0x4E>(s);  // quad_perm [2,3,0,1]
  if constexpr (DH == 64) {
    s += dpp_mov<0x141>(s);  // row_half_mirror
  } else if constexpr (DH == 128) {
    s += dpp_mov<0x124>(s);  // row_ror:4
    s += dpp_mov<0x128>(s);  // row_ror:8
  }
  return s;
}

// Per-lane view of its 8 channels: which output (0 q, 1 k, 2 v), the
// channel within it, and the conv taps aligned to the 4-row window (slot s
// holds y[t - 3 + s]; tap i of K sits at slot i + 4 - K).
struct Lane {
  int c0, part, cc;
  bool on;
  float wr[FT_LC][FT_KMAX], br[FT_LC];
  GMDN_DEV Lane(int chunk, int C3, int D, int K, const float* w, const float* bias) {
    c0 = chunk * FT_WC + FT_LC * (threadIdx.x & 63);
    on = c0 < C3;
    part = on ? c0 / D : 0;
    cc = c0 - part * D;
    if (on && K == FT_KMAX) {  // the common kernel size: one 16-byte load per channel
#pragma unroll
      for (int j = 0; j < FT_LC; ++j) {
        const f32x4 r = *reinterpret_cast<const f32x4*>(w + (int64_t)(c0 + j) * FT_KMAX);
#pragma unroll
        for (int s = 0; s < FT_KMAX; ++s) wr[j][s] = r[s];
      }
    } else {
#pragma unroll
      for (int j = 0; j < FT_LC; ++j)
#pragma unroll
        for (int s = 0; s < FT_KMAX; ++s) {
          const int i = s - (FT_KMAX - K);
          wr[j][s] = (on && i >= 0) ? w[(int64_t)(c0 + j) * K + i] : 0.f;
        }
    }
    if (on) {
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(bias + c0), b1 = *reinterpret_cast<const f32x4*>(bias + c0 + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        br[j] = b0[j];
        br[4 + j] = b1[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < FT_LC; ++j) br[j] = 0.f;
    }
  }
};

template <typename T, int DH>
__global__ void __launch_bounds__(64 * FT_WAVES)
front_fwd(const T* __restrict__ y, const float* __restrict__ w, const float* __restrict__ bias,
          T* __restrict__ q, T* __restrict__ k, T* __restrict__ v, int T_, int D, int K) {
  const int C3 = 3 * D;
  const int ntiles = (T_ + FT_TOK - 1) / FT_TOK;
  const int64_t b = blockIdx.x / ntiles;
  const int t0 = (int)(blockIdx.x % ntiles) * FT_TOK;
  const Lane ln(blockIdx.y * FT_WAVES + (threadIdx.x >> 6), C3, D, K, w, bias);
  T* dst = (ln.part == 0 ? q : ln.part == 1 ? k : v) + b * T_ * (int64_t)D + ln.cc;
  const T* yb = y + b * T_ * (int64_t)C3 + ln.c0;
  const bool norm = ln.part < 2;

  float win[FT_KMAX - 1][FT_LC];
#pragma unroll
  for (int s = 0; s < FT_KMAX - 1; ++s) {
    const int t = t0 - (FT_KMAX - 1) + s;
    if (ln.on && t >= 0) {
      Row8<T>::load(yb + (int64_t)t * C3, win[s]);
    } else {
#pragma unroll
      for (int j = 0; j < FT_LC; ++j) win[s][j] = 0.f;
    }
  }
  const int t1 = min(t0 + FT_TOK, T_);
  for (int tg = t0; tg < t1; tg += FT_GF) {
    // the group's rows in flight together, then the tokens in order
    Raw8<T> rows[FT_GF];
#pragma unroll
    for (int g = 0; g < FT_GF; ++g) {
      if (ln.on && tg + g < t1)
        rows[g].load(yb + (int64_t)(tg + g) * C3);
      else
        rows[g].zero();
    }
#pragma unroll
    for (int g = 0; g < FT_GF; ++g) {
    const int t = tg + g;
    float cur[FT_LC], a[FT_LC];
    rows[g].get(cur);
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < FT_LC; ++j) {
      const float z = ln.br[j] + ln.wr[j][0] * win[0][j] + ln.wr[j][1] * win[1][j] + ln.wr[j][2] * win[2][j] +
                      ln.wr[j][3] * cur[j];
      a[j] = z * __builtin_amdgcn_rcpf(1.f + __expf(-z));  // silu, v_rcp_f32 (1 ulp)
      ss += a[j] * a[j];
    }
    ss = head_sum<DH>(ss);
    const float sc = norm ? __builtin_amdgcn_rcpf(fmaxf(sqrtf(ss), FT_EPS)) : 1.f;
#pragma unroll
    for (int j = 0; j < FT_LC; ++j) a[j] *= sc;
    if (ln.on && t < t1) Row8<T>::store(dst + (int64_t)t * D, a);
#pragma unroll
    for (int j = 0; j < FT_LC; ++j) {
      win[0][j] = win[1][j];
      win[1][j] = win[2][j];
      win[2][j] = cur[j];
    }
    }
  }
}

template <typename T, int DH>
__global__ void __launch_bounds__(64 * FT_WAVES)
front_bwd(const T* __restrict__ y, const float* __restrict__ w, const float* __restrict__ bias,
          const T* __restrict__ dq, const T* __restrict__ dk, const T* __restrict__ dv, T* __restrict__ dy,
          float* __restrict__ partial, int T_, int D, int K) {
  const int C3 = 3 * D;
  const int ntiles = (T_ + FT_TOK - 1) / FT_TOK;
  const int64_t b = blockIdx.x / ntiles;
  const int t0 = (int)(blockIdx.x % ntiles) * FT_TOK;
  const Lane ln(blockIdx.y * FT_WAVES + (threadIdx.x >> 6), C3, D, K, w, bias);
  const T* gb = (ln.part == 0 ? dq : ln.part == 1 ? dk : dv) + b * T_ * (int64_t)D + ln.cc;
  const T* yb = y + b * T_ * (int64_t)C3 + ln.c0;
  T* dyb = dy + b * T_ * (int64_t)C3 + ln.c0;
  const bool norm = ln.part < 2;

  float win[FT_KMAX - 1][FT_LC], dzw[FT_KMAX - 1][FT_LC], acc[FT_LC][FT_KMAX + 1];
#pragma unroll
  for (int s = 0; s < FT_KMAX - 1; ++s) {
    const int t = t0 - (FT_KMAX - 1) + s;
    if (ln.on && t >= 0) {
      Row8<T>::load(yb + (int64_t)t * C3, win[s]);
    } else {
#pragma unroll
      for (int j = 0; j < FT_LC; ++j) win[s][j] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < FT_LC; ++j) dzw[s][j] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < FT_LC; ++j)
#pragma unroll
    for (int s = 0; s <= FT_KMAX; ++s) acc[j][s] = 0.f;

  // tokens t0 .. t0 + 66: the tile's own dz, then the 3 after it that its
  // last dy rows need (zero beyond T)
  constexpr int NT_B = FT_TOK + FT_KMAX - 1;
  for (int tg = t0; tg < t0 + NT_B; tg += FT_GB) {
    Raw8<T> ry[FT_GB], rg[FT_GB];
#pragma unroll
    for (int g = 0; g < FT_GB; ++g) {
      const int t = tg + g;
      if (ln.on && t < T_ && t < t0 + NT_B) {
        ry[g].load(yb + (int64_t)t * C3);
        rg[g].load(gb + (int64_t)t * D);
      } else {
        ry[g].zero();
        rg[g].zero();
      }
    }
#pragma unroll
    for (int g = 0; g < FT_GB; ++g) {
    const int t = tg + g;
    const bool tv = t < T_ && t < t0 + NT_B;
    float cur[FT_LC], du[FT_LC];
    ry[g].get(cur);
    rg[g].get(du);
    float z[FT_LC], sg[FT_LC], a[FT_LC], ss = 0.f, sd = 0.f;
#pragma unroll
    for (int j = 0; j < FT_LC; ++j) {
      z[j] = ln.br[j] + ln.wr[j][0] * win[0][j] + ln.wr[j][1] * win[1][j] + ln.wr[j][2] * win[2][j] +
             ln.wr[j][3] * cur[j];
      sg[j] = __builtin_amdgcn_rcpf(1.f + __expf(-z[j]));
      a[j] = z[j] * sg[j];
      ss += a[j] * a[j];
      sd += a[j] * du[j];
    }
    ss = head_sum<DH>(ss);
    sd = head_sum<DH>(sd);
    float dz[FT_LC];
    {
      // F.normalize's backward: with n = |a|, u = a / n,
      // da = (du - u (u . du)) / n for n > eps, da = du / eps otherwise
      const float n = sqrtf(ss);
      const bool big = n > FT_EPS;
      const float inv = big ? __builtin_amdgcn_rcpf(n) : 1.f / FT_EPS;
      const float ud = big ? sd * inv : 0.f;
#pragma unroll
      for (int j = 0; j < FT_LC; ++j) {
        const float da = norm ? (du[j] - a[j] * inv * ud) * inv : du[j];
        // silu'(z) = s (1 + z (1 - s))
        dz[j] = tv ? da * sg[j] * (1.f + z[j] * (1.f - sg[j])) : 0.f;
      }
    }
    if (t < t0 + FT_TOK && tv) {
#pragma unroll
      for (int j = 0; j < FT_LC; ++j) {
        acc[j][0] += dz[j] * win[0][j];
        acc[j][1] += dz[j] * win[1][j];
        acc[j][2] += dz[j] * win[2][j];
        acc[j][3] += dz[j] * cur[j];
        acc[j][4] += dz[j];
      }
    }
    // dy[s] = sum over the taps of w (slot) dz[s + 3 - slot], complete at t = s + 3
    const int s = t - (FT_KMAX - 1);
    if (ln.on && s >= t0 && s < t0 + FT_TOK && s < T_) {  // only the tile's own rows
      float g[FT_LC];
#pragma unroll
      for (int j = 0; j < FT_LC; ++j)
        g[j] = ln.wr[j][3] * dzw[0][j] + ln.wr[j][2] * dzw[1][j] + ln.wr[j][1] * dzw[2][j] + ln.wr[j][0] * dz[j];
      Row8<T>::store(dyb + (int64_t)s * C3, g);
    }
#pragma unroll
    for (int j = 0; j < FT_LC; ++j) {
      win[0][j] = win[1][j];
      win[1][j] = win[2][j];
      win[2][j] = cur[j];
      dzw[0][j] = dzw[1][j];
      dzw[1][j] = dzw[2][j];
      dzw[2][j] = dz[j];
    }
    }
  }
  if (ln.on) {
    // partial[(b, tile)][channel][K taps, bias]
    float* pp = partial + ((int64_t)blockIdx.x * C3 + ln.c0) * (K + 1);
#pragma unroll
    for (int j = 0; j < FT_LC; ++j) {
#pragma unroll
      for (int s = 0; s < FT_KMAX; ++s)  // window slot s holds tap s - (4 - K)
        if (s >= FT_KMAX - K) pp[j * (K + 1) + s - (FT_KMAX - K)] = acc[j][s];
      pp[j * (K + 1) + K] = acc[j][FT_KMAX];
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int check_front(const void* y, const float* w, const float* bias, int64_t B, int64_t T, int32_t D, int32_t dh,
                int32_t K, int32_t dtype) {
  if (B < 0 || T < 0 || D <= 0 || K < 1 || K > FT_KMAX) return GMDN_ERR_ARG;
  if (dh != 16 && dh != 32 && dh != 64 && dh != 128) return GMDN_ERR_UNSUPPORTED;
  if (D % dh) return GMDN_ERR_ARG;
  if (dtype != GMDN_DTYPE_BF16 && dtype != GMDN_DTYPE_F32) return GMDN_ERR_UNSUPPORTED;
  if (B * T == 0) return GMDN_OK;
  if (B * T > ((int64_t)1 << 31) / 3 || (int64_t)D * 3 > (1 << 24)) return GMDN_ERR_ARG;
  if (!y || !w || !bias || !aligned16(y) || !aligned16(w) || !aligned16(bias)) return GMDN_ERR_ARG;
  return GMDN_OK;
}

template <typename T, int DH>
hipError_t launch_fwd(const void* y, const float* w, const float* bias, void* q, void* k, void* v, int64_t B,
                      int64_t T_, int32_t D, int32_t K, hipStream_t st) {
  const int ntiles = (int)((T_ + FT_TOK - 1) / FT_TOK);
  const int nchunks = (3 * D + FT_WC - 1) / FT_WC;
  const dim3 grid((unsigned)(B * ntiles), (unsigned)((nchunks + FT_WAVES - 1) / FT_WAVES));
  hipLaunchKernelGGL((front_fwd<T, DH>), grid, dim3(64 * FT_WAVES), 0, st, static_cast<const T*>(y), w, bias,
                     static_cast<T*>(q), static_cast<T*>(k), static_cast<T*>(v), (int)T_, D, K);
  return hipGetLastError();
}

template <typename T, int DH>
hipError_t launch_bwd(const void* y, const float* w, const float* bias, const void* dq, const void* dk,
                      const void* dv, void* dy, float* partial, int64_t B, int64_t T_, int32_t D, int32_t K,
                      hipStream_t st) {
  const int ntiles = (int)((T_ + FT_TOK - 1) / FT_TOK);
  const int nchunks = (3 * D + FT_WC - 1) / FT_WC;
  const dim3 grid((unsigned)(B * ntiles), (unsigned)((nchunks + FT_WAVES - 1) / FT_WAVES));
  hipLaunchKernelGGL((front_bwd<T, DH>), grid, dim3(64 * FT_WAVES), 0, st, static_cast<const T*>(y), w, bias,
                     static_cast<const T*>(dq), static_cast<const T*>(dk), static_cast<const T*>(dv),
                     static_cast<T*>(dy), partial, (int)T_, D, K);
  return hipGetLastError();
}

// f(std::integral_constant<int, DH>{}) for the built head dims
template <class F>
hipError_t with_dh(int dh, F&& f) {
  switch (dh) {
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, 64>{});
    default: return f(std::integral_constant<int, 128>{});
  }
}

}  // namespace
}  // namespace gmdn

using namespace gmdn;

extern "C" {

int gmdn_front_fwd(const void* y, const float* weight, const float* bias, void* q, void* k, void* v, int64_t B,
                   int64_t T, int32_t D, int32_t dh, int32_t K, int32_t dtype, void* stream) {
  int rc = check_front(y, weight, bias, B, T, D, dh, K, dtype);
  if (rc != GMDN_OK || B * T == 0) return rc;
  if (!q || !k || !v || !aligned16(q) || !aligned16(k) || !aligned16(v)) return GMDN_ERR_ARG;
  const hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  e = with_dh(dh, [&](auto c) {
    constexpr int DH = decltype(c)::value;
    return dtype == GMDN_DTYPE_BF16 ? launch_fwd<bf16, DH>(y, weight, bias, q, k, v, B, T, D, K, st)
                                    : launch_fwd<float, DH>(y, weight, bias, q, k, v, B, T, D, K, st);
  });
  return e == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

size_t gmdn_front_bwd_workspace_floats(int64_t B, int64_t T, int32_t D, int32_t K) {
  if (B <= 0 || T <= 0 || D <= 0 || K < 1) return 0;
  return (size_t)(B * ((T + FT_TOK - 1) / FT_TOK)) * (size_t)(3 * D) * (size_t)(K + 1);
}

int gmdn_front_bwd(const void* y, const float* weight, const float* bias, const void* dq, const void* dk,
                   const void* dv, void* dy, float* partial, int64_t B, int64_t T, int32_t D, int32_t dh, int32_t K,
                   int32_t dtype, void* stream) {
  int rc = check_front(y, weight, bias, B, T, D, dh, K, dtype);
  if (rc != GMDN_OK || B * T == 0) return rc;
  if (!dq || !dk || !dv || !dy || !partial) return GMDN_ERR_ARG;
  if (!aligned16(dq) || !aligned16(dk) || !aligned16(dv) || !aligned16(dy)) return GMDN_ERR_ARG;
  const hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  e = with_dh(dh, [&](auto c) {
    constexpr int DH = decltype(c)::value;
    return dtype == GMDN_DTYPE_BF16 ? launch_bwd<bf16, DH>(y, weight, bias, dq, dk, dv, dy, partial, B, T, D, K, st)
                                    : launch_bwd<float, DH>(y, weight, bias, dq, dk, dv, dy, partial, B, T, D, K, st);
  });
  return e == hipSuccess ? GMDN_OK : GMDN_ERR_LAUNCH;
}

}  // extern "C"
