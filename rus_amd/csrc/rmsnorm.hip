// Residual + RMSNorm forward and its one-pass backward for gfx950.
//
// Behaviour follows solution/kernels.py:125-199 (rms_norm_residual_fwd_kernel,
// rms_norm_bwd_kernel) with the cast order of Qwen2RMSNorm: h = T(x + res), fp32 statistics,
// y = T(fp32(T(h * rstd)) * w). Design (CDNA4, wave64):
//   * one wavefront owns one row; each lane moves 16-byte packs (8 x fp16 or 4 x fp32), so a
//     1536-wide fp16 row is 3 fully coalesced 1 KiB wave accesses per tensor; the packs stay in
//     registers between the sum-of-squares reduction and the normalisation, so every input byte
//     is read from HBM once and each output byte written once;
//   * the row reduction is a 64-lane butterfly (no LDS, no block barrier);
//   * rows narrower than NIT*64*pack or with a width that is not a multiple of the pack fall back
//     to a scalar two-pass kernel (the second pass re-reads the row from L1/L2, not HBM);
//   * built with -ffp-contract=off so every product and sum is rounded as in an eager fp32
//     restatement (only the reduction order differs).
#include <type_traits>

#include "common.h"
#include "rmsnorm_rows.h"

namespace rus {
namespace {

template <typename T, typename W, int NIT, bool HAS_RES>
__global__ __launch_bounds__(256) void rmsnorm_fwd_vec(const T* __restrict__ x,
                                                      const T* __restrict__ res,
                                                      const W* __restrict__ w,
                                                      T* __restrict__ sum_out, T* __restrict__ y,
                                                      float* __restrict__ rstd, int n_rows,
                                                      int n_cols, int64_t stride, float eps) {
  rmsnorm_fwd_row<T, W, NIT, HAS_RES>(x, res, w, sum_out, y, rstd,
                                      blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave,
                                      n_rows, n_cols, stride, eps);
}

// Scalar two-pass fallback for any width.
template <typename T, typename W, bool HAS_RES>
__global__ __launch_bounds__(256) void rmsnorm_fwd_any(const T* __restrict__ x,
                                                      const T* __restrict__ res,
                                                      const W* __restrict__ w, T* sum_out,
                                                      T* __restrict__ y, float* __restrict__ rstd,
                                                      int n_rows, int n_cols, int64_t stride,
                                                      float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int64_t off = static_cast<int64_t>(row) * stride;
  float ss = 0.0f;
  for (int c = lane; c < n_cols; c += kWave) {
    float h = static_cast<float>(x[off + c]);
    if (HAS_RES) {
      h = round_to<T>(h + static_cast<float>(res[off + c]));
      sum_out[off + c] = from_f32<T>(h);
    }
    ss += h * h;
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(n_cols) + eps);
  if (lane == 0) rstd[row] = r;
  const T* hsrc = HAS_RES ? sum_out : x;  // this lane wrote these sum_out elements itself
  for (int c = lane; c < n_cols; c += kWave) {
    const float h = static_cast<float>(hsrc[off + c]);
    y[off + c] = from_f32<T>(round_to<T>(h * r) * static_cast<float>(w[c]));
  }
}

template <typename T, typename W, int NIT, bool HAS_DRES>
__global__ __launch_bounds__(256) void rmsnorm_bwd_vec(const T* __restrict__ dy,
                                                      const T* __restrict__ h,
                                                      const W* __restrict__ w,
                                                      const float* __restrict__ rstd,
                                                      const T* __restrict__ dres,
                                                      T* __restrict__ dx, int n_rows, int n_cols,
                                                      int64_t stride) {
  rmsnorm_bwd_row<T, W, NIT, HAS_DRES>(dy, h, w, rstd, dres, dx,
                                       blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave,
                                       n_rows, n_cols, stride);
}

// rmsnorm_bwd_vec whose dy is the fp16 rounding of the sum of n_parts fp32 partial products
// (parts [n_parts, n_rows, n_cols], added in part order): the split-K MLP-backward product
// (d_norm2 = gu W_gu) feeds the norm backward without a separate reduce launch, with the values
// that launch would have written.
template <typename W, int NIT, int NP, bool HAS_DRES>
__global__ __launch_bounds__(256) void rmsnorm_bwd_parts_vec(
    const float* __restrict__ parts, int64_t part_stride, const f16* __restrict__ h,
    const W* __restrict__ w, const float* __restrict__ rstd, const f16* __restrict__ dres,
    f16* __restrict__ dx, int n_rows, int n_cols, int64_t stride) {
  constexpr int V = 8;
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int64_t off = static_cast<int64_t>(row) * stride;
  const float* prow = parts + static_cast<int64_t>(row) * n_cols;
  const float r = rstd[row];

  float xh[NIT][V], g[NIT][V];
  float acc = 0.0f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int c = (it * kWave + lane) * V;
    if (c < n_cols) {
      float dv[V], wv[V], pv[NP][V];
      load_f32<f16, V>(h + off + c, xh[it]);
#pragma unroll
      for (int q = 0; q < NP; ++q) load_f32<float, V>(prow + q * part_stride + c, pv[q]);
      load16<W, V>(w + c, wv);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        dv[i] = pv[0][i];
#pragma unroll
        for (int q = 1; q < NP; ++q) dv[i] += pv[q][i];  // part order
      }
#pragma unroll
      for (int i = 0; i < V; ++i) {
        dv[i] = round_to<f16>(dv[i]);  // the fp16 product the reduce would have written
        xh[it][i] = xh[it][i] * r;
        g[it][i] = wv[i] * dv[i];
        acc += xh[it][i] * g[it][i];
      }
    }
  }
  const float cm = wave_sum(acc) / static_cast<float>(n_cols);
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int c = (it * kWave + lane) * V;
    if (c < n_cols) {
      float o[V];
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = (g[it][i] - xh[it][i] * cm) * r;
      if (HAS_DRES) {
        float d[V];
        load_f32<f16, V>(dres + off + c, d);
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = o[i] + d[i];
      }
      store_from_f32<f16, V>(dx + off + c, o);
    }
  }
}

template <typename T, typename W, bool HAS_DRES>
__global__ __launch_bounds__(256) void rmsnorm_bwd_any(const T* __restrict__ dy,
                                                      const T* __restrict__ h,
                                                      const W* __restrict__ w,
                                                      const float* __restrict__ rstd,
                                                      const T* __restrict__ dres,
                                                      T* __restrict__ dx, int n_rows, int n_cols,
                                                      int64_t stride) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  if (row >= n_rows) return;
  const int64_t off = static_cast<int64_t>(row) * stride;
  const float r = rstd[row];
  float acc = 0.0f;
  for (int c = lane; c < n_cols; c += kWave) {
    const float xh = static_cast<float>(h[off + c]) * r;
    const float g = static_cast<float>(w[c]) * static_cast<float>(dy[off + c]);
    acc += xh * g;
  }
  const float cm = wave_sum(acc) / static_cast<float>(n_cols);
  for (int c = lane; c < n_cols; c += kWave) {
    const float xh = static_cast<float>(h[off + c]) * r;
    const float g = static_cast<float>(w[c]) * static_cast<float>(dy[off + c]);
    float o = (g - xh * cm) * r;
    if (HAS_DRES) o = o + static_cast<float>(dres[off + c]);
    dx[off + c] = from_f32<T>(o);
  }
}

// Iteration counts instantiated for the register-resident path (row width <= NIT*64*pack).
constexpr int kNitChoices[] = {1, 2, 3, 4, 6, 8, 12, 16};

int pick_nit(int64_t n_cols, int pack, int max_nit) {
  for (int nit : kNitChoices) {
    if (nit > max_nit) break;
    if (n_cols <= static_cast<int64_t>(nit) * kWave * pack) return nit;
  }
  return 0;
}

struct Launch {
  dim3 grid, block;
};

Launch row_launch(int64_t n_rows) {
  // Four rows (waves) per workgroup once there are enough rows to fill every CU several times;
  // otherwise one row per workgroup so that small batches still spread over all 256 CUs.
  const int rows_per_block = n_rows >= 4096 ? 4 : 1;
  Launch l;
  l.block = dim3(kWave * rows_per_block);
  l.grid = dim3(static_cast<unsigned>((n_rows + rows_per_block - 1) / rows_per_block));
  return l;
}

template <typename T, typename W>
int fwd_typed(const void* x, const void* res, const void* w, void* sum_out, void* y, float* rstd,
              int64_t n_rows, int64_t n_cols, int64_t stride, float eps, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const T* xp = static_cast<const T*>(x);
  const T* rp = static_cast<const T*>(res);
  const W* wp = static_cast<const W*>(w);
  T* sp = static_cast<T*>(sum_out);
  T* yp = static_cast<T*>(y);
  const Launch l = row_launch(n_rows);
  const bool vec_ok = n_cols % V == 0 && stride % V == 0 && aligned(x, 16) && aligned(y, 16) &&
                      aligned(w, 16) && (!res || (aligned(res, 16) && aligned(sum_out, 16)));
  const int nit = vec_ok ? pick_nit(n_cols, V, 16) : 0;
  const int nr = static_cast<int>(n_rows), nc = static_cast<int>(n_cols);
#define RUS_FWD_VEC(NIT)                                                                      \
  case NIT:                                                                                   \
    if (res)                                                                                  \
      hipLaunchKernelGGL((rmsnorm_fwd_vec<T, W, NIT, true>), l.grid, l.block, 0, st, xp, rp,  \
                         wp, sp, yp, rstd, nr, nc, stride, eps);                              \
    else                                                                                      \
      hipLaunchKernelGGL((rmsnorm_fwd_vec<T, W, NIT, false>), l.grid, l.block, 0, st, xp, rp, \
                         wp, sp, yp, rstd, nr, nc, stride, eps);                              \
    break;
  switch (nit) {
    RUS_FWD_VEC(1)
    RUS_FWD_VEC(2)
    RUS_FWD_VEC(3)
    RUS_FWD_VEC(4)
    RUS_FWD_VEC(6)
    RUS_FWD_VEC(8)
    RUS_FWD_VEC(12)
    RUS_FWD_VEC(16)
    default:
      if (res)
        hipLaunchKernelGGL((rmsnorm_fwd_any<T, W, true>), l.grid, l.block, 0, st, xp, rp, wp, sp,
                           yp, rstd, nr, nc, stride, eps);
      else
        hipLaunchKernelGGL((rmsnorm_fwd_any<T, W, false>), l.grid, l.block, 0, st, xp, rp, wp,
                           sp, yp, rstd, nr, nc, stride, eps);
  }
#undef RUS_FWD_VEC
  return check_launch("rus_rmsnorm_fwd");
}

template <typename T, typename W>
int bwd_typed(const void* dy, const void* h, const void* w, const float* rstd, const void* dres,
              void* dx, int64_t n_rows, int64_t n_cols, int64_t stride, hipStream_t st) {
  constexpr int V = 16 / sizeof(T);
  const T* dyp = static_cast<const T*>(dy);
  const T* hp = static_cast<const T*>(h);
  const W* wp = static_cast<const W*>(w);
  const T* dp = static_cast<const T*>(dres);
  T* dxp = static_cast<T*>(dx);
  const Launch l = row_launch(n_rows);
  const bool vec_ok = n_cols % V == 0 && stride % V == 0 && aligned(dy, 16) && aligned(h, 16) &&
                      aligned(w, 16) && aligned(dx, 16) && (!dres || aligned(dres, 16));
  // Two register-resident arrays per lane: cap the width so they stay within the VGPR budget.
  const int nit = vec_ok ? pick_nit(n_cols, V, 8) : 0;
  const int nr = static_cast<int>(n_rows), nc = static_cast<int>(n_cols);
#define RUS_BWD_VEC(NIT)                                                                      \
  case NIT:                                                                                   \
    if (dres)                                                                                 \
      hipLaunchKernelGGL((rmsnorm_bwd_vec<T, W, NIT, true>), l.grid, l.block, 0, st, dyp, hp, \
                         wp, rstd, dp, dxp, nr, nc, stride);                                  \
    else                                                                                      \
      hipLaunchKernelGGL((rmsnorm_bwd_vec<T, W, NIT, false>), l.grid, l.block, 0, st, dyp,    \
                         hp, wp, rstd, dp, dxp, nr, nc, stride);                              \
    break;
  switch (nit) {
    RUS_BWD_VEC(1)
    RUS_BWD_VEC(2)
    RUS_BWD_VEC(3)
    RUS_BWD_VEC(4)
    RUS_BWD_VEC(6)
    RUS_BWD_VEC(8)
    default:
      if (dres)
        hipLaunchKernelGGL((rmsnorm_bwd_any<T, W, true>), l.grid, l.block, 0, st, dyp, hp, wp,
                           rstd, dp, dxp, nr, nc, stride);
      else
        hipLaunchKernelGGL((rmsnorm_bwd_any<T, W, false>), l.grid, l.block, 0, st, dyp, hp, wp,
                           rstd, dp, dxp, nr, nc, stride);
  }
#undef RUS_BWD_VEC
  return check_launch("rus_rmsnorm_bwd");
}

int check_common(const char* fn, int64_t n_rows, int64_t n_cols, int64_t stride, int32_t dtype,
                 int32_t w_dtype) {
  if (n_rows < 0 || n_cols <= 0 || n_rows >= (int64_t(1) << 31) || n_cols >= (int64_t(1) << 30))
    return fail(RUS_ERR_INVALID, "%s: bad shape [%lld, %lld]", fn, (long long)n_rows,
                (long long)n_cols);
  if (stride < n_cols)
    return fail(RUS_ERR_INVALID, "%s: stride_row %lld < n_cols %lld", fn, (long long)stride,
                (long long)n_cols);
  if ((dtype != RUS_DTYPE_F16 && dtype != RUS_DTYPE_F32) ||
      (w_dtype != RUS_DTYPE_F16 && w_dtype != RUS_DTYPE_F32))
    return fail(RUS_ERR_INVALID, "%s: dtype %d / w_dtype %d not fp16(0)/fp32(1)", fn, dtype,
                w_dtype);
  return RUS_OK;
}

}  // namespace
}  // namespace rus

extern "C" int rus_rmsnorm_fwd(const void* x, const void* residual, const void* weight,
                               int32_t w_dtype, void* sum_out, void* y, float* rstd,
                               int64_t n_rows, int64_t n_cols, int64_t stride_row, float eps,
                               int32_t dtype, void* stream) {
  using namespace rus;
  if (int e = check_common("rus_rmsnorm_fwd", n_rows, n_cols, stride_row, dtype, w_dtype)) return e;
  if (n_rows == 0) return RUS_OK;
  if (!x || !weight || !y || !rstd || (residual && !sum_out))
    return fail(RUS_ERR_INVALID, "rus_rmsnorm_fwd: null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RUS_DTYPE_F16) {
    if (w_dtype == RUS_DTYPE_F16)
      return fwd_typed<f16, f16>(x, residual, weight, sum_out, y, rstd, n_rows, n_cols,
                                 stride_row, eps, st);
    return fwd_typed<f16, float>(x, residual, weight, sum_out, y, rstd, n_rows, n_cols,
                                 stride_row, eps, st);
  }
  if (w_dtype == RUS_DTYPE_F16)
    return fwd_typed<float, f16>(x, residual, weight, sum_out, y, rstd, n_rows, n_cols,
                                 stride_row, eps, st);
  return fwd_typed<float, float>(x, residual, weight, sum_out, y, rstd, n_rows, n_cols,
                                 stride_row, eps, st);
}

extern "C" int rus_rmsnorm_bwd_parts(const float* dy_parts, int32_t n_parts, const void* h,
                                     const void* weight, int32_t w_dtype, const float* rstd,
                                     const void* dresidual, void* dx, int64_t n_rows,
                                     int64_t n_cols, int64_t stride_row, void* stream) {
  using namespace rus;
  const char* fn = "rus_rmsnorm_bwd_parts";
  if (int e = check_common(fn, n_rows, n_cols, stride_row, RUS_DTYPE_F16, w_dtype)) return e;
  if (n_parts < 1 || n_parts > 8)
    return fail(RUS_ERR_INVALID, "%s: n_parts=%d outside [1, 8]", fn, n_parts);
  if (n_rows == 0) return RUS_OK;
  if (!dy_parts || !h || !weight || !rstd || !dx)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_cols % 8 || stride_row % 8 || !aligned(dy_parts, 16) || !aligned(h, 16) ||
      !aligned(weight, 16) || !aligned(dx, 16) || (dresidual && !aligned(dresidual, 16)))
    return fail(RUS_ERR_INVALID, "%s: need n_cols and stride_row multiples of 8 and 16-byte "
                "aligned operands", fn);
  const int nit = pick_nit(n_cols, 8, 8);
  if (nit == 0 || nit * kWave * 8 < n_cols)
    return fail(RUS_ERR_UNSUPPORTED, "%s: n_cols=%lld too wide", fn, (long long)n_cols);
  const int64_t pstride = n_rows * n_cols;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const Launch l = row_launch(n_rows);
  const f16* hp = static_cast<const f16*>(h);
  const f16* dp = static_cast<const f16*>(dresidual);
  f16* dxp = static_cast<f16*>(dx);
  const int nr = static_cast<int>(n_rows), nc = static_cast<int>(n_cols);
  // Parts count and width are compile-time so that every load of a row is issued together.
  auto launch = [&](auto wtag, auto nit_c, auto np_c) {
    using WT = decltype(wtag);
    constexpr int NIT = decltype(nit_c)::value, NP = decltype(np_c)::value;
    if (dp)
      hipLaunchKernelGGL((rmsnorm_bwd_parts_vec<WT, NIT, NP, true>), l.grid, l.block, 0, st,
                         dy_parts, pstride, hp, static_cast<const WT*>(weight), rstd, dp, dxp, nr,
                         nc, stride_row);
    else
      hipLaunchKernelGGL((rmsnorm_bwd_parts_vec<WT, NIT, NP, false>), l.grid, l.block, 0, st,
                         dy_parts, pstride, hp, static_cast<const WT*>(weight), rstd, dp, dxp, nr,
                         nc, stride_row);
  };
  auto by_parts = [&](auto wtag, auto nit_c) {
    switch (n_parts) {
      case 1: launch(wtag, nit_c, std::integral_constant<int, 1>{}); break;
      case 2: launch(wtag, nit_c, std::integral_constant<int, 2>{}); break;
      case 3: launch(wtag, nit_c, std::integral_constant<int, 3>{}); break;
      case 4: launch(wtag, nit_c, std::integral_constant<int, 4>{}); break;
      case 5: launch(wtag, nit_c, std::integral_constant<int, 5>{}); break;
      case 6: launch(wtag, nit_c, std::integral_constant<int, 6>{}); break;
      case 7: launch(wtag, nit_c, std::integral_constant<int, 7>{}); break;
      default: launch(wtag, nit_c, std::integral_constant<int, 8>{}); break;
    }
  };
  auto by_width = [&](auto wtag) {
    switch (nit) {
      case 1: by_parts(wtag, std::integral_constant<int, 1>{}); return true;
      case 2: by_parts(wtag, std::integral_constant<int, 2>{}); return true;
      case 3: by_parts(wtag, std::integral_constant<int, 3>{}); return true;
      case 4: by_parts(wtag, std::integral_constant<int, 4>{}); return true;
      case 6: by_parts(wtag, std::integral_constant<int, 6>{}); return true;
      case 8: by_parts(wtag, std::integral_constant<int, 8>{}); return true;
      default: return false;
    }
  };
  const bool ok = w_dtype == RUS_DTYPE_F16 ? by_width(f16{}) : by_width(float{});
  if (!ok) return fail(RUS_ERR_UNSUPPORTED, "%s: n_cols=%lld unsupported", fn, (long long)n_cols);
  return check_launch(fn);
}

extern "C" int rus_rmsnorm_bwd(const void* dy, const void* h, const void* weight, int32_t w_dtype,
                               const float* rstd, const void* dresidual, void* dx, int64_t n_rows,
                               int64_t n_cols, int64_t stride_row, int32_t dtype, void* stream) {
  using namespace rus;
  if (int e = check_common("rus_rmsnorm_bwd", n_rows, n_cols, stride_row, dtype, w_dtype)) return e;
  if (n_rows == 0) return RUS_OK;
  if (!dy || !h || !weight || !rstd || !dx)
    return fail(RUS_ERR_INVALID, "rus_rmsnorm_bwd: null pointer argument");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RUS_DTYPE_F16) {
    if (w_dtype == RUS_DTYPE_F16)
      return bwd_typed<f16, f16>(dy, h, weight, rstd, dresidual, dx, n_rows, n_cols, stride_row,
                                 st);
    return bwd_typed<f16, float>(dy, h, weight, rstd, dresidual, dx, n_rows, n_cols, stride_row,
                                 st);
  }
  if (w_dtype == RUS_DTYPE_F16)
    return bwd_typed<float, f16>(dy, h, weight, rstd, dresidual, dx, n_rows, n_cols, stride_row,
                                 st);
  return bwd_typed<float, float>(dy, h, weight, rstd, dresidual, dx, n_rows, n_cols, stride_row,
                                 st);
}
