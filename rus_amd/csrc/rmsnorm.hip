// Residual + RMSNorm forward and its one-pass backward for gfx950.
//
// Behaviour follows solution/kernels.py:125-199 (rms_norm_residual_fwd_kernel,
// rms_norm_bwd_kernel) with the cast order of Qwen2RMSNorm: h = T(x + res), fp32 statistics,
// y = T(fp32(T(h * rstd)) * w). Design (CDNA4, wave64):
//   * rows of up to 1024 16-byte packs (8192 fp16 / 4096 fp32 columns): one workgroup per row,
//     one pack (8 x fp16 or 4 x fp32) per lane, ceil(packs / 64) waves, so a 1536-wide fp16 row
//     is 3 waves and 700-900 rows put 2,000-2,700 waves on the 256 CUs; the pack stays in
//     registers between the row reduction and the normalisation, so every input byte is read
//     from HBM once and each output byte written once;
//   * the row reduction: per-lane pack sums through LDS, added per lane in pack order, then a
//     64-lane butterfly (one barrier) -- the order of the one-wave row functions in
//     rmsnorm_rows.h, which the norm riding in the dequant launch runs, so both give the same
//     bits;
//   * wider rows, and widths that are not a multiple of the pack, fall back to a scalar
//     two-pass kernel (the second pass re-reads the row from L1/L2, not HBM);
//   * built with -ffp-contract=off so every product and sum is rounded as in an eager fp32
//     restatement (only the reduction order differs).
#include <type_traits>

#include "common.h"
#include "rmsnorm_rows.h"

namespace rus {
namespace {

// Row sum over a workgroup of ceil(packs / 64) waves in the one-wave order: lane l of wave w
// holds pack 64 w + l's sum s (0 past the row); lane l's packs are added in pack order, then the
// lanes by a butterfly. Every wave forms the same total.
__device__ __forceinline__ float row_sum_waves(float s, float* red) {
  const int lane = threadIdx.x & (kWave - 1), nw = blockDim.x / kWave;
  red[threadIdx.x] = s;
  __syncthreads();
  float t = red[lane];
  for (int w = 1; w < nw; ++w) t += red[w * kWave + lane];
  return wave_sum(t);
}

constexpr int kWideMaxPacks = 1024;

template <typename T, typename W, bool HAS_RES>
__global__ __launch_bounds__(kWideMaxPacks) void rmsnorm_fwd_wide(
    const T* __restrict__ x, const T* __restrict__ res, const W* __restrict__ w,
    T* __restrict__ sum_out, T* __restrict__ y, float* __restrict__ rstd, int n_cols,
    int64_t stride, float eps) {
  constexpr int V = 16 / sizeof(T);
  __shared__ float red[kWideMaxPacks];
  const int row = blockIdx.x, c = threadIdx.x * V;
  const int64_t off = static_cast<int64_t>(row) * stride;
  float h[V];
  float sp = 0.0f;
  if (c < n_cols) {
    load_f32<T, V>(x + off + c, h);
    if (HAS_RES) {
      float r[V];
      load_f32<T, V>(res + off + c, r);
#pragma unroll
      for (int i = 0; i < V; ++i) h[i] = round_to<T>(h[i] + r[i]);
      store_from_f32<T, V>(sum_out + off + c, h);
    }
#pragma unroll
    for (int i = 0; i < V; ++i) sp += h[i] * h[i];
  }
  const float ss = row_sum_waves(sp, red);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(n_cols) + eps);
  if (threadIdx.x == 0) rstd[row] = r;
  if (c < n_cols) {
    float wv[V], o[V];
    load16<W, V>(w + c, wv);
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = round_to<T>(h[i] * r) * wv[i];
    store_from_f32<T, V>(y + off + c, o);
  }
}

// The backward row, dy read as such (NP == 0) or formed as the fp16 rounding of the in-order sum
// of n_parts fp32 partials [n_parts][n_rows][n_cols] (loaded NP at a time).
template <typename T, typename W, int NP, bool HAS_DRES>
__global__ __launch_bounds__(kWideMaxPacks) void rmsnorm_bwd_wide(
    const T* __restrict__ dy, const float* __restrict__ parts, int n_parts, int64_t part_stride,
    const T* __restrict__ h, const W* __restrict__ w, const float* __restrict__ rstd,
    const T* __restrict__ dres, T* __restrict__ dx, int n_cols, int64_t stride) {
  constexpr int V = 16 / sizeof(T);
  __shared__ float red[kWideMaxPacks];
  const int row = blockIdx.x, c = threadIdx.x * V;
  const int64_t off = static_cast<int64_t>(row) * stride;
  const float r = rstd[row];
  float xh[V], g[V];
  float ap = 0.0f;
  if (c < n_cols) {
    float dv[V], wv[V];
    load_f32<T, V>(h + off + c, xh);
    if constexpr (NP == 0) {
      load_f32<T, V>(dy + off + c, dv);
    } else {
      const float* prow = parts + static_cast<int64_t>(row) * n_cols + c;
      float pv[NP][V];
#pragma unroll
      for (int q = 0; q < NP; ++q) load_f32<float, V>(prow + q * part_stride, pv[q]);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        dv[i] = pv[0][i];
#pragma unroll
        for (int q = 1; q < NP; ++q) dv[i] += pv[q][i];  // part order
      }
      for (int q0 = NP; q0 < n_parts; q0 += NP) {  // more parts: NP at a time, still in order
#pragma unroll
        for (int q = 0; q < NP; ++q)
          if (q0 + q < n_parts) load_f32<float, V>(prow + (q0 + q) * part_stride, pv[q]);
#pragma unroll
        for (int q = 0; q < NP; ++q)
          if (q0 + q < n_parts) {
#pragma unroll
            for (int i = 0; i < V; ++i) dv[i] += pv[q][i];
          }
      }
#pragma unroll
      for (int i = 0; i < V; ++i) dv[i] = round_to<T>(dv[i]);  // what a reduce would write
    }
    load16<W, V>(w + c, wv);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      xh[i] = xh[i] * r;
      g[i] = wv[i] * dv[i];
      ap += xh[i] * g[i];
    }
  }
  const float cm = row_sum_waves(ap, red) / static_cast<float>(n_cols);
  if (c < n_cols) {
    float o[V];
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = (g[i] - xh[i] * cm) * r;
    if (HAS_DRES) {
      float d[V];
      load_f32<T, V>(dres + off + c, d);
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = o[i] + d[i];
    }
    store_from_f32<T, V>(dx + off + c, o);
  }
}

// Workgroup size of the one-row kernels: ceil(packs / 64) waves.
dim3 wide_block(int64_t n_cols, int pack) {
  const int64_t packs = (n_cols + pack - 1) / pack;
  return dim3(static_cast<unsigned>((packs + kWave - 1) / kWave * kWave));
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

struct Launch {
  dim3 grid, block;
};

Launch row_launch(int64_t n_rows) {
  // Scalar fallback: four rows (waves) per workgroup once there are enough rows to fill every
  // CU several times; otherwise one row per workgroup so that small batches still spread over
  // all 256 CUs.
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
  const bool wide = n_cols % V == 0 && stride % V == 0 && n_cols <= kWideMaxPacks * V &&
                    aligned(x, 16) && aligned(y, 16) && aligned(w, 16) &&
                    (!res || (aligned(res, 16) && aligned(sum_out, 16)));
  const int nr = static_cast<int>(n_rows), nc = static_cast<int>(n_cols);
  if (wide) {
    const dim3 grid(static_cast<unsigned>(n_rows)), block = wide_block(n_cols, V);
    if (res)
      hipLaunchKernelGGL((rmsnorm_fwd_wide<T, W, true>), grid, block, 0, st, xp, rp, wp, sp, yp,
                         rstd, nc, stride, eps);
    else
      hipLaunchKernelGGL((rmsnorm_fwd_wide<T, W, false>), grid, block, 0, st, xp, rp, wp, sp, yp,
                         rstd, nc, stride, eps);
  } else {
    const Launch l = row_launch(n_rows);
    if (res)
      hipLaunchKernelGGL((rmsnorm_fwd_any<T, W, true>), l.grid, l.block, 0, st, xp, rp, wp, sp,
                         yp, rstd, nr, nc, stride, eps);
    else
      hipLaunchKernelGGL((rmsnorm_fwd_any<T, W, false>), l.grid, l.block, 0, st, xp, rp, wp, sp,
                         yp, rstd, nr, nc, stride, eps);
  }
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
  const bool wide = n_cols % V == 0 && stride % V == 0 && n_cols <= kWideMaxPacks * V &&
                    aligned(dy, 16) && aligned(h, 16) && aligned(w, 16) && aligned(dx, 16) &&
                    (!dres || aligned(dres, 16));
  const int nr = static_cast<int>(n_rows), nc = static_cast<int>(n_cols);
  if (wide) {
    const dim3 grid(static_cast<unsigned>(n_rows)), block = wide_block(n_cols, V);
    if (dres)
      hipLaunchKernelGGL((rmsnorm_bwd_wide<T, W, 0, true>), grid, block, 0, st, dyp, nullptr, 0,
                         int64_t(0), hp, wp, rstd, dp, dxp, nc, stride);
    else
      hipLaunchKernelGGL((rmsnorm_bwd_wide<T, W, 0, false>), grid, block, 0, st, dyp, nullptr, 0,
                         int64_t(0), hp, wp, rstd, dp, dxp, nc, stride);
  } else {
    const Launch l = row_launch(n_rows);
    if (dres)
      hipLaunchKernelGGL((rmsnorm_bwd_any<T, W, true>), l.grid, l.block, 0, st, dyp, hp, wp,
                         rstd, dp, dxp, nr, nc, stride);
    else
      hipLaunchKernelGGL((rmsnorm_bwd_any<T, W, false>), l.grid, l.block, 0, st, dyp, hp, wp,
                         rstd, dp, dxp, nr, nc, stride);
  }
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
  if (n_parts < 1 || n_parts > 64)
    return fail(RUS_ERR_INVALID, "%s: n_parts=%d outside [1, 64]", fn, n_parts);
  if (n_rows == 0) return RUS_OK;
  if (!dy_parts || !h || !weight || !rstd || !dx)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_cols % 8 || stride_row % 8 || !aligned(dy_parts, 16) || !aligned(h, 16) ||
      !aligned(weight, 16) || !aligned(dx, 16) || (dresidual && !aligned(dresidual, 16)))
    return fail(RUS_ERR_INVALID, "%s: need n_cols and stride_row multiples of 8 and 16-byte "
                "aligned operands", fn);
  if (n_cols > kWideMaxPacks * 8)
    return fail(RUS_ERR_UNSUPPORTED, "%s: n_cols=%lld too wide", fn, (long long)n_cols);
  const int64_t pstride = n_rows * n_cols;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(n_rows)), block = wide_block(n_cols, 8);
  const f16* hp = static_cast<const f16*>(h);
  const f16* dp = static_cast<const f16*>(dresidual);
  f16* dxp = static_cast<f16*>(dx);
  const int nc = static_cast<int>(n_cols);
  // Up to 8 partials are loaded together; more run in batches of 8.
  auto launch = [&](auto wtag, auto np_c) {
    using WT = decltype(wtag);
    constexpr int NP = decltype(np_c)::value;
    if (dp)
      hipLaunchKernelGGL((rmsnorm_bwd_wide<f16, WT, NP, true>), grid, block, 0, st, nullptr,
                         dy_parts, n_parts, pstride, hp, static_cast<const WT*>(weight), rstd, dp,
                         dxp, nc, stride_row);
    else
      hipLaunchKernelGGL((rmsnorm_bwd_wide<f16, WT, NP, false>), grid, block, 0, st, nullptr,
                         dy_parts, n_parts, pstride, hp, static_cast<const WT*>(weight), rstd, dp,
                         dxp, nc, stride_row);
  };
  auto by_parts = [&](auto wtag) {
    switch (n_parts) {
      case 1: launch(wtag, std::integral_constant<int, 1>{}); break;
      case 2: launch(wtag, std::integral_constant<int, 2>{}); break;
      case 3: launch(wtag, std::integral_constant<int, 3>{}); break;
      case 4: launch(wtag, std::integral_constant<int, 4>{}); break;
      case 5: launch(wtag, std::integral_constant<int, 5>{}); break;
      case 6: launch(wtag, std::integral_constant<int, 6>{}); break;
      case 7: launch(wtag, std::integral_constant<int, 7>{}); break;
      default: launch(wtag, std::integral_constant<int, 8>{}); break;
    }
  };
  if (w_dtype == RUS_DTYPE_F16)
    by_parts(f16{});
  else
    by_parts(float{});
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
