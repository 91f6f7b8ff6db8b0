// Row functions of the vectorised RMSNorm forward and backward (one wavefront per row, 16-byte
// packs held in registers between the reduction and the output pass), used by launches that run
// a norm beside other work (the NF4 dequant) and by the norm kernels for wide rows. No barriers:
// a wave whose row is past the end returns.
//
// Row sums follow one fixed order, which the multi-wave norm kernels (rmsnorm.hip) reproduce:
// each 16-byte pack's terms are summed in element order, lane l adds its packs l, 64 + l,
// 128 + l, ... in that order (a pack past the row contributes nothing), and a 64-lane butterfly
// adds the lanes. The standalone and the riding norm therefore give the same bits.
#pragma once

#include "common.h"

namespace rus {

// Loads a pack of N weights as 16-byte chunks (fp32 weights for 8 fp16 activations: two 16-byte
// loads) or as one narrower access (fp16 weights for 4 fp32 activations: one 8-byte load).
template <typename T, int N>
__device__ __forceinline__ void load16(const T* __restrict__ p, float (&out)[N]) {
  constexpr int per = 16 / sizeof(T);
  if constexpr (N >= per) {
    static_assert(N % per == 0, "pack must be whole 16-byte chunks");
#pragma unroll
    for (int k = 0; k < N / per; ++k) {
      float tmp[per];
      load_f32<T, per>(p + k * per, tmp);
#pragma unroll
      for (int i = 0; i < per; ++i) out[k * per + i] = tmp[i];
    }
  } else {
    load_f32<T, N>(p, out);
  }
}

// y = T(T(h * rstd) * w) with h = T(x + res) (HAS_RES, also stored to sum_out) or x.
template <typename T, typename W, int NIT, bool HAS_RES>
__device__ __forceinline__ void rmsnorm_fwd_row(const T* __restrict__ x, const T* __restrict__ res,
                                                const W* __restrict__ w, T* __restrict__ sum_out,
                                                T* __restrict__ y, float* __restrict__ rstd,
                                                int row, int n_rows, int n_cols, int64_t stride,
                                                float eps) {
  constexpr int V = 16 / sizeof(T);
  const int lane = threadIdx.x & (kWave - 1);
  if (row >= n_rows) return;
  const int64_t off = static_cast<int64_t>(row) * stride;

  float h[NIT][V];
  float ss = 0.0f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int c = (it * kWave + lane) * V;
    if (c < n_cols) {
      load_f32<T, V>(x + off + c, h[it]);
      if (HAS_RES) {
        float r[V];
        load_f32<T, V>(res + off + c, r);
#pragma unroll
        for (int i = 0; i < V; ++i) h[it][i] = round_to<T>(h[it][i] + r[i]);
        store_from_f32<T, V>(sum_out + off + c, h[it]);
      }
      float sp = 0.0f;
#pragma unroll
      for (int i = 0; i < V; ++i) sp += h[it][i] * h[it][i];
      ss += sp;
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / static_cast<float>(n_cols) + eps);
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int c = (it * kWave + lane) * V;
    if (c < n_cols) {
      float wv[V], o[V];
      load16<W, V>(w + c, wv);
#pragma unroll
      for (int i = 0; i < V; ++i) o[i] = round_to<T>(h[it][i] * r) * wv[i];
      store_from_f32<T, V>(y + off + c, o);
    }
  }
}


// dx = (w dy - xh mean(xh w dy)) rstd (+ dres), xh = h rstd.
template <typename T, typename W, int NIT, bool HAS_DRES>
__device__ __forceinline__ void rmsnorm_bwd_row(const T* __restrict__ dy, const T* __restrict__ h,
                                                const W* __restrict__ w,
                                                const float* __restrict__ rstd,
                                                const T* __restrict__ dres, T* __restrict__ dx,
                                                int row, int n_rows, int n_cols, int64_t stride) {
  constexpr int V = 16 / sizeof(T);
  const int lane = threadIdx.x & (kWave - 1);
  if (row >= n_rows) return;
  const int64_t off = static_cast<int64_t>(row) * stride;
  const float r = rstd[row];

  float xh[NIT][V], g[NIT][V];
  float acc = 0.0f;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int c = (it * kWave + lane) * V;
    if (c < n_cols) {
      float dv[V], wv[V];
      load_f32<T, V>(h + off + c, xh[it]);
      load_f32<T, V>(dy + off + c, dv);
      load16<W, V>(w + c, wv);
      float ap = 0.0f;
#pragma unroll
      for (int i = 0; i < V; ++i) {
        xh[it][i] = xh[it][i] * r;
        g[it][i] = wv[i] * dv[i];
        ap += xh[it][i] * g[it][i];
      }
      acc += ap;
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
        load_f32<T, V>(dres + off + c, d);
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = o[i] + d[i];
      }
      store_from_f32<T, V>(dx + off + c, o);
    }
  }
}


}  // namespace rus
