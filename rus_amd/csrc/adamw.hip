// AdamW update of one flat fp32 parameter buffer for gfx950.
//
// The update is torch.optim.AdamW's (decoupled weight decay, amsgrad and maximize off), the
// optimizer the reference's trainer runs over the LoRA factors (harness/_train.py:30 forwards
// the trainer's optim settings; HF "adamw_torch"), in the order of torch's single- and
// multi-tensor paths, with every scalar formed in double on the host and rounded once to fp32
// (as torch applies Python floats to fp32 tensors). Per element, in fp32:
//   p *= (1 - lr wd);  m = lerp(m, g, 1 - b1);  v = v b2 + ((1 - b2) g) g;
//   p += (-lr / bc1) (m / (sqrt(v) / sqrt(bc2) + eps)),   bc1 = 1 - b1^t, bc2 = 1 - b2^t.
// Design (CDNA4, wave64): one 16-byte pack of p, g, m and v per thread (a wave moves 4 KiB per
// array), enough 256-thread blocks to cover the buffer in one pass (2,179,072 LoRA values: 2,128
// blocks, about eight per CU), where torch's fused AdamW covers 65,536 values per block (34
// blocks for that buffer). Built with -ffp-contract=off: every product and sum rounds on its own.
#include <cmath>

#include "common.h"

namespace rus {
namespace {

constexpr int kThreads = 256;

struct AdamHyper {
  float decay;      // 1 - lr wd
  float w1;         // 1 - b1, the lerp weight
  float b2, w2;     // b2, 1 - b2
  float neg_step;   // -lr / bc1
  float bc2_sqrt;   // sqrt(bc2)
  float eps;
};

__device__ __forceinline__ void adamw_one(float& p, float g, float& m, float& v,
                                          const AdamHyper& h) {
  p = p * h.decay;
  // torch's lerp: start + w (end - start) for |w| < 0.5, else end - (end - start)(1 - w)
  m = h.w1 < 0.5f ? m + h.w1 * (g - m) : g - (g - m) * (1.0f - h.w1);
  v = v * h.b2;
  v = v + (h.w2 * g) * g;
  const float denom = sqrtf(v) / h.bc2_sqrt + h.eps;
  p = p + h.neg_step * (m / denom);
}

__global__ __launch_bounds__(kThreads) void adamw_kernel(float* __restrict__ p,
                                                         const float* __restrict__ g,
                                                         float* __restrict__ m,
                                                         float* __restrict__ v, int64_t n,
                                                         AdamHyper h) {
  const int64_t n4 = n >> 2;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n4) {
    float4 pp = reinterpret_cast<const float4*>(p)[i];
    const float4 gg = reinterpret_cast<const float4*>(g)[i];
    float4 mm = reinterpret_cast<const float4*>(m)[i];
    float4 vv = reinterpret_cast<const float4*>(v)[i];
    adamw_one(pp.x, gg.x, mm.x, vv.x, h);
    adamw_one(pp.y, gg.y, mm.y, vv.y, h);
    adamw_one(pp.z, gg.z, mm.z, vv.z, h);
    adamw_one(pp.w, gg.w, mm.w, vv.w, h);
    reinterpret_cast<float4*>(p)[i] = pp;
    reinterpret_cast<float4*>(m)[i] = mm;
    reinterpret_cast<float4*>(v)[i] = vv;
  }
  // The (< 4) values past the last whole pack: the first threads of block 0.
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
    const int64_t e = (n4 << 2) + threadIdx.x;
    float pe = p[e], me = m[e], ve = v[e];
    adamw_one(pe, g[e], me, ve, h);
    p[e] = pe;
    m[e] = me;
    v[e] = ve;
  }
}

}  // namespace
}  // namespace rus

using namespace rus;

extern "C" int rus_adamw_step(float* param, const float* grad, float* exp_avg, float* exp_avg_sq,
                              int64_t n, double lr, double beta1, double beta2, double eps,
                              double weight_decay, int64_t step, void* stream) {
  const char* fn = "rus_adamw_step";
  if (n < 0 || n >= (int64_t(1) << 40))
    return fail(RUS_ERR_INVALID, "%s: bad size n=%lld", fn, (long long)n);
  if (n == 0) return RUS_OK;
  if (!param || !grad || !exp_avg || !exp_avg_sq)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (!aligned(param, 16) || !aligned(grad, 16) || !aligned(exp_avg, 16) ||
      !aligned(exp_avg_sq, 16))
    return fail(RUS_ERR_INVALID, "%s: every buffer must be 16-byte aligned", fn);
  if (!(lr >= 0.0) || !(beta1 >= 0.0 && beta1 < 1.0) || !(beta2 >= 0.0 && beta2 < 1.0) ||
      !(eps >= 0.0) || !(weight_decay >= 0.0) || step < 1)
    return fail(RUS_ERR_INVALID,
                "%s: need lr, eps, weight_decay >= 0, betas in [0, 1) and step >= 1", fn);
  const double bc1 = 1.0 - std::pow(beta1, static_cast<double>(step));
  const double bc2 = 1.0 - std::pow(beta2, static_cast<double>(step));
  if (!(bc1 > 0.0) || !(bc2 > 0.0))
    return fail(RUS_ERR_INVALID, "%s: a bias correction rounds to zero (beta^step == 1)", fn);
  AdamHyper h;
  h.decay = static_cast<float>(1.0 - lr * weight_decay);
  h.w1 = static_cast<float>(1.0 - beta1);
  h.b2 = static_cast<float>(beta2);
  h.w2 = static_cast<float>(1.0 - beta2);
  h.neg_step = static_cast<float>(-(lr / bc1));
  h.bc2_sqrt = static_cast<float>(std::sqrt(bc2));
  h.eps = static_cast<float>(eps);
  const int64_t blocks = ((n >> 2) + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(adamw_kernel, dim3(static_cast<unsigned>(blocks > 0 ? blocks : 1)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), param, grad, exp_avg,
                     exp_avg_sq, n, h);
  return check_launch(fn);
}
