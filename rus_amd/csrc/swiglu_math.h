// SwiGLU element math shared by the SwiGLU kernels (swiglu.hip) and the split-K product that
// forms d_gate / d_up on the fly (gemm.hip), so both produce the same bits.
// Formulas of solution/kernels.py:355-446: out = silu(g) u; d_gate = (dout u) silu'(g),
// d_up = dout silu(g), silu'(g) = s + silu (1 - s), s = sigmoid(g). The sigmoid uses the hardware
// exp and reciprocal (about 1 fp32 ulp each).
#pragma once

namespace rus {

__device__ __forceinline__ float glu_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// d_gate and d_up (fp32, before rounding) of one element.
__device__ __forceinline__ void glu_bwd(float d, float g, float u, float& dg, float& du) {
  const float sg = glu_sigmoid(g);
  const float silu = g * sg;
  du = d * silu;
  const float dsilu = sg + silu * (1.0f - sg);
  dg = (d * u) * dsilu;
}

// d_up alone.
__device__ __forceinline__ float glu_bwd_up(float d, float g) { return d * (g * glu_sigmoid(g)); }

}  // namespace rus
