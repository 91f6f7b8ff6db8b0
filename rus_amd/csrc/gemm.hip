// Split-K fp16 GEMM into fp32 partials for the projections of the layer backward.
//
// The reference forms the MLP input gradient as one fp16 product, d_norm2 = torch.mm(d_gu, W_gu)
// (solution/ops.py:939): a [tokens, 17920] x [17920, 1536] product whose output is small and whose
// reduction is long. On 256 CUs its 256 x 256 output tiles are few (24 at 876 tokens), so the
// reduction is split: block (tile, s) sums the K range of split s and writes its fp32 partial
// parts[s][M][N]; the consumer (the RMSNorm backward, which adds the split parts while it forms
// its row statistics) sums the splits. The mainloop is the shared eight-wave MFMA loop
// (mfma_gemm.h); B is either K-contiguous ([N, ldb], C = A . B^T) or N-contiguous ([K, ldb],
// C = A . B, the weight as the dequant writes it, transposed while it leaves LDS).
#include "common.h"
#include "mfma_gemm.h"

namespace rus {
namespace {

// parts[split][row][col] = acc for the block's 256 x 256 tile (rows < M, cols < N).
__device__ __forceinline__ void store_parts(const GemmArgs& g, const Tile& tl, float* parts,
                                            const f32x16 (&acc)[kMT][2]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 2, wn = wave & 3, h = lane >> 5;
  float* base = parts + static_cast<int64_t>(tl.split) * g.M * g.N;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int col = tl.n0 + wn * 64 + nt * 32 + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = tl.m0 + wm * kWM + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < g.M) base[static_cast<int64_t>(row) * g.N + col] = acc[mt][nt][r];
      }
  }
}

__global__ __launch_bounds__(kThreads8) __attribute__((amdgpu_waves_per_eu(2, 2))) void
gemm_parts_nt_kernel(GemmArgs g, float* parts) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  Tile tl;
  if (!tile_of(g, tl)) return;
  f32x16 acc[kMT][2];
  mainloop(g, tl, smem, acc);
  store_parts(g, tl, parts, acc);
}

__global__ __launch_bounds__(kThreads8) __attribute__((amdgpu_waves_per_eu(2, 2))) void
gemm_parts_kn_kernel(GemmArgs g, float* parts) {
  __shared__ __attribute__((aligned(16))) char smem[kSmem64];
  Tile tl;
  if (!tile_of(g, tl)) return;
  f32x16 acc[kMT][2];
  mainloop_kn(g, tl, smem, acc);
  store_parts(g, tl, parts, acc);
}

}  // namespace
}  // namespace rus

using namespace rus;

extern "C" int rus_gemm_parts(const void* a, int64_t lda, const void* b, int64_t ldb,
                              int32_t b_kn, int64_t m, int64_t n, int64_t k, float* parts,
                              int32_t n_split, void* stream) {
  const char* fn = "rus_gemm_parts";
  if (m < 0 || m >= (1 << 30) || n <= 0 || n >= (1 << 30) || k <= 0 || k >= (1 << 30) ||
      n_split <= 0 || n_split > 64 || (b_kn != 0 && b_kn != 1))
    return fail(RUS_ERR_INVALID, "%s: bad sizes m=%lld n=%lld k=%lld n_split=%d b_kn=%d", fn,
                (long long)m, (long long)n, (long long)k, n_split, b_kn);
  if (k % kBK)
    return fail(RUS_ERR_INVALID, "%s: k=%lld is not a multiple of %d", fn, (long long)k, kBK);
  if (n % 8) return fail(RUS_ERR_INVALID, "%s: n=%lld is not a multiple of 8", fn, (long long)n);
  if (m == 0) return RUS_OK;
  if (lda < k || ldb < (b_kn ? n : k))
    return fail(RUS_ERR_INVALID, "%s: row strides lda=%lld ldb=%lld too small", fn,
                (long long)lda, (long long)ldb);
  if (int e = check_operand(fn, a, lda, "a")) return e;
  if (int e = check_operand(fn, b, ldb, "b")) return e;
  if (!parts || !aligned(parts, 4)) return fail(RUS_ERR_INVALID, "%s: parts is null or misaligned", fn);
  // The mainloop addresses each operand with 32-bit byte offsets.
  if (m * lda * 2 >= (int64_t(1) << 32) || (b_kn ? k : n) * ldb * 2 >= (int64_t(1) << 32))
    return fail(RUS_ERR_INVALID, "%s: an operand exceeds the 4 GiB limit of the MFMA kernels", fn);
  GemmArgs g;
  g.A = static_cast<const f16*>(a);
  g.lda = lda;
  g.B = static_cast<const f16*>(b);
  g.ldb = ldb;
  g.M = static_cast<int>(m);
  g.N = static_cast<int>(n);
  g.K = static_cast<int>(k);
  const int64_t per = (k + n_split - 1) / n_split;
  g.k_per_split = static_cast<int>((per + kBK - 1) / kBK * kBK);
  g.splits = static_cast<int>((k + g.k_per_split - 1) / g.k_per_split);
  if (g.splits != n_split)
    return fail(RUS_ERR_INVALID, "%s: n_split=%d does not divide k=%lld into %d-wide pieces", fn,
                n_split, (long long)k, kBK);
  g.tiles_m = (g.M + kBM - 1) / kBM;
  g.tiles_n = (g.N + kBN - 1) / kBN;
  if (b_kn)
    hipLaunchKernelGGL(gemm_parts_kn_kernel, dim3(launch_grid(g)), dim3(kThreads8), 0,
                       static_cast<hipStream_t>(stream), g, parts);
  else
    hipLaunchKernelGGL(gemm_parts_nt_kernel, dim3(launch_grid(g)), dim3(kThreads8), 0,
                       static_cast<hipStream_t>(stream), g, parts);
  return check_launch(fn);
}
