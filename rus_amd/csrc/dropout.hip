// LoRA-input dropout on gfx950 with a counter-based generator, so that the forward, the backward
// recompute and a captured HIP graph all draw the same mask without any generator state on the
// host.
//
// Reference behaviour (solution/ops.py:775-777 forward, 882-886 recompute, 986-992 backward): the q
// and v LoRA branches each apply F.dropout(p) to the attention-norm output x; the backward replays
// the generator state saved in forward to draw the same masks again, applies them to the LoRA
// input gradients and adds both to the gradient of x. Here a mask bit is a pure function
// of (seed, stream, element index):
//
//   key     = (seed, stream)          stream = 2 * layer + {0: q branch, 1: v branch}
//   block b = element_index / 8       element_index = row * n_cols + col (logical, stride-free)
//   (w0..w3) = Philox4x64-10(counter = (b, 0, 0, 0), key)   [Salmon et al., SC'11]
//   u_j     = 32-bit word j of (w0.lo, w0.hi, w1.lo, w1.hi, ..., w3.hi), j = element_index % 8
//   keep    = u_j >= T,  T = round(p * 2^32)
//   out     = keep ? T(float(x) * (1 / (1 - p))) : 0
//
// The seed is read from device memory, so a graph replays with whatever seed the host (or a
// captured increment kernel) last wrote there.

#include "common.h"

namespace rus {
namespace {

constexpr uint64_t kPhiloxM0 = 0xD2E7470EE14C6C93ull;
constexpr uint64_t kPhiloxM1 = 0xCA5A826395121157ull;
constexpr uint64_t kPhiloxW0 = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kPhiloxW1 = 0xBB67AE8584CAA73Bull;
constexpr int kThreads = 256;

// Philox4x64 with 10 rounds; returns the four output words in c.
__device__ __forceinline__ void philox4x64_10(uint64_t (&c)[4], uint64_t k0, uint64_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t lo0 = kPhiloxM0 * c[0], hi0 = __umul64hi(kPhiloxM0, c[0]);
    const uint64_t lo1 = kPhiloxM1 * c[2], hi1 = __umul64hi(kPhiloxM1, c[2]);
    const uint64_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += kPhiloxW0;
    k1 += kPhiloxW1;
  }
}

// Keep bits of the 8 elements of block b: bit j set when element 8b+j is kept.
__device__ __forceinline__ uint32_t keep_bits(uint64_t seed, uint64_t stream, uint64_t b,
                                              uint32_t thresh) {
  uint64_t c[4] = {b, 0ull, 0ull, 0ull};
  philox4x64_10(c, seed, stream);
  uint32_t bits = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t lo = static_cast<uint32_t>(c[w]), hi = static_cast<uint32_t>(c[w] >> 32);
    bits |= (lo >= thresh ? 1u : 0u) << (2 * w);
    bits |= (hi >= thresh ? 1u : 0u) << (2 * w + 1);
  }
  return bits;
}

struct DropShape {
  int64_t n_rows, n_cols;
  int64_t stride_x, stride_a, stride_b;  // row strides (elements)
  uint64_t stream_a, stream_b;
  uint32_t thresh_a, thresh_b;
  float scale_a, scale_b;
  int64_t n_blocks;  // ceil(n_rows * n_cols / 8)
  bool vec;          // n_cols % 8 == 0 and every row start 16-byte aligned
};

// out_a = dropout_a(x), out_b = dropout_b(x): one read of x, two masked writes.
template <typename T>
__global__ __launch_bounds__(kThreads) void dropout_fwd_kernel(const T* __restrict__ x,
                                                               T* __restrict__ out_a,
                                                               T* __restrict__ out_b,
                                                               const uint64_t* __restrict__ seed_p,
                                                               DropShape s) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (b >= s.n_blocks) return;
  const uint64_t seed = *seed_p;
  const uint32_t ma = keep_bits(seed, s.stream_a, static_cast<uint64_t>(b), s.thresh_a);
  const uint32_t mb = keep_bits(seed, s.stream_b, static_cast<uint64_t>(b), s.thresh_b);
  const int64_t e0 = b * 8;
  if (s.vec) {
    const int64_t row = e0 / s.n_cols, col = e0 - row * s.n_cols;
    float v[8], ra[8], rb[8];
    load_f32<T, 8>(x + row * s.stride_x + col, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      ra[j] = (ma >> j) & 1u ? v[j] * s.scale_a : 0.0f;
      rb[j] = (mb >> j) & 1u ? v[j] * s.scale_b : 0.0f;
    }
    store_from_f32<T, 8>(out_a + row * s.stride_a + col, ra);
    store_from_f32<T, 8>(out_b + row * s.stride_b + col, rb);
    return;
  }
  const int64_t total = s.n_rows * s.n_cols;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t e = e0 + j;
    if (e >= total) break;
    const int64_t row = e / s.n_cols, col = e - row * s.n_cols;
    const float v = static_cast<float>(x[row * s.stride_x + col]);
    out_a[row * s.stride_a + col] = from_f32<T>((ma >> j) & 1u ? v * s.scale_a : 0.0f);
    out_b[row * s.stride_b + col] = from_f32<T>((mb >> j) & 1u ? v * s.scale_b : 0.0f);
  }
}

// acc = T(T(acc + T(dropout_a(ga))) + T(dropout_b(gb))): the reference's two masked gradients
// and its two in-place adds (each rounded to T), in one pass. Strides: x <- acc, a <- ga, b <- gb.
template <typename T>
__global__ __launch_bounds__(kThreads) void dropout_bwd_add_kernel(T* __restrict__ acc,
                                                                   const T* __restrict__ ga,
                                                                   const T* __restrict__ gb,
                                                                   const uint64_t* __restrict__ seed_p,
                                                                   DropShape s) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (b >= s.n_blocks) return;
  const uint64_t seed = *seed_p;
  const uint32_t ma = keep_bits(seed, s.stream_a, static_cast<uint64_t>(b), s.thresh_a);
  const uint32_t mb = keep_bits(seed, s.stream_b, static_cast<uint64_t>(b), s.thresh_b);
  const int64_t e0 = b * 8;
  if (s.vec) {
    const int64_t row = e0 / s.n_cols, col = e0 - row * s.n_cols;
    float av[8], gav[8], gbv[8], r[8];
    load_f32<T, 8>(acc + row * s.stride_x + col, av);
    load_f32<T, 8>(ga + row * s.stride_a + col, gav);
    load_f32<T, 8>(gb + row * s.stride_b + col, gbv);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float ta = round_to<T>((ma >> j) & 1u ? gav[j] * s.scale_a : 0.0f);
      const float tb = round_to<T>((mb >> j) & 1u ? gbv[j] * s.scale_b : 0.0f);
      r[j] = round_to<T>(av[j] + ta) + tb;
    }
    store_from_f32<T, 8>(acc + row * s.stride_x + col, r);
    return;
  }
  const int64_t total = s.n_rows * s.n_cols;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t e = e0 + j;
    if (e >= total) break;
    const int64_t row = e / s.n_cols, col = e - row * s.n_cols;
    const float ta = round_to<T>((ma >> j) & 1u ? static_cast<float>(ga[row * s.stride_a + col]) * s.scale_a : 0.0f);
    const float tb = round_to<T>((mb >> j) & 1u ? static_cast<float>(gb[row * s.stride_b + col]) * s.scale_b : 0.0f);
    T* p = acc + row * s.stride_x + col;
    *p = from_f32<T>(round_to<T>(static_cast<float>(*p) + ta) + tb);
  }
}

// Packed keep bits of n_streams masks [n_rows, n_cols] (n_cols % 8 == 0): word w of row t of
// stream s (stream0 + s) holds elements 32 w .. 32 w + 31 of that row, bit i for element 32 w + i
// (0 past the row's end), thresholds alternating thresh_even / thresh_odd with s. One word (four
// Philox blocks) per thread.
struct BitsShape {
  uint64_t stream0;
  int64_t n_streams, n_rows, n_cols, words, total;
  uint32_t thresh_even, thresh_odd;
};

__global__ __launch_bounds__(kThreads) void keep_bits_kernel(const uint64_t* __restrict__ seed_p,
                                                             uint32_t* __restrict__ out,
                                                             BitsShape s) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= s.total) return;
  const int64_t w = i % s.words;
  const int64_t rs = i / s.words;
  const int64_t t = rs % s.n_rows;
  const int64_t st = rs / s.n_rows;
  const uint64_t seed = *seed_p;
  const uint32_t thresh = (st & 1) ? s.thresh_odd : s.thresh_even;
  const int64_t chunks = s.n_cols / 8;  // Philox blocks per row
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t c = 4 * w + j;  // block within the row
    if (c < chunks)
      word |= keep_bits(seed, s.stream0 + static_cast<uint64_t>(st),
                        static_cast<uint64_t>(t * chunks + c), thresh)
              << (8 * j);
  }
  out[i] = word;
}

uint32_t threshold(float p) {
  const double t = static_cast<double>(p) * 4294967296.0 + 0.5;
  return t >= 4294967295.0 ? 0xffffffffu : static_cast<uint32_t>(t);
}

int make_shape(const char* fn, const void* x, const void* a, const void* b, int64_t n_rows,
               int64_t n_cols, int64_t stride_x, int64_t stride_a, int64_t stride_b,
               const uint64_t* seed, uint64_t stream_a, uint64_t stream_b, float p_a, float p_b,
               int dtype, DropShape& s) {
  if (!x || !a || !b || !seed) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (dtype != RUS_DTYPE_F16 && dtype != RUS_DTYPE_F32)
    return fail(RUS_ERR_INVALID, "%s: dtype %d not supported", fn, dtype);
  if (n_rows < 0 || n_cols <= 0 || stride_x < n_cols || stride_a < n_cols || stride_b < n_cols)
    return fail(RUS_ERR_INVALID, "%s: bad shape rows=%lld cols=%lld or stride smaller than cols", fn,
                (long long)n_rows, (long long)n_cols);
  if (!(p_a >= 0.0f && p_a < 1.0f && p_b >= 0.0f && p_b < 1.0f))
    return fail(RUS_ERR_INVALID, "%s: dropout probabilities must be in [0, 1)", fn);
  const int64_t total = n_rows * n_cols;
  if (n_rows > 0 && total / n_rows != n_cols)
    return fail(RUS_ERR_UNSUPPORTED, "%s: element count overflows", fn);
  s.n_rows = n_rows;
  s.n_cols = n_cols;
  s.stride_x = stride_x;
  s.stride_a = stride_a;
  s.stride_b = stride_b;
  s.stream_a = stream_a;
  s.stream_b = stream_b;
  s.thresh_a = threshold(p_a);
  s.thresh_b = threshold(p_b);
  s.scale_a = 1.0f / (1.0f - p_a);
  s.scale_b = 1.0f / (1.0f - p_b);
  s.n_blocks = (total + 7) / 8;
  s.vec = n_cols % 8 == 0 && stride_x % 8 == 0 && stride_a % 8 == 0 && stride_b % 8 == 0 &&
          aligned(x, 16) && aligned(a, 16) && aligned(b, 16);
  if (s.n_blocks > (int64_t(1) << 31) * kThreads / 2)
    return fail(RUS_ERR_UNSUPPORTED, "%s: too many elements", fn);
  return RUS_OK;
}

}  // namespace
}  // namespace rus

extern "C" int rus_lora_dropout_fwd(const void* x, void* out_a, void* out_b, int64_t n_rows,
                                    int64_t n_cols, int64_t stride_x, int64_t stride_a,
                                    int64_t stride_b, const uint64_t* seed, uint64_t stream_a,
                                    uint64_t stream_b, float p_a, float p_b, int32_t dtype,
                                    void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_dropout_fwd";
  DropShape s;
  if (int e = make_shape(fn, x, out_a, out_b, n_rows, n_cols, stride_x, stride_a, stride_b, seed,
                         stream_a, stream_b, p_a, p_b, dtype, s))
    return e;
  if (s.n_blocks == 0) return RUS_OK;
  const dim3 grid(static_cast<uint32_t>((s.n_blocks + kThreads - 1) / kThreads));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RUS_DTYPE_F16)
    hipLaunchKernelGGL(dropout_fwd_kernel<f16>, grid, dim3(kThreads), 0, st,
                       static_cast<const f16*>(x), static_cast<f16*>(out_a),
                       static_cast<f16*>(out_b), seed, s);
  else
    hipLaunchKernelGGL(dropout_fwd_kernel<float>, grid, dim3(kThreads), 0, st,
                       static_cast<const float*>(x), static_cast<float*>(out_a),
                       static_cast<float*>(out_b), seed, s);
  return check_launch(fn);
}

extern "C" int rus_lora_dropout_bwd_add(void* acc, const void* grad_a, const void* grad_b,
                                        int64_t n_rows, int64_t n_cols, int64_t stride_acc,
                                        int64_t stride_a, int64_t stride_b, const uint64_t* seed,
                                        uint64_t stream_a, uint64_t stream_b, float p_a, float p_b,
                                        int32_t dtype, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_dropout_bwd_add";
  DropShape s;
  if (int e = make_shape(fn, acc, grad_a, grad_b, n_rows, n_cols, stride_acc, stride_a, stride_b,
                         seed, stream_a, stream_b, p_a, p_b, dtype, s))
    return e;
  if (s.n_blocks == 0) return RUS_OK;
  const dim3 grid(static_cast<uint32_t>((s.n_blocks + kThreads - 1) / kThreads));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == RUS_DTYPE_F16)
    hipLaunchKernelGGL(dropout_bwd_add_kernel<f16>, grid, dim3(kThreads), 0, st,
                       static_cast<f16*>(acc), static_cast<const f16*>(grad_a),
                       static_cast<const f16*>(grad_b), seed, s);
  else
    hipLaunchKernelGGL(dropout_bwd_add_kernel<float>, grid, dim3(kThreads), 0, st,
                       static_cast<float*>(acc), static_cast<const float*>(grad_a),
                       static_cast<const float*>(grad_b), seed, s);
  return check_launch(fn);
}

extern "C" int rus_dropout_keep_bits(const uint64_t* seed, uint64_t stream0, int32_t n_streams,
                                     int64_t n_rows, int64_t n_cols, float p_even, float p_odd,
                                     uint32_t* bits, void* stream) {
  using namespace rus;
  const char* fn = "rus_dropout_keep_bits";
  if (!seed || !bits) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_streams <= 0 || n_rows < 0 || n_cols <= 0 || n_cols % 8)
    return fail(RUS_ERR_INVALID, "%s: need n_streams > 0, n_rows >= 0, n_cols > 0 and a multiple "
                "of 8", fn);
  if (!(p_even >= 0.0f && p_even < 1.0f && p_odd >= 0.0f && p_odd < 1.0f))
    return fail(RUS_ERR_INVALID, "%s: dropout probabilities must be in [0, 1)", fn);
  BitsShape s;
  s.stream0 = stream0;
  s.n_streams = n_streams;
  s.n_rows = n_rows;
  s.n_cols = n_cols;
  s.words = (n_cols + 31) / 32;
  s.total = s.n_streams * n_rows * s.words;
  s.thresh_even = threshold(p_even);
  s.thresh_odd = threshold(p_odd);
  if (s.total == 0) return RUS_OK;
  if (s.total / kThreads >= (int64_t(1) << 31))
    return fail(RUS_ERR_UNSUPPORTED, "%s: too many words", fn);
  hipLaunchKernelGGL(keep_bits_kernel, dim3(static_cast<uint32_t>((s.total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, static_cast<hipStream_t>(stream), seed, bits, s);
  return check_launch(fn);
}
