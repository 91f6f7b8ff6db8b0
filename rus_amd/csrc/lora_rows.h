// The LoRA-down products of four token rows in one 256-thread block, shared by the LoRA kernels
// (rus_lora_down_rows) and the per-layer dequant launch, whose input-norm rows produce exactly
// the tokens they reduce (nf4_dequant.hip), so both give the same bits.
//
// Reference arithmetic (solution/ops.py:775-778): mid_q = drop_q(x) A_q^T, mid_v = drop_v(x)
// A_v^T, fp16 products with fp32 accumulation, x the attention norm's output [N, D], A [r, D].
#pragma once

#include "common.h"

namespace rus {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16x8 ld8(const f16* p) { return *reinterpret_cast<const f16x8*>(p); }

__device__ __forceinline__ f16x8 zero8() { return f16x8{0, 0, 0, 0, 0, 0, 0, 0}; }

// The reference's fp16 dropout of 8 values (keep bit sh + i of word w for value i).
__device__ __forceinline__ f16x8 drop8(f16x8 x, uint32_t w, int sh, float scale) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f16 v = from_f32<f16>(static_cast<float>(x[i]) * scale);
    r[i] = (w >> (sh + i)) & 1u ? v : static_cast<f16>(0.0f);
  }
  return r;
}

struct DownRows {
  const f16* x;  // [n_tok, sx]
  int64_t sx, n_tok;
  int d, r;      // d a multiple of 64; r in {4, 8, 16}
  const f16* aq;  // A_q, A_v [r, d]
  const f16* av;
  const uint32_t* bits_q;  // keep bits [n_tok, words] of both branches, or both null
  const uint32_t* bits_v;
  int64_t words;
  float scale_q, scale_v;  // 1 / (1 - p)
  f16* mid_q;  // [n_tok, r]
  f16* mid_v;
};

// Validates a rus_lora_rows (ranks 4, 8, 16; d a multiple of 64) and fills the kernel
// arguments; returns RUS_OK or the error code (message set).
inline int lora_rows_args(const char* fn, const rus_lora_rows& q, DownRows& a) {
  if ((q.bits_q == nullptr) != (q.bits_v == nullptr))
    return fail(RUS_ERR_INVALID, "%s: give the keep bits of both branches or of neither", fn);
  if (q.r != 4 && q.r != 8 && q.r != 16)
    return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16}", fn, q.r);
  if (!q.x || !q.a_q || !q.a_v || !q.mid_q || !q.mid_v)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (q.n_tokens < 0 || q.n_tokens >= (int64_t(1) << 31) || q.d <= 0 || q.d % 64 ||
      q.d >= (int64_t(1) << 30) || q.stride_x < q.d || q.stride_x % 8)
    return fail(RUS_ERR_INVALID,
                "%s: need d a multiple of 64, stride_x >= d and stride_x a multiple of 8", fn);
  if (!aligned(q.x, 16) || !aligned(q.a_q, 16) || !aligned(q.a_v, 16) || !aligned(q.mid_q, 2) ||
      !aligned(q.mid_v, 2) || !aligned(q.bits_q, 4) || !aligned(q.bits_v, 4))
    return fail(RUS_ERR_INVALID, "%s: x and A must be 16-byte aligned", fn);
  if (!(q.p_q >= 0.0f && q.p_q < 1.0f && q.p_v >= 0.0f && q.p_v < 1.0f))
    return fail(RUS_ERR_INVALID, "%s: dropout probabilities must be in [0, 1)", fn);
  a = DownRows{static_cast<const f16*>(q.x), q.stride_x, q.n_tokens, static_cast<int>(q.d), q.r,
               static_cast<const f16*>(q.a_q), static_cast<const f16*>(q.a_v), q.bits_q, q.bits_v,
               (q.d + 31) / 32, q.bits_q ? 1.0f / (1.0f - q.p_q) : 1.0f,
               q.bits_v ? 1.0f / (1.0f - q.p_v) : 1.0f, static_cast<f16*>(q.mid_q),
               static_cast<f16*>(q.mid_v)};
  return RUS_OK;
}

constexpr int kDownRows = 4;             // tokens per block
constexpr int kDownParkFloats = 4 * 128;  // LDS the block's four wave sums take

// mid_q / mid_v of tokens t0 .. t0 + 3 (those below n_tok), by all four waves of the block: wave
// w reduces columns [w d/4, (w+1) d/4) on v_mfma_f32_32x32x16_f16 with ranks as rows (rows
// 0 .. r-1 the q ranks against drop_q(x), r .. 2r-1 the v ranks against drop_v(x), the rest
// zero) and tokens as columns (4 .. 31 zero); the waves' sums meet in `park` (kDownParkFloats of
// LDS) and are added in wave order, then rounded to fp16 once. Every thread of the block must
// call it (it holds barriers); x's rows must be visible to the whole block.
template <int U = 4>
__device__ __forceinline__ void lora_down_rows4(const DownRows& a, int64_t t0, float* park) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const bool is_q = col < a.r, is_v = col >= a.r && col < 2 * a.r;
  const f16* arow = is_q ? a.aq + static_cast<int64_t>(col) * a.d
                         : a.av + static_cast<int64_t>(is_v ? col - a.r : 0) * a.d;
  const int64_t t = t0 + col;
  const bool live = col < kDownRows && t < a.n_tok;
  const f16* xrow = a.x + (live ? t : 0) * a.sx;
  const bool drop = a.bits_q != nullptr;  // uniform
  const uint32_t* mq = drop ? a.bits_q + (live ? t : 0) * a.words : nullptr;
  const uint32_t* mv = drop ? a.bits_v + (live ? t : 0) * a.words : nullptr;
  const int per = a.d / 4;  // a multiple of 16
  const int c_begin = wave * per;
  f32x16 acc = f32x16{};
  // U: K steps whose loads are issued together (register budget vs latency; no effect on the
  // arithmetic)
  for (int s0 = 0; s0 < per; s0 += 16 * U) {
    f16x8 af[U], xf[U];
    uint32_t wq[U], wv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c_begin + min(s0 + 16 * u, per - 16) + 8 * h;
      af[u] = (is_q || is_v) ? ld8(arow + c) : zero8();
      xf[u] = live ? ld8(xrow + c) : zero8();
      if (drop) {
        wq[u] = live ? mq[c >> 5] : 0u;
        wv[u] = live ? mv[c >> 5] : 0u;
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any MFMA
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // Steps past the wave's range add zero products: no branch, the batch's loads stay ahead.
      const f16x8 x = s0 + 16 * u < per ? xf[u] : zero8();
      if (drop) {
        const int sh = (c_begin + min(s0 + 16 * u, per - 16) + 8 * h) & 31;
        acc = mfma(is_q ? af[u] : zero8(), drop8(x, wq[u], sh, a.scale_q), acc);
        acc = mfma(is_v ? af[u] : zero8(), drop8(x, wv[u], sh, a.scale_v), acc);
      } else {
        acc = mfma(af[u], x, acc);
      }
    }
  }
  // Register j of lane l: rank row 8 (j / 4) + 4 h + j % 4, token column l % 32.
  if (col < kDownRows) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      park[wave * 128 + col * 32 + 8 * (j >> 2) + 4 * h + (j & 3)] = acc[j];
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    const int tok = threadIdx.x >> 5, row = threadIdx.x & 31;
    const float s = ((park[threadIdx.x] + park[128 + threadIdx.x]) + park[256 + threadIdx.x]) +
                    park[384 + threadIdx.x];
    const int64_t tt = t0 + tok;
    if (tt < a.n_tok && row < 2 * a.r) {
      if (row < a.r)
        a.mid_q[tt * a.r + row] = from_f32<f16>(s);
      else
        a.mid_v[tt * a.r + row - a.r] = from_f32<f16>(s);
    }
  }
}

// LDS that lora_down_rows4_staged needs beside `park` (kDownParkFloats floats): the block's
// four x rows (fp16) and both branches' keep-bit words.
__host__ __device__ constexpr int down_stage_bytes(int d) {
  return kDownRows * d * 2 + 2 * kDownRows * ((d + 31) / 32) * 4;
}

// Copies x rows t0 .. t0 + 3 (zero past n_tok) into xs [kDownRows][d] and their keep-bit words
// into bq / bv [kDownRows][words] (when the branches drop): 16-byte chunks, all loads of a
// thread issued before its LDS stores. Every thread of the block must call it (it ends with a
// barrier); x's rows must be visible to the whole block.
__device__ __forceinline__ void stage_down_rows(const DownRows& a, int64_t t0, f16* xs,
                                                uint32_t* bq, uint32_t* bv) {
  const int per_row = a.d / 8;
  const int chunks = kDownRows * per_row;
  for (int i = threadIdx.x; i < chunks; i += blockDim.x) {
    const int tok = i / per_row, c = (i - tok * per_row) * 8;
    const int64_t t = t0 + tok;
    const f16x8 v = t < a.n_tok ? ld8(a.x + t * a.sx + c) : zero8();
    *reinterpret_cast<f16x8*>(xs + tok * a.d + c) = v;
  }
  if (a.bits_q != nullptr) {
    const int nw = kDownRows * static_cast<int>(a.words);
    for (int i = threadIdx.x; i < nw; i += blockDim.x) {
      const int tok = i / static_cast<int>(a.words);
      const int64_t t = t0 + tok, w = i - tok * a.words;
      const bool live = t < a.n_tok;
      const uint32_t q = live ? a.bits_q[t * a.words + w] : 0u;
      const uint32_t v = live ? a.bits_v[t * a.words + w] : 0u;
      bq[i] = q;
      bv[i] = v;
    }
  }
  __syncthreads();
}

// lora_down_rows4 with the block's x rows and keep bits already in LDS (stage_down_rows): the
// same MFMA sequence on the same operands, so the same bits. Only the A fragments come from
// global memory, U K steps of them issued together; x and the bits are read from LDS at each
// step, so a batch holds 4 U registers per lane.
template <int U>
__device__ __forceinline__ void lora_down_rows4_staged(const DownRows& a, int64_t t0,
                                                       const f16* xs, const uint32_t* bq,
                                                       const uint32_t* bv, float* park) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const bool is_q = col < a.r, is_v = col >= a.r && col < 2 * a.r;
  const f16* arow = is_q ? a.aq + static_cast<int64_t>(col) * a.d
                         : a.av + static_cast<int64_t>(is_v ? col - a.r : 0) * a.d;
  const bool live = col < kDownRows && t0 + col < a.n_tok;
  const f16* xrow = xs + (col < kDownRows ? col : 0) * a.d;
  const int words = static_cast<int>(a.words);
  const uint32_t* mq = bq + (col < kDownRows ? col : 0) * words;
  const uint32_t* mv = bv + (col < kDownRows ? col : 0) * words;
  const bool drop = a.bits_q != nullptr;  // uniform
  const int per = a.d / 4;  // a multiple of 16
  const int c_begin = wave * per;
  f32x16 acc = f32x16{};
  for (int s0 = 0; s0 < per; s0 += 16 * U) {
    f16x8 af[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c_begin + min(s0 + 16 * u, per - 16) + 8 * h;
      af[u] = (is_q || is_v) ? ld8(arow + c) : zero8();
    }
    __builtin_amdgcn_sched_barrier(0);  // every A load of the batch is issued before any MFMA
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c_begin + min(s0 + 16 * u, per - 16) + 8 * h;
      // Steps past the wave's range add zero products, as in lora_down_rows4.
      const f16x8 x = (live && s0 + 16 * u < per) ? ld8(xrow + c) : zero8();
      if (drop) {
        const uint32_t wq = live ? mq[c >> 5] : 0u, wv = live ? mv[c >> 5] : 0u;
        const int sh = c & 31;
        acc = mfma(is_q ? af[u] : zero8(), drop8(x, wq, sh, a.scale_q), acc);
        acc = mfma(is_v ? af[u] : zero8(), drop8(x, wv, sh, a.scale_v), acc);
      } else {
        acc = mfma(af[u], x, acc);
      }
    }
  }
  if (col < kDownRows) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      park[wave * 128 + col * 32 + 8 * (j >> 2) + 4 * h + (j & 3)] = acc[j];
  }
  __syncthreads();
  if (threadIdx.x < 128) {
    const int tok = threadIdx.x >> 5, row = threadIdx.x & 31;
    const float s = ((park[threadIdx.x] + park[128 + threadIdx.x]) + park[256 + threadIdx.x]) +
                    park[384 + threadIdx.x];
    const int64_t tt = t0 + tok;
    if (tt < a.n_tok && row < 2 * a.r) {
      if (row < a.r)
        a.mid_q[tt * a.r + row] = from_f32<f16>(s);
      else
        a.mid_v[tt * a.r + row - a.r] = from_f32<f16>(s);
    }
  }
}

}  // namespace
}  // namespace rus
