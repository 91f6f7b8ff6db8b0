// Rank-r LoRA branches of the q and v projections, fused, for gfx950 (fp16 activations).
//
// Reference arithmetic (solution/ops.py:775-778 forward, 975-992 backward), every product an fp16
// tensor with fp32 accumulation:
//   x_q = drop_q(x), x_v = drop_v(x)                       (x: attention-norm output [N, D])
//   mid_q = x_q A_q^T [N, r],  q_lora = mid_q B_q^T [N, Dq]  (v alike with A_v [r, D], B_v [Dv, r])
//   d_mid_q = dq B_q [N, r], dx_q = d_mid_q A_q [N, D]      (dq = scaled LoRA-delta gradient)
//   gB_q = dq^T mid_q [Dq, r], gA_q = d_mid_q^T x_q [r, D]
//   dx += drop_q(dx_q), then += drop_v(dx_v)
// The rank-r products are far too thin for MFMA tiles and, as library GEMMs, cost a launch each
// (13 per layer per step). Here:
//   * lora_down: one wave per group of 64/r tokens; lanes split the reduction dimension in chunks
//     of 8 (one 16-byte load, one Philox block of dropout mask bits), accumulate all 2r outputs
//     of every token of the group in fp32 (v_dot2_f32_f16), then reduce the 128 partial sums
//     across the wave with a 6-step transpose butterfly (each lane ends with two finished sums);
//     it also writes the dropped inputs when the backward needs them;
//   * q_lora / v_lora are formed inside the RoPE kernel from mid and B (rope.hip);
//   * lora_bwd_x: the same reduction for d_mid, the d_mid values shared through LDS, then the
//     expansion d_mid A, the two dropout masks and both adds into dx, in place;
//   * lora_bwd_w: the four weight gradients, one lane per output column, the workgroup's 16 waves
//     splitting the tokens and reducing through LDS in a fixed order (deterministic).
// Every value the reference rounds to fp16 is rounded here at the same point; sums are fp32 in a
// fixed order. The dropout masks are those of dropout.hip (same seed/stream/element convention).

#include "common.h"

namespace rus {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr uint64_t kPhiloxM0 = 0xD2E7470EE14C6C93ull;
constexpr uint64_t kPhiloxM1 = 0xCA5A826395121157ull;
constexpr uint64_t kPhiloxW0 = 0x9E3779B97F4A7C15ull;
constexpr uint64_t kPhiloxW1 = 0xBB67AE8584CAA73Bull;

__device__ __forceinline__ uint32_t philox_keep_bits(uint64_t seed, uint64_t stream, uint64_t b,
                                                     uint32_t thresh) {
  uint64_t c0 = b, c1 = 0, c2 = 0, c3 = 0, k0 = seed, k1 = stream;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t lo0 = kPhiloxM0 * c0, hi0 = __umul64hi(kPhiloxM0, c0);
    const uint64_t lo1 = kPhiloxM1 * c2, hi1 = __umul64hi(kPhiloxM1, c2);
    const uint64_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += kPhiloxW0;
    k1 += kPhiloxW1;
  }
  const uint64_t w[4] = {c0, c1, c2, c3};
  uint32_t bits = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bits |= (static_cast<uint32_t>(w[i]) >= thresh ? 1u : 0u) << (2 * i);
    bits |= (static_cast<uint32_t>(w[i] >> 32) >= thresh ? 1u : 0u) << (2 * i + 1);
  }
  return bits;
}

struct Drop {
  const uint64_t* seed;  // nullptr: no dropout (keep everything, scale 1)
  uint64_t stream_q, stream_v;
  uint32_t thresh_q, thresh_v;
  float scale_q, scale_v;
};

__device__ __forceinline__ u32x4 load16(const f16* p) { return *reinterpret_cast<const u32x4*>(p); }

// Whole-vector bit casts only: a bit cast of a single ext-vector element (v[i]) is not used.
__device__ __forceinline__ void unpack8(u32x4 v, float (&o)[8]) {
  const f16x8 h = __builtin_bit_cast(f16x8, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = static_cast<float>(h[i]);
}

__device__ __forceinline__ u32x4 pack8(const float (&x)[8]) {
  f16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = static_cast<f16>(x[i]);
  return __builtin_bit_cast(u32x4, h);
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  const uint32_t ua = a, ub = b;  // scalar copies, then the bit casts
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, ua), __builtin_bit_cast(half2_t, ub),
                                c, false);
}

// Tokens per wave and partial sums per lane: V = 2 * TT * R (q and v outputs of TT tokens).
template <int R>
struct Tile {
  static constexpr int TT = R >= 32 ? 2 : 4;
  static constexpr int V = 2 * TT * R;
  static constexpr int KEEP = V >= 128 ? V / 64 : 1;  // finished sums per lane
};

// One step over lanes l and l ^ M. While a lane holds N >= 2 entries, both partners hold the same
// range [base, base + N); the lane with bit M set keeps the upper half, the other the lower, each
// adding the partner's copy. With one entry left both keep it and add.
template <int M, int N>
__device__ __forceinline__ void butterfly_step(float* v) {
  if constexpr (N >= 2) {
    constexpr int H = N / 2;
    const bool up = (threadIdx.x & M) != 0;
#pragma unroll
    for (int i = 0; i < H; ++i) {
      const float send = up ? v[i] : v[i + H];
      const float keep = up ? v[i + H] : v[i];
      v[i] = keep + __shfl_xor(send, M, 64);
    }
  } else {
    v[0] += __shfl_xor(v[0], M, 64);
  }
}

// V per-lane partial sums -> wave totals; lane l then holds entries first_entry<V>(l) ..
// + KEEP - 1 in v[0 .. KEEP).
template <int V>
__device__ __forceinline__ void butterfly(float (&v)[V]) {
  butterfly_step<32, V>(v);
  butterfly_step<16, (V >= 2 ? V / 2 : 1)>(v);
  butterfly_step<8, (V >= 4 ? V / 4 : 1)>(v);
  butterfly_step<4, (V >= 8 ? V / 8 : 1)>(v);
  butterfly_step<2, (V >= 16 ? V / 16 : 1)>(v);
  butterfly_step<1, (V >= 32 ? V / 32 : 1)>(v);
}

template <int V>
__device__ __forceinline__ int first_entry(int lane) {
  // Each halving step at lane bit m contributes (bit ? half : 0); half = V / (2 * 64 / m).
  int base = 0;
#pragma unroll
  for (int m = 32, n = V; m >= 1; m >>= 1) {
    if (n >= 2) {
      n /= 2;
      base += (lane & m) ? n : 0;
    }
  }
  return base;
}

// R consecutive fp16 values (R = 4: one 8-byte load; else 16-byte loads) as floats.
template <int R>
__device__ __forceinline__ void load_row(const f16* __restrict__ p, float (&o)[R]) {
  if constexpr (R == 4) {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    const f16x4 h = *reinterpret_cast<const f16x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = static_cast<float>(h[i]);
  } else {
#pragma unroll
    for (int j = 0; j < R; j += 8) {
      float t[8];
      unpack8(load16(p + j), t);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[j + i] = t[i];
    }
  }
}

// Accumulates, for the Tile<R>::TT tokens t0 .. t0+TT-1, this wave's share of the 2R reductions
// of branch q (input xq, length dq, weights wq) and branch v into acc[(tt * 2 + br) * R + j]:
// the four waves of the block take consecutive quarters of each branch's 8-element chunks, the
// lanes of a wave consecutive chunks of its quarter. WT: weights stored [len, R] (B) instead of
// [R, len] (A). With a Drop seed the inputs are dropped (and the dropped fp16 rows written to
// xq_out / xv_out when given).
template <int R, bool WT>
__device__ __forceinline__ void reduce_rows(float (&acc)[Tile<R>::V], int64_t t0, int64_t n_tok,
                                            const f16* __restrict__ xq, int64_t sxq, int64_t dq,
                                            const f16* __restrict__ xv, int64_t sxv, int64_t dv,
                                            const f16* __restrict__ wq, const f16* __restrict__ wv,
                                            const Drop& dr, f16* __restrict__ xq_out,
                                            f16* __restrict__ xv_out) {
  constexpr int TT = Tile<R>::TT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x / 64;
  const uint64_t seed = dr.seed ? *dr.seed : 0ull;
#pragma unroll
  for (int br = 0; br < 2; ++br) {
    const f16* x = br ? xv : xq;
    const int64_t sx = br ? sxv : sxq;
    const int64_t len = br ? dv : dq;
    const f16* w = br ? wv : wq;
    f16* xo = br ? xv_out : xq_out;
    const uint64_t stream = br ? dr.stream_v : dr.stream_q;
    const uint32_t thresh = br ? dr.thresh_v : dr.thresh_q;
    const float scale = br ? dr.scale_v : dr.scale_q;
    const int64_t chunks = len / 8;
    const int64_t per_wave = (chunks + 3) / 4;
    const int64_t c_end = min(chunks, (wave + 1) * per_wave);
    for (int64_t c = wave * per_wave + lane; c < c_end; c += 64) {
      u32x4 xr[TT];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) {
        const int64_t t = t0 + tt;
        xr[tt] = u32x4{0u, 0u, 0u, 0u};
        if (t >= n_tok) continue;
        xr[tt] = load16(x + t * sx + c * 8);
        if (dr.seed) {
          const uint32_t bits =
              philox_keep_bits(seed, stream, static_cast<uint64_t>(t * chunks + c), thresh);
          float xf[8];
          unpack8(xr[tt], xf);
#pragma unroll
          for (int i = 0; i < 8; ++i) xf[i] = (bits >> i) & 1u ? xf[i] * scale : 0.0f;
          xr[tt] = pack8(xf);  // the reference's fp16 dropout output
          if (xo) *reinterpret_cast<u32x4*>(xo + t * len + c * 8) = xr[tt];
        }
      }
      if (WT) {
        // [len, R]: row i of the chunk holds the i-th reduction entry of all R outputs
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float b[R];
          load_row<R>(w + (c * 8 + i) * R, b);
#pragma unroll
          for (int tt = 0; tt < TT; ++tt) {
            const f16x8 xh = __builtin_bit_cast(f16x8, xr[tt]);
            const float xi = static_cast<float>(xh[i]);
#pragma unroll
            for (int j = 0; j < R; ++j)
              acc[(tt * 2 + br) * R + j] = __builtin_fmaf(xi, b[j], acc[(tt * 2 + br) * R + j]);
          }
        }
      } else {
        // [R, len]: wc = 8 consecutive reduction entries of output j
#pragma unroll
        for (int j = 0; j < R; ++j) {
          const u32x4 wc = load16(w + j * len + c * 8);
#pragma unroll
          for (int tt = 0; tt < TT; ++tt) {
            float s = acc[(tt * 2 + br) * R + j];
#pragma unroll
            for (int i = 0; i < 4; ++i) s = dot2(xr[tt][i], wc[i], s);
            acc[(tt * 2 + br) * R + j] = s;
          }
        }
      }
    }
  }
}

// Block-wide totals of the V entries: wave butterflies, then a fixed-order sum over the four
// waves through LDS. Afterwards s_tot[e] holds entry e (rounded to fp16 and back) for every
// thread of the block.
template <int R>
__device__ __forceinline__ void block_totals(float (&acc)[Tile<R>::V], float* s_part,
                                             float* s_tot) {
  using TL = Tile<R>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x / 64;
  butterfly<TL::V>(acc);
  if (TL::V >= 64 || (lane & 1) == 0) {
    const int idx = first_entry<TL::V>(lane);
#pragma unroll
    for (int k = 0; k < TL::KEEP; ++k) s_part[wave * TL::V + idx + k] = acc[k];
  }
  __syncthreads();
  if (threadIdx.x < TL::V) {
    const int e = threadIdx.x;
    const float t = ((s_part[e] + s_part[TL::V + e]) + s_part[2 * TL::V + e]) + s_part[3 * TL::V + e];
    s_tot[e] = static_cast<float>(static_cast<f16>(t));
  }
  __syncthreads();
}

// mid_q = fp16(drop_q(x) A_q^T), mid_v = fp16(drop_v(x) A_v^T); optionally the dropped rows.
// One block of four waves per Tile<R>::TT tokens.
template <int R>
__global__ __launch_bounds__(256) void lora_down_kernel(const f16* __restrict__ x, int64_t sx,
                                                        int64_t n_tok, int64_t d,
                                                        const f16* __restrict__ aq,
                                                        const f16* __restrict__ av,
                                                        f16* __restrict__ mid_q,
                                                        f16* __restrict__ mid_v,
                                                        f16* __restrict__ xq_out,
                                                        f16* __restrict__ xv_out, Drop dr) {
  using TL = Tile<R>;
  __shared__ float s_part[4 * TL::V];
  __shared__ float s_tot[TL::V];
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TL::TT;
  float acc[TL::V];
#pragma unroll
  for (int i = 0; i < TL::V; ++i) acc[i] = 0.0f;
  reduce_rows<R, false>(acc, t0, n_tok, x, sx, d, x, sx, d, aq, av, dr, xq_out, xv_out);
  block_totals<R>(acc, s_part, s_tot);
  if (threadIdx.x < TL::V) {
    const int e = threadIdx.x;
    const int tt = e / (2 * R), br = (e / R) & 1, j = e % R;
    const int64_t t = t0 + tt;
    if (t < n_tok) (br ? mid_v : mid_q)[t * R + j] = static_cast<f16>(s_tot[e]);
  }
}

// d_mid = fp16(dq B) per branch, then dx += fp16 drop_q(fp16(d_mid_q A_q)), += drop_v(...).
// One block of four waves per Tile<R>::TT tokens; the waves split the chunks of both phases.
template <int R>
__global__ __launch_bounds__(256) void lora_bwd_x_kernel(
    const f16* __restrict__ dq, const f16* __restrict__ dv, int64_t n_tok, int64_t len_q,
    int64_t len_v, const f16* __restrict__ aq, const f16* __restrict__ av,
    const f16* __restrict__ bq, const f16* __restrict__ bv, int64_t d, f16* __restrict__ dmid_q,
    f16* __restrict__ dmid_v, f16* __restrict__ dx, int64_t sdx, Drop dr) {
  using TL = Tile<R>;
  constexpr int TT = TL::TT;
  __shared__ float s_part[4 * TL::V];
  __shared__ float s_mid[TL::V];  // entry (tt * 2 + br) * R + j
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TT;
  const int lane = threadIdx.x & 63, wave = threadIdx.x / 64;
  float acc[TL::V];
#pragma unroll
  for (int i = 0; i < TL::V; ++i) acc[i] = 0.0f;
  const Drop none{nullptr, 0, 0, 0, 0, 1.0f, 1.0f};
  reduce_rows<R, true>(acc, t0, n_tok, dq, len_q, len_q, dv, len_v, len_v, bq, bv, none,
                       nullptr, nullptr);
  block_totals<R>(acc, s_part, s_mid);
  if (threadIdx.x < TL::V) {
    const int e = threadIdx.x;
    const int tt = e / (2 * R), br = (e / R) & 1, j = e % R;
    const int64_t t = t0 + tt;
    if (t < n_tok) (br ? dmid_v : dmid_q)[t * R + j] = static_cast<f16>(s_mid[e]);
  }
  const uint64_t seed = dr.seed ? *dr.seed : 0ull;
  const int64_t chunks = d / 8;
  const int64_t per_wave = (chunks + 3) / 4;
  const int64_t c_end = min(chunks, (wave + 1) * per_wave);
  for (int64_t c = wave * per_wave + lane; c < c_end; c += 64) {
    float xq[TT][8], xv[TT][8];
#pragma unroll
    for (int br = 0; br < 2; ++br) {
      const f16* a = br ? av : aq;
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int i = 0; i < 8; ++i) (br ? xv : xq)[tt][i] = 0.0f;
#pragma unroll
      for (int j = 0; j < R; ++j) {
        float arow[8];
        unpack8(load16(a + j * d + c * 8), arow);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
          const float m = s_mid[(tt * 2 + br) * R + j];
#pragma unroll
          for (int i = 0; i < 8; ++i)
            (br ? xv : xq)[tt][i] = __builtin_fmaf(m, arow[i], (br ? xv : xq)[tt][i]);
        }
      }
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const int64_t t = t0 + tt;
      if (t >= n_tok) continue;
      uint32_t bq_bits = 0xffu, bv_bits = 0xffu;
      if (dr.seed) {
        const uint64_t blk = static_cast<uint64_t>(t * chunks + c);
        bq_bits = philox_keep_bits(seed, dr.stream_q, blk, dr.thresh_q);
        bv_bits = philox_keep_bits(seed, dr.stream_v, blk, dr.thresh_v);
      }
      f16* p = dx + t * sdx + c * 8;
      float cur[8];
      unpack8(load16(p), cur);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float hq = round_to<f16>(xq[tt][i]), hv = round_to<f16>(xv[tt][i]);  // fp16 dx_q/v
        const float tq = round_to<f16>((bq_bits >> i) & 1u ? hq * dr.scale_q : 0.0f);
        const float tv = round_to<f16>((bv_bits >> i) & 1u ? hv * dr.scale_v : 0.0f);
        cur[i] = round_to<f16>(cur[i] + tq) + tv;
      }
      *reinterpret_cast<u32x4*>(p) = pack8(cur);
    }
  }
}

// Weight gradients: G[c, j] = fp16(sum_t X[t, c] * M[t, j]) over four (X, M, G) problems laid
// end to end in column space: A_q (X = x_q, M = d_mid_q, G stored [R, D]), B_q (X = dq,
// M = mid_q, G [Dq, R]), A_v, B_v. Block: 64 columns x 16 waves over the tokens.
struct BwdWArgs {
  const f16* x[4];
  int64_t sx[4];
  const f16* m[4];
  f16* g[4];
  int64_t cols[4];
  int32_t transposed[4];  // G stored [R, cols]
  int64_t first_block[5];
  int64_t n_tok;
};

template <int R>
__global__ __launch_bounds__(1024) void lora_bwd_w_kernel(BwdWArgs a) {
  constexpr int kW = 16;  // waves per block, splitting the tokens
  __shared__ float s_acc[kW][64][R + 1];
  int p = 0;
#pragma unroll
  for (int k = 1; k < 4; ++k) p += blockIdx.x >= a.first_block[k] ? 1 : 0;
  const int64_t c0 = (blockIdx.x - a.first_block[p]) * 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x / 64;
  const int64_t c = c0 + lane;
  const bool live = c < a.cols[p];
  const f16* x = a.x[p];
  const f16* m = a.m[p];
  const int64_t sx = a.sx[p];
  float acc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) acc[j] = 0.0f;
  if (live) {
    for (int64_t t = w; t < a.n_tok; t += kW) {
      const float xv = static_cast<float>(x[t * sx + c]);
      float mv[R];
      load_row<R>(m + t * R, mv);
#pragma unroll
      for (int j = 0; j < R; ++j) acc[j] = __builtin_fmaf(xv, mv[j], acc[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < R; ++j) s_acc[w][lane][j] = acc[j];
  __syncthreads();
  // 64 * R outputs, summed over the 16 waves in order.
  for (int o = threadIdx.x; o < 64 * R; o += 1024) {
    const int cl = o / R, j = o % R;
    const int64_t col = c0 + cl;
    if (col >= a.cols[p]) continue;
    float s = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kW; ++ww) s += s_acc[ww][cl][j];
    const f16 h = static_cast<f16>(s);
    if (a.transposed[p])
      a.g[p][j * a.cols[p] + col] = h;
    else
      a.g[p][col * R + j] = h;
  }
}

uint32_t threshold(float p) {
  const double t = static_cast<double>(p) * 4294967296.0 + 0.5;
  return t >= 4294967295.0 ? 0xffffffffu : static_cast<uint32_t>(t);
}

int make_drop(const char* fn, const uint64_t* seed, uint64_t sq, uint64_t sv, float pq, float pv,
              Drop& dr) {
  if (!(pq >= 0.0f && pq < 1.0f && pv >= 0.0f && pv < 1.0f))
    return fail(RUS_ERR_INVALID, "%s: dropout probabilities must be in [0, 1)", fn);
  dr.seed = seed;
  dr.stream_q = sq;
  dr.stream_v = sv;
  dr.thresh_q = seed ? threshold(pq) : 0u;
  dr.thresh_v = seed ? threshold(pv) : 0u;
  dr.scale_q = seed ? 1.0f / (1.0f - pq) : 1.0f;
  dr.scale_v = seed ? 1.0f / (1.0f - pv) : 1.0f;
  return RUS_OK;
}

bool rank_ok(int r) { return r == 4 || r == 8 || r == 16 || r == 32; }

bool al16(const void* p) { return p == nullptr || aligned(p, 16); }

}  // namespace
}  // namespace rus

using rus::f16;

extern "C" int rus_lora_down_fwd(const void* x, int64_t n_tokens, int64_t d, int64_t stride_x,
                                 const void* a_q, const void* a_v, int32_t r, void* mid_q,
                                 void* mid_v, void* x_q_out, void* x_v_out, const uint64_t* seed,
                                 uint64_t stream_q, uint64_t stream_v, float p_q, float p_v,
                                 void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_down_fwd";
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (!x || !a_q || !a_v || !mid_q || !mid_v)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_tokens < 0 || d <= 0 || d % 8 || stride_x < d || stride_x % 8)
    return fail(RUS_ERR_INVALID, "%s: need d %% 8 == 0 and stride_x >= d, stride_x %% 8 == 0", fn);
  if (!al16(x) || !al16(a_q) || !al16(a_v) || !aligned(mid_q, 4) || !aligned(mid_v, 4) ||
      !al16(x_q_out) || !al16(x_v_out))
    return fail(RUS_ERR_INVALID, "%s: x, A and x outputs must be 16-byte aligned", fn);
  if ((x_q_out || x_v_out) && !(x_q_out && x_v_out && seed))
    return fail(RUS_ERR_INVALID, "%s: dropped-row outputs need both pointers and a seed", fn);
  if (n_tokens >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  Drop dr;
  if (int e = make_drop(fn, seed, stream_q, stream_v, p_q, p_v, dr)) return e;
  if (n_tokens == 0) return RUS_OK;
  const int64_t tt = r >= 32 ? 2 : 4;  // Tile<R>::TT tokens per block
  const dim3 grid(static_cast<uint32_t>((n_tokens + tt - 1) / tt));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const f16* xp = static_cast<const f16*>(x);
  const f16* aq = static_cast<const f16*>(a_q);
  const f16* av = static_cast<const f16*>(a_v);
  f16 *mq = static_cast<f16*>(mid_q), *mv = static_cast<f16*>(mid_v);
  f16 *xq = static_cast<f16*>(x_q_out), *xv = static_cast<f16*>(x_v_out);
#define RUS_DOWN(RR)                                                                          \
  case RR:                                                                                    \
    hipLaunchKernelGGL(lora_down_kernel<RR>, grid, dim3(256), 0, st, xp, stride_x, n_tokens, d, \
                       aq, av, mq, mv, xq, xv, dr);                                           \
    break;
  switch (r) { RUS_DOWN(4) RUS_DOWN(8) RUS_DOWN(16) RUS_DOWN(32) }
#undef RUS_DOWN
  return check_launch(fn);
}

extern "C" int rus_lora_bwd_x(const void* dq_lora, const void* dv_lora, int64_t n_tokens,
                              int64_t d_q, int64_t d_v, const void* a_q, const void* a_v,
                              const void* b_q, const void* b_v, int32_t r, int64_t d,
                              void* d_mid_q, void* d_mid_v, void* dx, int64_t stride_dx,
                              const uint64_t* seed, uint64_t stream_q, uint64_t stream_v,
                              float p_q, float p_v, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_bwd_x";
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (!dq_lora || !dv_lora || !a_q || !a_v || !b_q || !b_v || !d_mid_q || !d_mid_v || !dx)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_tokens < 0 || d <= 0 || d % 8 || d_q <= 0 || d_q % 8 || d_v <= 0 || d_v % 8 ||
      stride_dx < d || stride_dx % 8)
    return fail(RUS_ERR_INVALID, "%s: lengths must be positive multiples of 8, stride_dx >= d",
                fn);
  if (!al16(dq_lora) || !al16(dv_lora) || !al16(a_q) || !al16(a_v) || !aligned(b_q, 4) ||
      !aligned(b_v, 4) || !al16(dx) || !aligned(d_mid_q, 4) || !aligned(d_mid_v, 4))
    return fail(RUS_ERR_INVALID, "%s: misaligned operand", fn);
  if (n_tokens >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  Drop dr;
  if (int e = make_drop(fn, seed, stream_q, stream_v, p_q, p_v, dr)) return e;
  if (n_tokens == 0) return RUS_OK;
  const int64_t tt = r >= 32 ? 2 : 4;  // Tile<R>::TT tokens per block
  const dim3 grid(static_cast<uint32_t>((n_tokens + tt - 1) / tt));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_BX(RR)                                                                             \
  case RR:                                                                                     \
    hipLaunchKernelGGL(lora_bwd_x_kernel<RR>, grid, dim3(256), 0, st,                          \
                       static_cast<const f16*>(dq_lora), static_cast<const f16*>(dv_lora),     \
                       n_tokens, d_q, d_v, static_cast<const f16*>(a_q),                      \
                       static_cast<const f16*>(a_v), static_cast<const f16*>(b_q),             \
                       static_cast<const f16*>(b_v), d, static_cast<f16*>(d_mid_q),            \
                       static_cast<f16*>(d_mid_v), static_cast<f16*>(dx), stride_dx, dr);      \
    break;
  switch (r) { RUS_BX(4) RUS_BX(8) RUS_BX(16) RUS_BX(32) }
#undef RUS_BX
  return check_launch(fn);
}

extern "C" int rus_lora_bwd_w(const void* x_q, const void* x_v, int64_t stride_x,
                              const void* dq_lora, const void* dv_lora, const void* mid_q,
                              const void* mid_v, const void* d_mid_q, const void* d_mid_v,
                              int64_t n_tokens, int64_t d, int64_t d_q, int64_t d_v, int32_t r,
                              void* g_a_q, void* g_b_q, void* g_a_v, void* g_b_v, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_bwd_w";
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (!x_q || !x_v || !dq_lora || !dv_lora || !mid_q || !mid_v || !d_mid_q || !d_mid_v ||
      !g_a_q || !g_b_q || !g_a_v || !g_b_v)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_tokens < 0 || d <= 0 || d_q <= 0 || d_v <= 0 || stride_x < d)
    return fail(RUS_ERR_INVALID, "%s: bad lengths", fn);
  if (!aligned(mid_q, 8) || !aligned(mid_v, 8) || !aligned(d_mid_q, 8) || !aligned(d_mid_v, 8))
    return fail(RUS_ERR_INVALID, "%s: [N, r] operands must be 8-byte aligned", fn);
  if (n_tokens >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  BwdWArgs a;
  a.x[0] = static_cast<const f16*>(x_q);
  a.sx[0] = stride_x;
  a.m[0] = static_cast<const f16*>(d_mid_q);
  a.g[0] = static_cast<f16*>(g_a_q);
  a.cols[0] = d;
  a.transposed[0] = 1;
  a.x[1] = static_cast<const f16*>(dq_lora);
  a.sx[1] = d_q;
  a.m[1] = static_cast<const f16*>(mid_q);
  a.g[1] = static_cast<f16*>(g_b_q);
  a.cols[1] = d_q;
  a.transposed[1] = 0;
  a.x[2] = static_cast<const f16*>(x_v);
  a.sx[2] = stride_x;
  a.m[2] = static_cast<const f16*>(d_mid_v);
  a.g[2] = static_cast<f16*>(g_a_v);
  a.cols[2] = d;
  a.transposed[2] = 1;
  a.x[3] = static_cast<const f16*>(dv_lora);
  a.sx[3] = d_v;
  a.m[3] = static_cast<const f16*>(mid_v);
  a.g[3] = static_cast<f16*>(g_b_v);
  a.cols[3] = d_v;
  a.transposed[3] = 0;
  a.first_block[0] = 0;
  for (int k = 0; k < 4; ++k) a.first_block[k + 1] = a.first_block[k] + (a.cols[k] + 63) / 64;
  a.n_tok = n_tokens;
  const dim3 grid(static_cast<uint32_t>(a.first_block[4]));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_BW(RR)                                                                      \
  case RR:                                                                              \
    hipLaunchKernelGGL(lora_bwd_w_kernel<RR>, grid, dim3(1024), 0, st, a);              \
    break;
  switch (r) { RUS_BW(4) RUS_BW(8) RUS_BW(16) RUS_BW(32) }
#undef RUS_BW
  return check_launch(fn);
}
