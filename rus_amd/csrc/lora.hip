// Rank-r LoRA branches of the q and v projections, fused, for gfx950 (fp16 activations).
//
// Reference arithmetic (solution/ops.py:775-778 forward, 975-992 backward), every product an fp16
// tensor with fp32 accumulation:
//   x_q = drop_q(x), x_v = drop_v(x)                       (x: attention-norm output [N, D])
//   mid_q = x_q A_q^T [N, r],  q_lora = mid_q B_q^T [N, Dq]  (v alike with A_v [r, D], B_v [Dv, r])
//   d_mid_q = dq B_q [N, r], dx_q = d_mid_q A_q [N, D]      (dq = scaled LoRA-delta gradient)
//   gB_q = dq^T mid_q [Dq, r], gA_q = d_mid_q^T x_q [r, D]
//   dx += drop_q(dx_q), then += drop_v(dx_v)
// Dropout masks arrive as packed keep bits (rus_dropout_keep_bits: word w of row t holds
// elements 32 w .. 32 w + 31), drawn once per step for every layer, so no kernel here runs the
// generator and no dropped copy of x is stored. Kernels:
//   * lora_down: one block of 8 waves per 32 tokens; the rank-r products on MFMA
//     (v_mfma_f32_32x32x16_f16, tokens x ranks, ranks past r zero), the waves splitting the
//     reduction over D and summing their partials through LDS in a fixed order;
//   * q_lora / v_lora are formed inside the RoPE kernel from mid and B (rope.hip);
//   * lora_bwd_x: the same for d_mid = dq B (from rank-major B^T copies), then the expansion
//     d_mid A as MFMA tiles of dx^T (rank-major A^T copies), with the masks and both rounded adds
//     into dx in place;
//   * lora_bwd_w: the four weight gradients (reductions over tokens) on the vector units, one lane
//     per output column and token phase, 16 columns per block, waves splitting the tokens and
//     summing through LDS in a fixed order (deterministic).
// Every value the reference rounds to fp16 is rounded here at the same point; sums are fp32.

#include "common.h"

namespace rus {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTok = 32;  // tokens per block (down, bwd_x)
constexpr int kMS = 40;   // row stride (halfs) of the fp16 d_mid tile in LDS: 32 ranks + pad

__device__ __forceinline__ f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16x8 ld8(const f16* p) { return *reinterpret_cast<const f16x8*>(p); }

__device__ __forceinline__ f16x8 zero8() { return f16x8{0, 0, 0, 0, 0, 0, 0, 0}; }

// Accumulator row of register r for lane half h (v_mfma_f32_32x32x16: lane l holds column l % 32).
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ float round16(float x) { return static_cast<float>(static_cast<f16>(x)); }

// Ranks k0 .. k0+7 (k0 in {0, 8, 16, 24}) of a row of R fp16 values, zero past R.
template <int R>
__device__ __forceinline__ f16x8 frag_rank(const f16* row, int k0) {
  if constexpr (R >= 16) {
    return ld8(row + k0);
  } else if constexpr (R == 8) {
    return k0 == 0 ? ld8(row) : zero8();
  } else {
    if (k0 != 0) return zero8();
    const f16x4 v = *reinterpret_cast<const f16x4*>(row);
    return f16x8{v[0], v[1], v[2], v[3], 0, 0, 0, 0};
  }
}

// Waves per block of lora_down / lora_bwd_x and the accumulator layout: for R <= 16 the q and
// v results share one 32-column accumulator (q in columns 0 .. R-1, v in R .. 2R-1), for R = 32
// each branch has its own.
template <int R>
struct Cfg {
  static constexpr bool PACK = R <= 16;
  static constexpr int NACC = PACK ? 1 : 2;
  static constexpr int W = PACK ? 16 : 8;
};

// Stores a wave's accumulators in LDS (lane-contiguous) for the fixed-order sum over waves.
template <int NACC>
__device__ __forceinline__ void park(float* buf, const f32x16 (&c)[NACC], int wave, int lane) {
#pragma unroll
  for (int j = 0; j < NACC; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) buf[((wave * NACC + j) * 16 + r) * 64 + lane] = c[j][r];
}

template <int NACC, int W>
__device__ __forceinline__ float parked_sum(const float* buf, int j, int r, int lane) {
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) s += buf[((w * NACC + j) * 16 + r) * 64 + lane];
  return s;
}

// Branch and rank of accumulator column n of accumulator j (-1: unused column).
template <int R>
__device__ __forceinline__ void col_owner(int j, int n, int& br, int& rank) {
  if constexpr (Cfg<R>::PACK) {
    br = n < R ? 0 : (n < 2 * R ? 1 : -1);
    rank = n < R ? n : n - R;
  } else {
    br = j;
    rank = n;
  }
}

// The reference's fp16 dropout of 8 values (keep bit sh + i of word w for value i).
__device__ __forceinline__ f16x8 drop8(f16x8 x, uint32_t w, int sh, float scale) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f16 v = static_cast<f16>(static_cast<float>(x[i]) * scale);
    r[i] = (w >> (sh + i)) & 1u ? v : static_cast<f16>(0.0f);
  }
  return r;
}

struct DownArgs {
  const f16* x;
  int64_t sx, n_tok, d;
  const f16* aq;
  const f16* av;
  f16* mid_q;
  f16* mid_v;
  const uint32_t* bits_q;  // both or neither (nullptr: no dropout)
  const uint32_t* bits_v;
  int64_t words;  // mask words per row
  float scale_q, scale_v;
};

// mid_q = fp16(drop_q(x) A_q^T), mid_v = fp16(drop_v(x) A_v^T). C = tokens x ranks: the A operand
// is 8 dropped x values of the lane's token, the B operand 8 entries of the A row that owns the
// lane's column (zeros for unused columns). Wave w takes k-steps w, w + W, ...; the loads of up
// to U steps are issued together before their MFMAs, so a wave waits on memory once per batch.
template <int R, bool DROP>
__global__ __launch_bounds__(64 * Cfg<R>::W) void lora_down_kernel(DownArgs a) {
  using C = Cfg<R>;
  constexpr int W = C::W, NACC = C::NACC, U = 6;
  __shared__ float buf[W * NACC * 16 * 64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTok;
  const int64_t t = min(t0 + col, a.n_tok - 1);  // rows past the end are computed, not stored
  const f16* xrow = a.x + t * a.sx;
  int br0, rk0;
  col_owner<R>(0, col, br0, rk0);
  // B rows: PACK -> the owning branch's A row (row 0 of A_q for unused columns);
  // else A_q row col (accumulator 0) and A_v row col (accumulator 1).
  const f16* b0 = C::PACK ? (br0 == 1 ? a.av + rk0 * a.d : a.aq + (br0 == 0 ? rk0 : 0) * a.d)
                          : a.aq + col * a.d;
  const f16* b1 = a.av + (C::PACK ? 0 : col) * a.d;
  const uint32_t* mq = DROP ? a.bits_q + t * a.words : nullptr;
  const uint32_t* mv = DROP ? a.bits_v + t * a.words : nullptr;
  const int ks = static_cast<int>(a.d / 16);
  f32x16 acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) acc[j] = f32x16{};
  for (int s0 = wave; s0 < ks; s0 += W * U) {
    f16x8 xs[U], f0[U], f1[U];
    uint32_t wq[U], wv[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int c0 = 16 * min(s0 + W * i, ks - 1) + 8 * h;
      xs[i] = ld8(xrow + c0);
      f0[i] = ld8(b0 + c0);
      if constexpr (!C::PACK) f1[i] = ld8(b1 + c0);
      if constexpr (DROP) {
        wq[i] = mq[c0 >> 5];
        wv[i] = mv[c0 >> 5];
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any MFMA
#pragma unroll
    for (int i = 0; i < U; ++i) {
      // Steps past the end add zero products: no branch, so the batch's loads stay in front.
      if (s0 + W * i >= ks) xs[i] = zero8();
      const int sh = (16 * min(s0 + W * i, ks - 1) + 8 * h) & 31;
      if constexpr (C::PACK) {
        if constexpr (DROP) {
          acc[0] = mfma(drop8(xs[i], wq[i], sh, a.scale_q), br0 == 0 ? f0[i] : zero8(), acc[0]);
          acc[0] = mfma(drop8(xs[i], wv[i], sh, a.scale_v), br0 == 1 ? f0[i] : zero8(), acc[0]);
        } else {
          acc[0] = mfma(xs[i], br0 >= 0 ? f0[i] : zero8(), acc[0]);
        }
      } else {
        const f16x8 xq = DROP ? drop8(xs[i], wq[i], sh, a.scale_q) : xs[i];
        const f16x8 xv = DROP ? drop8(xs[i], wv[i], sh, a.scale_v) : xs[i];
        acc[0] = mfma(xq, f0[i], acc[0]);
        acc[NACC - 1] = mfma(xv, f1[i], acc[NACC - 1]);
      }
    }
  }
  park<NACC>(buf, acc, wave, lane);
  __syncthreads();
  for (int e = threadIdx.x; e < NACC * 16 * 64; e += 64 * W) {
    const int ln = e & 63, r = (e >> 6) & 15, j = e >> 10;
    int br, rank;
    col_owner<R>(j, ln & 31, br, rank);
    const int64_t tt = t0 + acc_row(r, ln >> 5);
    if (br < 0 || tt >= a.n_tok) continue;
    (br ? a.mid_v : a.mid_q)[tt * R + rank] =
        static_cast<f16>(parked_sum<NACC, W>(buf, j, r, ln));
  }
}

struct BwdXArgs {
  const f16* dq;
  const f16* dv;
  int64_t n_tok, len_q, len_v;
  const f16* at_q;  // A^T [d, R]
  const f16* at_v;
  const f16* bt_q;  // B^T [R, len]
  const f16* bt_v;
  int64_t d;
  f16* dmid_q;
  f16* dmid_v;
  f16* dx;
  int64_t sdx;
  const uint32_t* bits_q;
  const uint32_t* bits_v;
  int64_t words;
  float scale_q, scale_v;
};

// acc += sum over the wave's k-steps s = first, first + W, ... < ks of the MFMA of 8 values of
// row x and of row bt at 16 s + 8 h (bt zeroed when use is false). Loads of U steps are issued
// together; steps past the end multiply zeros (no branch between the loads and their MFMAs).
template <int U, int W>
__device__ __forceinline__ void reduce_batched(f32x16& acc, const f16* x, const f16* bt, bool use,
                                               int first, int ks, int h) {
  for (int s0 = first; s0 < ks; s0 += W * U) {
    f16x8 xs[U], fs[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int c0 = 16 * min(s0 + W * i, ks - 1) + 8 * h;
      xs[i] = ld8(x + c0);
      fs[i] = ld8(bt + c0);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any MFMA
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const f16x8 xi = s0 + W * i < ks ? xs[i] : zero8();
      acc = mfma(xi, use ? fs[i] : zero8(), acc);
    }
  }
}

// Phase 1: d_mid_q = fp16(dq B_q), d_mid_v = fp16(dv B_v) (tokens x ranks; the k-steps run over
// the q reduction, then the v one, each with the B^T row owning the lane's column). Phase 2, per
// 32 columns of dx: dx^T tile = A^T d_mid^T for each branch (MFMA, k = ranks), then per element
// dx = fp16(fp16(dx + fp16(drop_q(fp16(dx_q)))) + fp16(drop_v(fp16(dx_v)))). In both phases a
// wave issues the loads of a batch of its steps before their MFMAs.
template <int R, bool DROP>
__global__ __launch_bounds__(64 * Cfg<R>::W) void lora_bwd_x_kernel(BwdXArgs a) {
  using C = Cfg<R>;
  constexpr int W = C::W, NACC = C::NACC, U = 8, U2 = 3;
  __shared__ float buf[W * NACC * 16 * 64];
  __shared__ __attribute__((aligned(16))) f16 s_mid[2][kTok][kMS];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTok;
  const int64_t t = min(t0 + col, a.n_tok - 1);
  int br0, rk0;
  col_owner<R>(0, col, br0, rk0);
  const int ksq = static_cast<int>(a.len_q / 16), ksv = static_cast<int>(a.len_v / 16);
  // The lane's B^T rows for q-steps and v-steps, and whether it contributes to each.
  const bool in_q = C::PACK ? br0 == 0 : true;
  const bool in_v = C::PACK ? br0 == 1 : true;
  const f16* bq = a.bt_q + (C::PACK ? (in_q ? rk0 : 0) : col) * a.len_q;
  const f16* bv = a.bt_v + (C::PACK ? (in_v ? rk0 : 0) : col) * a.len_v;
  const f16* xq = a.dq + t * a.len_q;
  const f16* xv = a.dv + t * a.len_v;
  f32x16 acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) acc[j] = f32x16{};
  reduce_batched<U, W>(acc[0], xq, bq, in_q, wave, ksq, h);
  reduce_batched<U, W>(acc[NACC - 1], xv, bv, in_v, wave, ksv, h);
  park<NACC>(buf, acc, wave, lane);
  __syncthreads();
  for (int e = threadIdx.x; e < 2 * kTok * 32; e += 64 * W) {  // every (branch, row, rank<32)
    const int br = e >> 10, row = (e >> 5) & 31, n = e & 31;
    f16 v = static_cast<f16>(0.0f);
    if (n < R) {
      // accumulator j, column cc and register r holding (branch br, token row, rank n)
      const int j = C::PACK ? 0 : br, cc = C::PACK ? br * R + n : n;
      const int hh = (row >> 2) & 1, r = ((row >> 3) << 2) | (row & 3);
      v = static_cast<f16>(parked_sum<NACC, W>(buf, j, r, hh * 32 + cc));
      const int64_t tt = t0 + row;
      if (tt < a.n_tok) (br ? a.dmid_v : a.dmid_q)[tt * R + n] = v;
    }
    s_mid[br][row][n] = v;  // ranks past R are zero operands below
  }
  __syncthreads();

  // Phase 2. This lane's token is column col of every dx^T tile; rows past the end read row
  // n_tok - 1 and are not stored.
  constexpr int KS = R > 16 ? 2 : 1;
  f16x8 mq[KS], mv[KS];
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    mq[j] = *reinterpret_cast<const f16x8*>(&s_mid[0][col][16 * j + 8 * h]);
    mv[j] = *reinterpret_cast<const f16x8*>(&s_mid[1][col][16 * j + 8 * h]);
  }
  const bool tok_ok = t0 + col < a.n_tok;
  const int n_dt = static_cast<int>(a.d / 32);
  f16* dxrow = a.dx + t * a.sdx;
  const uint32_t* wbq = DROP ? a.bits_q + t * a.words : nullptr;
  const uint32_t* wbv = DROP ? a.bits_v + t * a.words : nullptr;
  for (int d0 = wave; d0 < n_dt; d0 += W * U2) {
    f16x8 aq[U2][KS], av[U2][KS];
    f16x4 dxv[U2][4];
    uint32_t wq[U2], wv[U2];
#pragma unroll
    for (int i = 0; i < U2; ++i) {
      const int dt = min(d0 + W * i, n_dt - 1);
      const int64_t drow = static_cast<int64_t>(dt) * 32 + col;  // A-operand row of this lane
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        aq[i][j] = frag_rank<R>(a.at_q + drow * R, 16 * j + 8 * h);
        av[i][j] = frag_rank<R>(a.at_v + drow * R, 16 * j + 8 * h);
      }
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        dxv[i][r4] = *reinterpret_cast<const f16x4*>(dxrow + dt * 32 + 8 * r4 + 4 * h);
      wq[i] = DROP ? wbq[dt] : 0xffffffffu;
      wv[i] = DROP ? wbv[dt] : 0xffffffffu;
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any MFMA
#pragma unroll
    for (int i = 0; i < U2; ++i) {
      const int dt = min(d0 + W * i, n_dt - 1);
      const bool store = tok_ok && d0 + W * i < n_dt;  // tiles past the end are not written
      f32x16 oq = f32x16{}, ov = f32x16{};
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        oq = mfma(aq[i][j], mq[j], oq);
        ov = mfma(av[i][j], mv[j], ov);
      }
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int off = 8 * r4 + 4 * h;
        f16x4 c = dxv[i][r4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int r = 4 * r4 + k, bit = off + k;
          const float hq = round16(oq[r]), hv = round16(ov[r]);  // fp16 dx_q, dx_v
          const float tq = round16((wq[i] >> bit) & 1u ? hq * a.scale_q : 0.0f);
          const float tv = round16((wv[i] >> bit) & 1u ? hv * a.scale_v : 0.0f);
          c[k] = static_cast<f16>(round16(static_cast<float>(c[k]) + tq) + tv);
        }
        if (store) *reinterpret_cast<f16x4*>(dxrow + dt * 32 + off) = c;
      }
    }
  }
}

// R consecutive fp16 values (R = 4: one 8-byte load; else 16-byte loads) as floats.
template <int R>
__device__ __forceinline__ void load_row(const f16* __restrict__ p, float (&o)[R]) {
  if constexpr (R == 4) {
    const f16x4 v = *reinterpret_cast<const f16x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = static_cast<float>(v[i]);
  } else {
#pragma unroll
    for (int j = 0; j < R; j += 8) {
      const f16x8 v = ld8(p + j);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[j + i] = static_cast<float>(v[i]);
    }
  }
}

// Weight gradients: G[c, j] = fp16(sum_t X[t, c] * M[t, j]) over four (X, M, G) problems laid
// end to end in column space: A_q (X = drop_q(x), M = d_mid_q, G stored [R, D]), B_q (X = dq,
// M = mid_q, G [Dq, R]), A_v, B_v. Block: 16 columns x (4 token phases per wave x 16 waves).
struct BwdWArgs {
  const f16* x[4];
  int64_t sx[4];
  const uint32_t* bits[4];  // A problems: x dropped with these keep bits (nullptr: no dropout)
  float scale[4];
  const f16* m[4];
  f16* g[4];
  int64_t cols[4];
  int32_t transposed[4];  // G stored [R, cols]
  int64_t first_block[5];
  int64_t n_tok, words;
};

constexpr int kWCols = 8;    // columns per block
constexpr int kWPh = 8;      // token phases per wave
constexpr int kWWaves = 16;  // waves per block

// acc[j] += sum over this lane's tokens of X[t, c] * M[t, j] (X dropped with the keep bits
// when MASK), tokens w * kWPh + ph + k * kWPh * kWWaves in batches of U whose loads are issued
// together; past the end (or for a dead column) the weight is zero.
template <int R, bool MASK>
__device__ __forceinline__ void bwd_w_tokens(float (&acc)[R], const f16* __restrict__ x,
                                             int64_t sx, const uint32_t* __restrict__ bits,
                                             float scale, const f16* __restrict__ m, int64_t c,
                                             bool live, int64_t n_tok, int64_t words, int first) {
  constexpr int U = R >= 32 ? 3 : 6;  // smaller batches keep 32 accumulators in registers
  constexpr int64_t kStride = kWPh * kWWaves;
  for (int64_t tb = first; tb < n_tok; tb += U * kStride) {
    float xv[U], mv[U][R];
    uint32_t word[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t tt = tb + u * kStride;
      const int64_t tc = tt < n_tok ? tt : n_tok - 1;
      xv[u] = static_cast<float>(x[tc * sx + c]);
      if constexpr (MASK) word[u] = bits[tc * words + (c >> 5)];
      load_row<R>(m + tc * R, mv[u]);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any FMA
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float v = xv[u];
      if constexpr (MASK) v = (word[u] >> (c & 31)) & 1u ? round16(v * scale) : 0.0f;
      v = (tb + u * kStride < n_tok && live) ? v : 0.0f;
#pragma unroll
      for (int j = 0; j < R; ++j) acc[j] = __builtin_fmaf(v, mv[u][j], acc[j]);
    }
  }
}

template <int R>
__global__ __launch_bounds__(64 * kWWaves) void lora_bwd_w_kernel(BwdWArgs a) {
  __shared__ float s_acc[kWWaves][kWCols][R + 1];
  int p = 0;
#pragma unroll
  for (int k = 1; k < 4; ++k) p += blockIdx.x >= a.first_block[k] ? 1 : 0;
  const int64_t c0 = (blockIdx.x - a.first_block[p]) * kWCols;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, cl = lane & (kWCols - 1);
  const int ph = lane / kWCols;
  const int64_t c = c0 + cl;
  const bool live = c < a.cols[p];
  const int64_t cc = live ? c : c0;  // column read (clamped into the problem)
  float acc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) acc[j] = 0.0f;
  if (a.bits[p])  // uniform over the block
    bwd_w_tokens<R, true>(acc, a.x[p], a.sx[p], a.bits[p], a.scale[p], a.m[p], cc, live, a.n_tok,
                          a.words, w * kWPh + ph);
  else
    bwd_w_tokens<R, false>(acc, a.x[p], a.sx[p], nullptr, 1.0f, a.m[p], cc, live, a.n_tok,
                           a.words, w * kWPh + ph);
#pragma unroll
  for (int j = 0; j < R; ++j) {  // the eight token phases of the column (same order every run)
    acc[j] += __shfl_xor(acc[j], 8, 64);
    acc[j] += __shfl_xor(acc[j], 16, 64);
    acc[j] += __shfl_xor(acc[j], 32, 64);
  }
  if (ph == 0) {
#pragma unroll
    for (int j = 0; j < R; ++j) s_acc[w][cl][j] = acc[j];
  }
  __syncthreads();
  for (int o = threadIdx.x; o < kWCols * R; o += 64 * kWWaves) {
    const int ci = o / R, j = o % R;
    const int64_t col = c0 + ci;
    if (col >= a.cols[p]) continue;
    float sum = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kWWaves; ++ww) sum += s_acc[ww][ci][j];
    const f16 hs = static_cast<f16>(sum);
    if (a.transposed[p])
      a.g[p][j * a.cols[p] + col] = hs;
    else
      a.g[p][col * R + j] = hs;
  }
}

bool rank_ok(int r) { return r == 4 || r == 8 || r == 16 || r == 32; }

int check_p(const char* fn, float pq, float pv) {
  if (!(pq >= 0.0f && pq < 1.0f && pv >= 0.0f && pv < 1.0f))
    return fail(RUS_ERR_INVALID, "%s: dropout probabilities must be in [0, 1)", fn);
  return RUS_OK;
}

}  // namespace
}  // namespace rus

using rus::f16;

extern "C" int rus_lora_down_fwd(const void* x, int64_t n_tokens, int64_t d, int64_t stride_x,
                                 const void* a_q, const void* a_v, int32_t r, void* mid_q,
                                 void* mid_v, const uint32_t* bits_q, const uint32_t* bits_v,
                                 float p_q, float p_v, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_down_fwd";
  if ((bits_q == nullptr) != (bits_v == nullptr))
    return fail(RUS_ERR_INVALID, "%s: give the keep bits of both branches or of neither", fn);
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (!x || !a_q || !a_v || !mid_q || !mid_v)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_tokens < 0 || d <= 0 || d % 16 || stride_x < d || stride_x % 8)
    return fail(RUS_ERR_INVALID, "%s: need d %% 16 == 0, stride_x >= d and stride_x %% 8 == 0",
                fn);
  if (!aligned(x, 16) || !aligned(a_q, 16) || !aligned(a_v, 16) || !aligned(mid_q, 2) ||
      !aligned(mid_v, 2) || !aligned(bits_q, 4) || !aligned(bits_v, 4))
    return fail(RUS_ERR_INVALID, "%s: x and A must be 16-byte aligned", fn);
  if (int e = check_p(fn, p_q, p_v)) return e;
  if (n_tokens >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  if (n_tokens == 0) return RUS_OK;
  DownArgs a{static_cast<const f16*>(x), stride_x, n_tokens, d,
             static_cast<const f16*>(a_q), static_cast<const f16*>(a_v),
             static_cast<f16*>(mid_q), static_cast<f16*>(mid_v), bits_q, bits_v,
             (d + 31) / 32, bits_q ? 1.0f / (1.0f - p_q) : 1.0f,
             bits_v ? 1.0f / (1.0f - p_v) : 1.0f};
  const dim3 grid(static_cast<uint32_t>((n_tokens + kTok - 1) / kTok));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_DOWN(RR)                                                                  \
  case RR:                                                                            \
    if (bits_q)                                                                       \
      hipLaunchKernelGGL((lora_down_kernel<RR, true>), grid, dim3(64 * Cfg<RR>::W), 0, st, a); \
    else                                                                              \
      hipLaunchKernelGGL((lora_down_kernel<RR, false>), grid, dim3(64 * Cfg<RR>::W), 0, st, a); \
    break;
  switch (r) { RUS_DOWN(4) RUS_DOWN(8) RUS_DOWN(16) RUS_DOWN(32) }
#undef RUS_DOWN
  return check_launch(fn);
}

extern "C" int rus_lora_bwd_x(const void* dq_lora, const void* dv_lora, int64_t n_tokens,
                              int64_t d_q, int64_t d_v, const void* a_t_q, const void* a_t_v,
                              const void* b_t_q, const void* b_t_v, int32_t r, int64_t d,
                              void* d_mid_q, void* d_mid_v, void* dx, int64_t stride_dx,
                              const uint32_t* bits_q, const uint32_t* bits_v, float p_q,
                              float p_v, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_bwd_x";
  if ((bits_q == nullptr) != (bits_v == nullptr))
    return fail(RUS_ERR_INVALID, "%s: give the keep bits of both branches or of neither", fn);
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (!dq_lora || !dv_lora || !a_t_q || !a_t_v || !b_t_q || !b_t_v || !d_mid_q || !d_mid_v || !dx)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_tokens < 0 || d <= 0 || d % 32 || d_q <= 0 || d_q % 16 || d_v <= 0 || d_v % 16 ||
      stride_dx < d || stride_dx % 4)
    return fail(RUS_ERR_INVALID, "%s: need d %% 32 == 0, d_q and d_v multiples of 16, "
                "stride_dx >= d and a multiple of 4", fn);
  const uintptr_t a_al = r >= 8 ? 16 : 8;
  if (!aligned(dq_lora, 16) || !aligned(dv_lora, 16) || !aligned(a_t_q, a_al) ||
      !aligned(a_t_v, a_al) || !aligned(b_t_q, 16) || !aligned(b_t_v, 16) || !aligned(dx, 8) ||
      !aligned(d_mid_q, 2) || !aligned(d_mid_v, 2) || !aligned(bits_q, 4) || !aligned(bits_v, 4))
    return fail(RUS_ERR_INVALID, "%s: misaligned operand", fn);
  if (int e = check_p(fn, p_q, p_v)) return e;
  if (n_tokens >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  if (n_tokens == 0) return RUS_OK;
  BwdXArgs a{static_cast<const f16*>(dq_lora), static_cast<const f16*>(dv_lora), n_tokens, d_q,
             d_v, static_cast<const f16*>(a_t_q), static_cast<const f16*>(a_t_v),
             static_cast<const f16*>(b_t_q), static_cast<const f16*>(b_t_v), d,
             static_cast<f16*>(d_mid_q), static_cast<f16*>(d_mid_v), static_cast<f16*>(dx),
             stride_dx, bits_q, bits_v, (d + 31) / 32,
             bits_q ? 1.0f / (1.0f - p_q) : 1.0f, bits_v ? 1.0f / (1.0f - p_v) : 1.0f};
  const dim3 grid(static_cast<uint32_t>((n_tokens + kTok - 1) / kTok));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_BX(RR)                                                                    \
  case RR:                                                                            \
    if (bits_q)                                                                       \
      hipLaunchKernelGGL((lora_bwd_x_kernel<RR, true>), grid, dim3(64 * Cfg<RR>::W), 0, st, a); \
    else                                                                              \
      hipLaunchKernelGGL((lora_bwd_x_kernel<RR, false>), grid, dim3(64 * Cfg<RR>::W), 0, st, a); \
    break;
  switch (r) { RUS_BX(4) RUS_BX(8) RUS_BX(16) RUS_BX(32) }
#undef RUS_BX
  return check_launch(fn);
}

extern "C" int rus_lora_bwd_w(const void* x, int64_t stride_x, const uint32_t* bits_q,
                              const uint32_t* bits_v, float p_q, float p_v, const void* dq_lora,
                              const void* dv_lora, const void* mid_q, const void* mid_v,
                              const void* d_mid_q, const void* d_mid_v, int64_t n_tokens,
                              int64_t d, int64_t d_q, int64_t d_v, int32_t r, void* g_a_q,
                              void* g_b_q, void* g_a_v, void* g_b_v, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_bwd_w";
  if ((bits_q == nullptr) != (bits_v == nullptr))
    return fail(RUS_ERR_INVALID, "%s: give the keep bits of both branches or of neither", fn);
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (!x || !dq_lora || !dv_lora || !mid_q || !mid_v || !d_mid_q || !d_mid_v || !g_a_q ||
      !g_b_q || !g_a_v || !g_b_v)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (n_tokens < 0 || d <= 0 || d_q <= 0 || d_v <= 0 || stride_x < d)
    return fail(RUS_ERR_INVALID, "%s: bad lengths", fn);
  if (!aligned(mid_q, 8) || !aligned(mid_v, 8) || !aligned(d_mid_q, 8) || !aligned(d_mid_v, 8) ||
      !aligned(bits_q, 4) || !aligned(bits_v, 4))
    return fail(RUS_ERR_INVALID, "%s: [N, r] operands must be 8-byte aligned", fn);
  if (int e = check_p(fn, p_q, p_v)) return e;
  if (n_tokens >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  BwdWArgs a;
  const f16* xs[4] = {static_cast<const f16*>(x), static_cast<const f16*>(dq_lora),
                      static_cast<const f16*>(x), static_cast<const f16*>(dv_lora)};
  const int64_t sxs[4] = {stride_x, d_q, stride_x, d_v};
  const uint32_t* bs[4] = {bits_q, nullptr, bits_v, nullptr};
  const float sc[4] = {bits_q ? 1.0f / (1.0f - p_q) : 1.0f, 1.0f,
                       bits_v ? 1.0f / (1.0f - p_v) : 1.0f, 1.0f};
  const void* ms[4] = {d_mid_q, mid_q, d_mid_v, mid_v};
  void* gs[4] = {g_a_q, g_b_q, g_a_v, g_b_v};
  const int64_t cols[4] = {d, d_q, d, d_v};
  a.first_block[0] = 0;
  for (int k = 0; k < 4; ++k) {
    a.x[k] = xs[k];
    a.sx[k] = sxs[k];
    a.bits[k] = bs[k];
    a.scale[k] = sc[k];
    a.m[k] = static_cast<const f16*>(ms[k]);
    a.g[k] = static_cast<f16*>(gs[k]);
    a.cols[k] = cols[k];
    a.transposed[k] = (k % 2 == 0) ? 1 : 0;
    a.first_block[k + 1] = a.first_block[k] + (cols[k] + kWCols - 1) / kWCols;
  }
  a.n_tok = n_tokens;
  a.words = (d + 31) / 32;
  const dim3 grid(static_cast<uint32_t>(a.first_block[4]));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_BW(RR)                                                                       \
  case RR:                                                                               \
    hipLaunchKernelGGL(lora_bwd_w_kernel<RR>, grid, dim3(64 * kWWaves), 0, st, a);       \
    break;
  switch (r) { RUS_BW(4) RUS_BW(8) RUS_BW(16) RUS_BW(32) }
#undef RUS_BW
  return check_launch(fn);
}
