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
// generator and no dropped copy of x is stored.
//
// The products are tiny (r = 16) but stream megabytes, so every kernel spreads its bytes over
// many short blocks:
//   * the rank-r reductions over D (mid) and over Dq + Dv (d_mid) are split: block (reduction
//     chunk, 32-token tile) forms an fp32 partial on MFMA (v_mfma_f32_32x32x16_f16, tokens x
//     ranks; q and v packed into one 32-column accumulator for r <= 16), and the last block of a
//     tile to finish (per-tile arrival counter) sums the chunks' partials in chunk order and
//     rounds once: deterministic, in the same launch;
//   * the expansion d_mid A runs as MFMA tiles of dx^T (32 columns x 32 tokens per wave) with the
//     masks and both rounded adds into dx in place;
//   * the weight gradients (reductions over tokens) run on the vector units, one lane per output
//     column, the tokens split over the waves of a block and over blocks, summed through LDS and
//     then across blocks by the same last-block rule;
//   * q_lora / v_lora are formed inside the RoPE kernel from mid and B (rope.hip).
// Every value the reference rounds to fp16 is rounded here at the same point; sums are fp32.
// The loads of a batch are issued before any of their uses (a scheduling barrier keeps the
// compiler from sinking them), so a wave waits on memory once per batch.
//
// Workspace: fp32 partials (rus_lora_workspace_size) and int32 arrival counters that are zero
// when a launch starts and are left zero by it. Launches that share counters must not overlap.

#include <mutex>

#include "common.h"
#include "lora_rows.h"

namespace rus {
namespace {

constexpr int kTok = 32;  // tokens per tile (down, d_mid, expansion)
constexpr int kSW = 4;    // waves per block (down, d_mid, expansion)

// Accumulator row of register r for lane half h (v_mfma_f32_32x32x16: lane l holds column l % 32).
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

__device__ __forceinline__ float round16(float x) { return static_cast<float>(from_f32<f16>(x)); }

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

// Accumulator layout of the tokens x ranks products: for R <= 16 the q and v results share one
// 32-column accumulator (q in columns 0 .. R-1, v in R .. 2R-1); for R = 32 each branch has its
// own.
template <int R>
struct Cfg {
  static constexpr bool PACK = R <= 16;
  static constexpr int NACC = PACK ? 1 : 2;
};

// Branch and rank of column n of accumulator j (branch -1: unused column).
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

// Split-K end of the tokens x ranks kernels: the waves' accumulators are summed through LDS in
// wave order into this block's partial part[chunk][tile] (NACC x 1024 fp32 in accumulator
// order); the last block of the tile sums every chunk's partial in chunk order into tot
// (element e = threadIdx.x + 256 k of the accumulator order) and returns true.
template <int NACC>
__device__ __forceinline__ bool split_reduce(const f32x16 (&acc)[NACC], float* s_park,
                                             float* __restrict__ part, int* __restrict__ counters,
                                             int chunk, int n_chunks, int tile, int n_tiles,
                                             float (&tot)[NACC * 4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < NACC; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s_park[((wave * NACC + j) * 16 + r) * 64 + lane] = acc[j][r];
  __syncthreads();
  constexpr int kTile = NACC * 1024;  // floats per partial
  float* mine = part + (static_cast<int64_t>(chunk) * n_tiles + tile) * kTile;
#pragma unroll
  for (int k = 0; k < NACC * 4; ++k) {
    const int e = threadIdx.x + 256 * k;  // (j, r, lane) = (e >> 10, (e >> 6) & 15, e & 63)
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kSW; ++w) s += s_park[w * kTile + e];
    store_partial(mine + e, s);
  }
  if (!arrive_last(counters + tile, n_chunks)) return false;
#pragma unroll
  for (int k = 0; k < NACC * 4; ++k) tot[k] = 0.0f;
  // The partials of kB chunks are loaded together, then added in chunk order.
  constexpr int kB = NACC == 1 ? 8 : 4;
  for (int c0 = 0; c0 < n_chunks; c0 += kB) {
    float v[kB][NACC * 4];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const int c = min(c0 + b, n_chunks - 1);
      const float* pc = part + (static_cast<int64_t>(c) * n_tiles + tile) * kTile;
#pragma unroll
      for (int k = 0; k < NACC * 4; ++k) v[b][k] = load_partial(pc + threadIdx.x + 256 * k);
    }
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
      for (int k = 0; k < NACC * 4; ++k) tot[k] += c0 + b < n_chunks ? v[b][k] : 0.0f;
  }
  return true;
}

// Stores the totals of split_reduce as fp16 [n_tok, R] rows of the two branches' outputs.
template <int R>
__device__ __forceinline__ void store_ranks(const float (&tot)[Cfg<R>::NACC * 4], int64_t t0,
                                            int64_t n_tok, f16* out_q, f16* out_v) {
#pragma unroll
  for (int k = 0; k < Cfg<R>::NACC * 4; ++k) {
    const int e = threadIdx.x + 256 * k;
    const int ln = e & 63, r = (e >> 6) & 15, j = e >> 10;
    int br, rank;
    col_owner<R>(j, ln & 31, br, rank);
    const int64_t tt = t0 + acc_row(r, ln >> 5);
    if (br >= 0 && tt < n_tok) (br ? out_v : out_q)[tt * R + rank] = from_f32<f16>(tot[k]);
  }
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
  float* part;
  int* counters;
  int kc;  // reduction columns per chunk (a multiple of 16 dividing d)
};

// mid_q = fp16(drop_q(x) A_q^T), mid_v = fp16(drop_v(x) A_v^T). Block (chunk, tile) reduces
// columns [chunk kc, +kc) for 32 tokens: the A operand is 8 dropped x values of the lane's
// token, the B operand 8 entries of the A row owning the lane's column (zeros if unused).
template <int R, bool DROP>
__global__ __launch_bounds__(64 * kSW) void lora_down_kernel(DownArgs a) {
  using C = Cfg<R>;
  constexpr int NACC = C::NACC, U = 2;
  __shared__ float s_park[kSW * NACC * 1024];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const int chunk = blockIdx.x, tile = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(tile) * kTok;
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
  const int ks = a.kc / 16, c_base = chunk * a.kc;
  f32x16 acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) acc[j] = f32x16{};
  for (int s0 = wave; s0 < ks; s0 += kSW * U) {
    f16x8 xs[U], f0[U], f1[U];
    uint32_t wq[U], wv[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int c0 = c_base + 16 * min(s0 + kSW * i, ks - 1) + 8 * h;
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
      // Steps past the chunk add zero products: no branch, so the batch's loads stay in front.
      if (s0 + kSW * i >= ks) xs[i] = zero8();
      const int shc = (c_base + 16 * min(s0 + kSW * i, ks - 1) + 8 * h) & 31;  // bit of value 0
      if constexpr (C::PACK) {
        if constexpr (DROP) {
          acc[0] = mfma(drop8(xs[i], wq[i], shc, a.scale_q), br0 == 0 ? f0[i] : zero8(), acc[0]);
          acc[0] = mfma(drop8(xs[i], wv[i], shc, a.scale_v), br0 == 1 ? f0[i] : zero8(), acc[0]);
        } else {
          acc[0] = mfma(xs[i], br0 >= 0 ? f0[i] : zero8(), acc[0]);
        }
      } else {
        const f16x8 xq = DROP ? drop8(xs[i], wq[i], shc, a.scale_q) : xs[i];
        const f16x8 xv = DROP ? drop8(xs[i], wv[i], shc, a.scale_v) : xs[i];
        acc[0] = mfma(xq, f0[i], acc[0]);
        acc[NACC - 1] = mfma(xv, f1[i], acc[NACC - 1]);
      }
    }
  }
  float tot[NACC * 4];
  if (split_reduce<NACC>(acc, s_park, a.part, a.counters, chunk, gridDim.x, tile, gridDim.y, tot))
    store_ranks<R>(tot, t0, a.n_tok, a.mid_q, a.mid_v);
}

struct MidArgs {
  const f16* dq;
  const f16* dv;
  int64_t n_tok, len_q, len_v;
  const f16* bt_q;  // B^T [R, len]
  const f16* bt_v;
  f16* dmid_q;
  f16* dmid_v;
  float* part;
  int* counters;
  int kc, chunks_q;  // chunks [0, chunks_q) reduce dq, the rest dv
};

// d_mid_q = fp16(dq B_q), d_mid_v = fp16(dv B_v): block (chunk, tile) reduces 32 tokens over kc
// columns of dq (or of dv) against the B^T row owning the lane's column.
template <int R>
__global__ __launch_bounds__(64 * kSW) void lora_bwd_mid_kernel(MidArgs a) {
  using C = Cfg<R>;
  constexpr int NACC = C::NACC, U = 2;
  __shared__ float s_park[kSW * NACC * 1024];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const int chunk = blockIdx.x, tile = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(tile) * kTok;
  const int64_t t = min(t0 + col, a.n_tok - 1);
  int br0, rk0;
  col_owner<R>(0, col, br0, rk0);
  const bool is_q = chunk < a.chunks_q;  // uniform over the block
  const bool use = C::PACK ? br0 == (is_q ? 0 : 1) : true;
  const int64_t len = is_q ? a.len_q : a.len_v;
  const f16* xrow = (is_q ? a.dq : a.dv) + t * len;
  const f16* brow = (is_q ? a.bt_q : a.bt_v) + (C::PACK ? (use ? rk0 : 0) : col) * len;
  const int c_base = (is_q ? chunk : chunk - a.chunks_q) * a.kc;
  const int ks = a.kc / 16;
  f32x16 acc[NACC];
#pragma unroll
  for (int j = 0; j < NACC; ++j) acc[j] = f32x16{};
  f32x16 sum = f32x16{};
  for (int s0 = wave; s0 < ks; s0 += kSW * U) {
    f16x8 xs[U], fs[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int c0 = c_base + 16 * min(s0 + kSW * i, ks - 1) + 8 * h;
      xs[i] = ld8(xrow + c0);
      fs[i] = ld8(brow + c0);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any MFMA
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const f16x8 xi = s0 + kSW * i < ks ? xs[i] : zero8();
      sum = mfma(xi, use ? fs[i] : zero8(), sum);
    }
  }
  // The chunk's branch owns accumulator 0 (PACK: both branches share it) or NACC - 1 (v, R = 32).
  if (C::PACK || is_q)
    acc[0] = sum;
  else
    acc[NACC - 1] = sum;
  float tot[NACC * 4];
  if (split_reduce<NACC>(acc, s_park, a.part, a.counters, chunk, gridDim.x, tile, gridDim.y, tot))
    store_ranks<R>(tot, t0, a.n_tok, a.dmid_q, a.dmid_v);
}

struct ExpandArgs {
  const f16* dmid_q;
  const f16* dmid_v;
  const f16* at_q;  // A^T [d, R]
  const f16* at_v;
  int64_t n_tok, d;
  f16* dx;
  int64_t sdx;
  const uint32_t* bits_q;
  const uint32_t* bits_v;
  int64_t words;
  float scale_q, scale_v;
};

// dx = fp16(fp16(dx + fp16(drop_q(fp16(d_mid_q A_q)))) + fp16(drop_v(fp16(d_mid_v A_v)))).
// Block (column group, tile): wave w forms the dx^T tiles of columns 32 (4 group + w) .. +31 and
// the tile's 32 tokens (MFMA over the ranks), then updates dx for its lane's token in place.
// One wave's dx^T tile: columns 32 dt .. +31, tokens t0 .. t0 + 31 (no barrier: the caller may
// return early per wave).
template <int R, bool DROP>
__device__ __forceinline__ void expand_wave(const ExpandArgs& a, int dt, int64_t t0) {
  constexpr int KS = R > 16 ? 2 : 1;
  const int lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  if (dt * 32 >= a.d) return;
  const int64_t t = min(t0 + col, a.n_tok - 1);  // this lane's token (column of dx^T)
  const int64_t drow = static_cast<int64_t>(dt) * 32 + col;  // A-operand row of this lane
  f16x8 aq[KS], av[KS], mq[KS], mv[KS];
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    aq[j] = frag_rank<R>(a.at_q + drow * R, 16 * j + 8 * h);
    av[j] = frag_rank<R>(a.at_v + drow * R, 16 * j + 8 * h);
    mq[j] = frag_rank<R>(a.dmid_q + t * R, 16 * j + 8 * h);
    mv[j] = frag_rank<R>(a.dmid_v + t * R, 16 * j + 8 * h);
  }
  f16* p = a.dx + t * a.sdx + static_cast<int64_t>(dt) * 32;
  f16x4 cur[4];
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) cur[r4] = *reinterpret_cast<const f16x4*>(p + 8 * r4 + 4 * h);
  const uint32_t wq = DROP ? a.bits_q[t * a.words + dt] : 0xffffffffu;
  const uint32_t wv = DROP ? a.bits_v[t * a.words + dt] : 0xffffffffu;
  __builtin_amdgcn_sched_barrier(0);  // every load is issued before any MFMA
  f32x16 oq = f32x16{}, ov = f32x16{};
#pragma unroll
  for (int j = 0; j < KS; ++j) {
    oq = mfma(aq[j], mq[j], oq);
    ov = mfma(av[j], mv[j], ov);
  }
  if (t0 + col >= a.n_tok) return;
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) {
    const int off = 8 * r4 + 4 * h;
    f16x4 c = cur[r4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = 4 * r4 + k, bit = off + k;
      const float hq = round16(oq[r]), hv = round16(ov[r]);  // fp16 dx_q, dx_v
      const float tq = round16((wq >> bit) & 1u ? hq * a.scale_q : 0.0f);
      const float tv = round16((wv >> bit) & 1u ? hv * a.scale_v : 0.0f);
      c[k] = from_f32<f16>(round16(static_cast<float>(c[k]) + tq) + tv);
    }
    *reinterpret_cast<f16x4*>(p + off) = c;
  }
}

template <int R, bool DROP>
__global__ __launch_bounds__(64 * kSW) void lora_bwd_expand_kernel(ExpandArgs a) {
  expand_wave<R, DROP>(a, blockIdx.x * kSW + (threadIdx.x >> 6),
                       static_cast<int64_t>(blockIdx.y) * kTok);
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
// M = mid_q, G [Dq, R]), A_v, B_v. Block (column block, token chunk): 64 columns, one per lane,
// x kWTok tokens split over kWWaves waves; partials [R][64] are summed across the chunks of a
// column block by its last block.
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
  float* part;
  int* counters;
};

constexpr int kWCols = 64;   // columns per block
constexpr int kWWaves = 8;   // waves per block
constexpr int kWTok = 128;   // tokens per chunk

// acc[j] += sum over tokens first, first + kWWaves, ... < t_end of X[t, c] * M[t, j] (X dropped
// with the keep bits when MASK) in batches of U whose loads are issued together; past the end
// (or for a dead column) the weight is zero.
template <int R, bool MASK>
__device__ __forceinline__ void bwd_w_tokens(float (&acc)[R], const f16* __restrict__ x,
                                             int64_t sx, const uint32_t* __restrict__ bits,
                                             float scale, const f16* __restrict__ m, int64_t c,
                                             bool live, int64_t first, int64_t t_end,
                                             int64_t words) {
  constexpr int U = R >= 32 ? 4 : 8;  // smaller batches keep 32 accumulators in registers
  for (int64_t tb = first; tb < t_end; tb += U * kWWaves) {
    float xv[U], mv[U][R];
    uint32_t word[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t tt = tb + u * kWWaves;
      const int64_t tc = tt < t_end ? tt : t_end - 1;
      xv[u] = static_cast<float>(x[tc * sx + c]);
      if constexpr (MASK) word[u] = bits[tc * words + (c >> 5)];
      load_row<R>(m + tc * R, mv[u]);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the batch is issued before any FMA
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float v = xv[u];
      if constexpr (MASK) v = (word[u] >> (c & 31)) & 1u ? round16(v * scale) : 0.0f;
      v = (tb + u * kWWaves < t_end && live) ? v : 0.0f;
#pragma unroll
      for (int j = 0; j < R; ++j) acc[j] = __builtin_fmaf(v, mv[u][j], acc[j]);
    }
  }
}

// Block (blk, chunk) of the n_blk x n_chunk weight-gradient grid.
template <int R>
__device__ __forceinline__ void bwd_w_block(const BwdWArgs& a, int blk, int chunk, int n_blk,
                                            int n_chunk) {
  constexpr int RS = R < 16 ? R : 16;  // ranks summed through LDS per pass
  __shared__ float s_acc[kWWaves][RS][kWCols];
  int p = 0;
#pragma unroll
  for (int k = 1; k < 4; ++k) p += blk >= a.first_block[k] ? 1 : 0;
  const int64_t c0 = (blk - a.first_block[p]) * kWCols;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t c = c0 + lane;
  const bool live = c < a.cols[p];
  const int64_t cc = live ? c : c0;  // column read (clamped into the problem)
  const int64_t t_begin = static_cast<int64_t>(chunk) * kWTok;
  const int64_t t_end = min(t_begin + kWTok, a.n_tok);
  float acc[R];
#pragma unroll
  for (int j = 0; j < R; ++j) acc[j] = 0.0f;
  if (a.bits[p])  // uniform over the block
    bwd_w_tokens<R, true>(acc, a.x[p], a.sx[p], a.bits[p], a.scale[p], a.m[p], cc, live,
                          t_begin + w, t_end, a.words);
  else
    bwd_w_tokens<R, false>(acc, a.x[p], a.sx[p], nullptr, 1.0f, a.m[p], cc, live, t_begin + w,
                           t_end, a.words);
  constexpr int kPart = R * kWCols;  // floats per partial, rank-major [R][64]
  float* mine = a.part + (static_cast<int64_t>(chunk) * n_blk + blk) * kPart;
#pragma unroll
  for (int j0 = 0; j0 < R; j0 += RS) {
#pragma unroll
    for (int j = 0; j < RS; ++j) s_acc[w][j][lane] = acc[j0 + j];
    __syncthreads();
    for (int o = threadIdx.x; o < RS * kWCols; o += 64 * kWWaves) {
      float s = 0.0f;
#pragma unroll
      for (int ww = 0; ww < kWWaves; ++ww) s += s_acc[ww][o / kWCols][o % kWCols];
      store_partial(mine + j0 * kWCols + o, s);
    }
    __syncthreads();
  }
  if (!arrive_last(a.counters + blk, n_chunk)) return;
  // Every thread owns kO outputs; the partials of kB chunks are loaded together, then added in
  // chunk order.
  constexpr int kThr = 64 * kWWaves, kO = (kPart + kThr - 1) / kThr, kB = kO > 2 ? 4 : 8;
  const int n_ch = n_chunk;
  float tot[kO];
#pragma unroll
  for (int i = 0; i < kO; ++i) tot[i] = 0.0f;
  for (int ch0 = 0; ch0 < n_ch; ch0 += kB) {
    float v[kB][kO];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      const float* pc =
          a.part + (static_cast<int64_t>(min(ch0 + b, n_ch - 1)) * n_blk + blk) * kPart;
#pragma unroll
      for (int i = 0; i < kO; ++i) v[b][i] = load_partial(pc + min<int>(threadIdx.x + kThr * i, kPart - 1));
    }
#pragma unroll
    for (int b = 0; b < kB; ++b)
#pragma unroll
      for (int i = 0; i < kO; ++i) tot[i] += ch0 + b < n_ch ? v[b][i] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < kO; ++i) {
    const int o = threadIdx.x + kThr * i;
    const int j = o / kWCols;
    const int64_t col = c0 + o % kWCols;
    if (o >= kPart || col >= a.cols[p]) continue;
    const f16 hs = from_f32<f16>(tot[i]);
    if (a.transposed[p])
      a.g[p][j * a.cols[p] + col] = hs;
    else
      a.g[p][col * R + j] = hs;
  }
}

template <int R>
__global__ __launch_bounds__(64 * kWWaves) __attribute__((amdgpu_waves_per_eu(4)))
void lora_bwd_w_kernel(BwdWArgs a) {
  bwd_w_block<R>(a, blockIdx.x, blockIdx.y, gridDim.x, gridDim.y);
}

// The weight gradients and the input-gradient expansion in one launch (both read the finished
// d_mid): blocks [0, n_blk * n_chunk) are weight-gradient blocks (blk fastest), the rest
// expansion blocks of kWWaves column tiles of one 32-token tile each. Each block's role is
// uniform, so the weight-gradient blocks' barriers and arrival counters involve only them.
template <int R, bool DROP>
__global__ __launch_bounds__(64 * kWWaves) __attribute__((amdgpu_waves_per_eu(4)))
void lora_bwd_xw_kernel(BwdWArgs a, ExpandArgs x,
                                                                  int n_blk, int n_chunk,
                                                                  int x_col_blocks) {
  const int b = blockIdx.x;
  const int n_w = n_blk * n_chunk;
  if (b < n_w) {
    bwd_w_block<R>(a, b % n_blk, b / n_blk, n_blk, n_chunk);
    return;
  }
  const int e = b - n_w;
  expand_wave<R, DROP>(x, (e % x_col_blocks) * kWWaves + (threadIdx.x >> 6),
                       static_cast<int64_t>(e / x_col_blocks) * kTok);
}

// LoRA-down by row blocks (lora_rows.h): block b forms mid_q / mid_v of tokens 4b .. 4b + 3.
__global__ __launch_bounds__(256) void lora_down_rows_kernel(DownRows a) {
  __shared__ float park[kDownParkFloats];
  lora_down_rows4(a, static_cast<int64_t>(blockIdx.x) * kDownRows, park);
}

bool rank_ok(int r) { return r == 4 || r == 8 || r == 16 || r == 32; }

int check_p(const char* fn, float pq, float pv) {
  if (!(pq >= 0.0f && pq < 1.0f && pv >= 0.0f && pv < 1.0f))
    return fail(RUS_ERR_INVALID, "%s: dropout probabilities must be in [0, 1)", fn);
  return RUS_OK;
}

// Largest chunk of {128, 64, 32, 16} columns dividing both lengths (0: none).
int chunk_cols(int64_t a, int64_t b) {
  for (int kc = 128; kc >= 16; kc /= 2)
    if (a % kc == 0 && b % kc == 0) return kc;
  return 0;
}

int64_t tiles(int64_t n) { return (n + kTok - 1) / kTok; }

int64_t w_blocks(int64_t d, int64_t d_q, int64_t d_v) {
  return 2 * ((d + kWCols - 1) / kWCols) + (d_q + kWCols - 1) / kWCols +
         (d_v + kWCols - 1) / kWCols;
}

int64_t w_chunks(int64_t n) { return n > 0 ? (n + kWTok - 1) / kWTok : 1; }

// Workspace floats and counters of each entry point (see rus_lora_workspace_size).
void scratch_need(int which, int64_t n, int64_t d, int64_t d_q, int64_t d_v, int r,
                  int64_t& floats, int64_t& counters) {
  const int64_t per = (r > 16 ? 2 : 1) * 1024;  // floats per tokens x ranks partial
  floats = counters = 0;
  if (which == RUS_LORA_DOWN) {
    const int kc = chunk_cols(d, d);
    floats = kc ? (d / kc) * tiles(n) * per : 0;
    counters = tiles(n);
  } else if (which == RUS_LORA_BWD_X) {
    const int kc = chunk_cols(d_q, d_v);
    floats = kc ? (d_q / kc + d_v / kc) * tiles(n) * per : 0;
    counters = tiles(n);
  } else {
    const int64_t nb = w_blocks(d, d_q, d_v);
    floats = w_chunks(n) * nb * r * kWCols;
    counters = nb;
  }
}

constexpr int64_t kMaxCounters = 65536;  // bound on each entry point's counters

}  // namespace
}  // namespace rus

using rus::f16;

extern "C" int rus_lora_workspace_size(int32_t which, int64_t n_tokens, int64_t d, int64_t d_q,
                                       int64_t d_v, int32_t r, int64_t* workspace_floats,
                                       int64_t* n_counters) {
  using namespace rus;
  const char* fn = "rus_lora_workspace_size";
  if (which != RUS_LORA_DOWN && which != RUS_LORA_BWD_X && which != RUS_LORA_BWD_W)
    return fail(RUS_ERR_INVALID, "%s: unknown entry point %d", fn, which);
  if (!workspace_floats || !n_counters) return fail(RUS_ERR_INVALID, "%s: null output", fn);
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (n_tokens < 0 || d <= 0 || d_q <= 0 || d_v <= 0)
    return fail(RUS_ERR_INVALID, "%s: bad lengths", fn);
  scratch_need(which, n_tokens, d, d_q, d_v, r, *workspace_floats, *n_counters);
  return RUS_OK;
}

// Common checks of the workspace arguments.
static int check_scratch(const char* fn, int which, int64_t n, int64_t d, int64_t d_q,
                         int64_t d_v, int r, const float* workspace, int64_t workspace_floats,
                         const int32_t* counters, int64_t n_counters) {
  using namespace rus;
  if (!workspace || !counters) return fail(RUS_ERR_INVALID, "%s: null workspace or counters", fn);
  if (!aligned(workspace, 16) || !aligned(counters, 4))
    return fail(RUS_ERR_INVALID, "%s: misaligned workspace or counters", fn);
  int64_t need_f, need_c;
  scratch_need(which, n, d, d_q, d_v, r, need_f, need_c);
  if (need_c > kMaxCounters)
    return fail(RUS_ERR_UNSUPPORTED, "%s: needs %lld counters (at most %lld)", fn,
                static_cast<long long>(need_c), static_cast<long long>(kMaxCounters));
  if (workspace_floats < need_f || n_counters < need_c)
    return fail(RUS_ERR_INVALID, "%s: workspace holds %lld floats and %lld counters, needs %lld "
                "and %lld", fn, static_cast<long long>(workspace_floats),
                static_cast<long long>(n_counters), static_cast<long long>(need_f),
                static_cast<long long>(need_c));
  return RUS_OK;
}

static int lora_down(const char* fn, const void* x, int64_t n_tokens, int64_t d,
                     int64_t stride_x, const void* a_q, const void* a_v, int32_t r, void* mid_q,
                     void* mid_v, const uint32_t* bits_q, const uint32_t* bits_v, float p_q,
                     float p_v, float* workspace, int64_t workspace_floats, int32_t* counters,
                     int64_t n_counters, void* stream) {
  using namespace rus;
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
  if (int e = check_scratch(fn, RUS_LORA_DOWN, n_tokens, d, 16, 16, r, workspace,
                            workspace_floats, counters, n_counters))
    return e;
  if (n_tokens == 0) return RUS_OK;
  const int kc = chunk_cols(d, d);
  if (tiles(n_tokens) > 65535) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  DownArgs a{static_cast<const f16*>(x), stride_x, n_tokens, d,
             static_cast<const f16*>(a_q), static_cast<const f16*>(a_v),
             static_cast<f16*>(mid_q), static_cast<f16*>(mid_v), bits_q, bits_v,
             (d + 31) / 32, bits_q ? 1.0f / (1.0f - p_q) : 1.0f,
             bits_v ? 1.0f / (1.0f - p_v) : 1.0f, workspace, counters, kc};
  const dim3 grid(static_cast<uint32_t>(d / kc), static_cast<uint32_t>(tiles(n_tokens)));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_DOWN(RR)                                                                      \
  case RR:                                                                                \
    if (bits_q)                                                                           \
      hipLaunchKernelGGL((lora_down_kernel<RR, true>), grid, dim3(64 * kSW), 0, st, a);  \
    else                                                                                  \
      hipLaunchKernelGGL((lora_down_kernel<RR, false>), grid, dim3(64 * kSW), 0, st, a); \
    break;
  switch (r) { RUS_DOWN(4) RUS_DOWN(8) RUS_DOWN(16) RUS_DOWN(32) }
#undef RUS_DOWN
  return check_launch(fn);
}

extern "C" int rus_lora_down_fwd(const void* x, int64_t n_tokens, int64_t d, int64_t stride_x,
                                 const void* a_q, const void* a_v, int32_t r, void* mid_q,
                                 void* mid_v, const uint32_t* bits_q, const uint32_t* bits_v,
                                 float p_q, float p_v, float* workspace, int64_t workspace_floats,
                                 int32_t* counters, int64_t n_counters, void* stream) {
  return lora_down("rus_lora_down_fwd", x, n_tokens, d, stride_x, a_q, a_v, r, mid_q, mid_v,
                   bits_q, bits_v, p_q, p_v, workspace, workspace_floats, counters, n_counters,
                   stream);
}

// ---------------------------------------------------------------------------------------------
// rus_lora_down_fwd_noalloc: the same launch with its workspace and counters in a file-scope
// device array, for callers that cannot allocate. Each device holds its own copy of the array
// (16 MiB of fp32 partials + 16 KiB of counters) until the process ends; its address on a device
// is taken once with hipGetSymbolAddress and kept, and the counters are cleared then (every launch
// leaves them zero). All calls on one device share the array: calls that overlap on one device
// race.
// ---------------------------------------------------------------------------------------------

namespace rus {
namespace {
constexpr int64_t kNoAllocFloats = int64_t(1) << 22;
constexpr int64_t kNoAllocCounters = 4096;
constexpr int kMaxDevices = 64;
}  // namespace
}  // namespace rus

static __device__ __align__(256) float scratch[rus::kNoAllocFloats + rus::kNoAllocCounters];

namespace rus {
namespace {

__global__ __launch_bounds__(256) void zero_words_kernel(int32_t* p, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    p[i] = 0;
}

std::mutex g_noalloc_mutex;
float* g_noalloc_base[kMaxDevices] = {};

// The current device's copy of `scratch` (address taken on the first call on that device, when
// its counters are also cleared on `stream`).
int noalloc_scratch(const char* fn, void* stream, float** base) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(RUS_ERR_LAUNCH, "%s: no current device (%s)", fn, hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_noalloc_mutex);
  if (!g_noalloc_base[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(RUS_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn,
                  dev, hipGetErrorString(e));
    float* f = static_cast<float*>(p);
    hipLaunchKernelGGL(zero_words_kernel, dim3(16), dim3(256), 0,
                       static_cast<hipStream_t>(stream),
                       reinterpret_cast<int32_t*>(f + kNoAllocFloats), kNoAllocCounters);
    if (int rc = check_launch(fn)) return rc;
    g_noalloc_base[dev] = f;
  }
  *base = g_noalloc_base[dev];
  return RUS_OK;
}

}  // namespace
}  // namespace rus

extern "C" int rus_lora_down_fwd_noalloc(const void* x, int64_t n_tokens, int64_t d,
                                         int64_t stride_x, const void* a_q, const void* a_v,
                                         int32_t r, void* mid_q, void* mid_v,
                                         const uint32_t* bits_q, const uint32_t* bits_v,
                                         float p_q, float p_v, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_down_fwd_noalloc";
  if (!rank_ok(r)) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  if (n_tokens < 0 || d <= 0 || d % 16)
    return fail(RUS_ERR_INVALID, "%s: need n_tokens >= 0 and d %% 16 == 0", fn);
  int64_t need_f = 0, need_c = 0;
  scratch_need(RUS_LORA_DOWN, n_tokens, d, 16, 16, r, need_f, need_c);
  if (need_f > kNoAllocFloats || need_c > kNoAllocCounters)
    return fail(RUS_ERR_UNSUPPORTED,
                "%s: n_tokens=%lld, d=%lld, r=%d need %lld scratch floats and %lld counters; the "
                "static scratch holds %lld and %lld (use rus_lora_down_fwd with a workspace)",
                fn, static_cast<long long>(n_tokens), static_cast<long long>(d), r,
                static_cast<long long>(need_f), static_cast<long long>(need_c),
                static_cast<long long>(kNoAllocFloats), static_cast<long long>(kNoAllocCounters));
  float* base = nullptr;
  if (int e = noalloc_scratch(fn, stream, &base)) return e;
  return lora_down(fn, x, n_tokens, d, stride_x, a_q, a_v, r, mid_q, mid_v, bits_q, bits_v, p_q,
                   p_v, base, kNoAllocFloats, reinterpret_cast<int32_t*>(base + kNoAllocFloats),
                   kNoAllocCounters, stream);
}

extern "C" int rus_lora_bwd_x(const void* dq_lora, const void* dv_lora, int64_t n_tokens,
                              int64_t d_q, int64_t d_v, const void* a_t_q, const void* a_t_v,
                              const void* b_t_q, const void* b_t_v, int32_t r, int64_t d,
                              void* d_mid_q, void* d_mid_v, void* dx, int64_t stride_dx,
                              const uint32_t* bits_q, const uint32_t* bits_v, float p_q,
                              float p_v, float* workspace, int64_t workspace_floats,
                              int32_t* counters, int64_t n_counters, void* stream) {
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
      !aligned(d_mid_q, a_al) || !aligned(d_mid_v, a_al) || !aligned(bits_q, 4) ||
      !aligned(bits_v, 4))
    return fail(RUS_ERR_INVALID, "%s: misaligned operand", fn);
  if (int e = check_p(fn, p_q, p_v)) return e;
  if (n_tokens >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  if (int e = check_scratch(fn, RUS_LORA_BWD_X, n_tokens, d, d_q, d_v, r, workspace,
                            workspace_floats, counters, n_counters))
    return e;
  if (n_tokens == 0) return RUS_OK;
  if (tiles(n_tokens) > 65535) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  const int kc = chunk_cols(d_q, d_v);
  MidArgs m{static_cast<const f16*>(dq_lora), static_cast<const f16*>(dv_lora), n_tokens, d_q,
            d_v, static_cast<const f16*>(b_t_q), static_cast<const f16*>(b_t_v),
            static_cast<f16*>(d_mid_q), static_cast<f16*>(d_mid_v), workspace, counters, kc,
            static_cast<int>(d_q / kc)};
  ExpandArgs x{static_cast<const f16*>(d_mid_q), static_cast<const f16*>(d_mid_v),
               static_cast<const f16*>(a_t_q), static_cast<const f16*>(a_t_v), n_tokens, d,
               static_cast<f16*>(dx), stride_dx, bits_q, bits_v, (d + 31) / 32,
               bits_q ? 1.0f / (1.0f - p_q) : 1.0f, bits_v ? 1.0f / (1.0f - p_v) : 1.0f};
  const dim3 grid_m(static_cast<uint32_t>(d_q / kc + d_v / kc),
                    static_cast<uint32_t>(tiles(n_tokens)));
  const dim3 grid_x(static_cast<uint32_t>((d / 32 + kSW - 1) / kSW),
                    static_cast<uint32_t>(tiles(n_tokens)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 blk(64 * kSW);
#define RUS_BX(RR)                                                                    \
  case RR:                                                                            \
    hipLaunchKernelGGL((lora_bwd_mid_kernel<RR>), grid_m, blk, 0, st, m);             \
    if (int e = check_launch(fn)) return e;                                           \
    if (bits_q)                                                                       \
      hipLaunchKernelGGL((lora_bwd_expand_kernel<RR, true>), grid_x, blk, 0, st, x);  \
    else                                                                              \
      hipLaunchKernelGGL((lora_bwd_expand_kernel<RR, false>), grid_x, blk, 0, st, x); \
    break;
  switch (r) { RUS_BX(4) RUS_BX(8) RUS_BX(16) RUS_BX(32) }
#undef RUS_BX
  return check_launch(fn);
}

// Checks and fills the weight-gradient arguments shared by rus_lora_bwd_w and rus_lora_bwd_xw.
static int bwd_w_args(const char* fn, const void* x, int64_t stride_x, const uint32_t* bits_q,
                      const uint32_t* bits_v, float p_q, float p_v, const void* dq_lora,
                      const void* dv_lora, const void* mid_q, const void* mid_v,
                      const void* d_mid_q, const void* d_mid_v, int64_t n_tokens, int64_t d,
                      int64_t d_q, int64_t d_v, int32_t r, void* g_a_q, void* g_b_q,
                      void* g_a_v, void* g_b_v, float* workspace, int64_t workspace_floats,
                      int32_t* counters, int64_t n_counters, rus::BwdWArgs& a) {
  using namespace rus;
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
  if (int e = check_scratch(fn, RUS_LORA_BWD_W, n_tokens, d, d_q, d_v, r, workspace,
                            workspace_floats, counters, n_counters))
    return e;
  if (w_chunks(n_tokens) > 65535) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
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
  a.part = workspace;
  a.counters = counters;
  return RUS_OK;
}

extern "C" int rus_lora_bwd_w(const void* x, int64_t stride_x, const uint32_t* bits_q,
                              const uint32_t* bits_v, float p_q, float p_v, const void* dq_lora,
                              const void* dv_lora, const void* mid_q, const void* mid_v,
                              const void* d_mid_q, const void* d_mid_v, int64_t n_tokens,
                              int64_t d, int64_t d_q, int64_t d_v, int32_t r, void* g_a_q,
                              void* g_b_q, void* g_a_v, void* g_b_v, float* workspace,
                              int64_t workspace_floats, int32_t* counters, int64_t n_counters,
                              void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_bwd_w";
  BwdWArgs a;
  if (int e = bwd_w_args(fn, x, stride_x, bits_q, bits_v, p_q, p_v, dq_lora, dv_lora, mid_q,
                         mid_v, d_mid_q, d_mid_v, n_tokens, d, d_q, d_v, r, g_a_q, g_b_q, g_a_v,
                         g_b_v, workspace, workspace_floats, counters, n_counters, a))
    return e;
  const dim3 grid(static_cast<uint32_t>(a.first_block[4]),
                  static_cast<uint32_t>(w_chunks(n_tokens)));
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_BW(RR)                                                                       \
  case RR:                                                                               \
    hipLaunchKernelGGL(lora_bwd_w_kernel<RR>, grid, dim3(64 * kWWaves), 0, st, a);       \
    break;
  switch (r) { RUS_BW(4) RUS_BW(8) RUS_BW(16) RUS_BW(32) }
#undef RUS_BW
  return check_launch(fn);
}

extern "C" int rus_lora_bwd_xw(const void* x, int64_t stride_x, const uint32_t* bits_q,
                               const uint32_t* bits_v, float p_q, float p_v, const void* dq_lora,
                               const void* dv_lora, const void* mid_q, const void* mid_v,
                               const void* d_mid_q, const void* d_mid_v, int64_t n_tokens,
                               int64_t d, int64_t d_q, int64_t d_v, int32_t r, void* g_a_q,
                               void* g_b_q, void* g_a_v, void* g_b_v, const void* a_t_q,
                               const void* a_t_v, void* dx, int64_t stride_dx, float* workspace,
                               int64_t workspace_floats, int32_t* counters, int64_t n_counters,
                               void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_bwd_xw";
  BwdWArgs a;
  if (int e = bwd_w_args(fn, x, stride_x, bits_q, bits_v, p_q, p_v, dq_lora, dv_lora, mid_q,
                         mid_v, d_mid_q, d_mid_v, n_tokens, d, d_q, d_v, r, g_a_q, g_b_q, g_a_v,
                         g_b_v, workspace, workspace_floats, counters, n_counters, a))
    return e;
  if (!a_t_q || !a_t_v || !dx) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (d % 32 || stride_dx < d || stride_dx % 4)
    return fail(RUS_ERR_INVALID, "%s: need d %% 32 == 0 and stride_dx >= d, a multiple of 4", fn);
  const uintptr_t a_al = r >= 8 ? 16 : 8;
  if (!aligned(a_t_q, a_al) || !aligned(a_t_v, a_al) || !aligned(dx, 8) ||
      !aligned(d_mid_q, a_al) || !aligned(d_mid_v, a_al))
    return fail(RUS_ERR_INVALID, "%s: misaligned operand", fn);
  // n_tokens == 0: no expansion blocks; the weight-gradient blocks still write zeros.
  const int64_t n_blk = a.first_block[4], n_chunk = w_chunks(n_tokens);
  const int64_t x_col_blocks = (d / 32 + kWWaves - 1) / kWWaves;
  const int64_t blocks = n_blk * n_chunk + x_col_blocks * tiles(n_tokens);
  if (blocks >= (int64_t(1) << 31)) return fail(RUS_ERR_UNSUPPORTED, "%s: too many tokens", fn);
  ExpandArgs xa{static_cast<const f16*>(d_mid_q), static_cast<const f16*>(d_mid_v),
                static_cast<const f16*>(a_t_q), static_cast<const f16*>(a_t_v), n_tokens, d,
                static_cast<f16*>(dx), stride_dx, bits_q, bits_v, (d + 31) / 32,
                bits_q ? 1.0f / (1.0f - p_q) : 1.0f, bits_v ? 1.0f / (1.0f - p_v) : 1.0f};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<uint32_t>(blocks)), blk(64 * kWWaves);
  const int nb = static_cast<int>(n_blk), nc = static_cast<int>(n_chunk),
            xc = static_cast<int>(x_col_blocks);
#define RUS_BXW(RR)                                                                          \
  case RR:                                                                                   \
    if (bits_q)                                                                              \
      hipLaunchKernelGGL((lora_bwd_xw_kernel<RR, true>), grid, blk, 0, st, a, xa, nb, nc, xc); \
    else                                                                                     \
      hipLaunchKernelGGL((lora_bwd_xw_kernel<RR, false>), grid, blk, 0, st, a, xa, nb, nc, xc); \
    break;
  switch (r) { RUS_BXW(4) RUS_BXW(8) RUS_BXW(16) RUS_BXW(32) }
#undef RUS_BXW
  return check_launch(fn);
}

// ---------------------------------------------------------------------------------------------
// rus_lora_down_rows: LoRA-down by blocks of four token rows (no workspace), the arithmetic the
// per-layer dequant launch uses when it carries the input norm and this product.
// ---------------------------------------------------------------------------------------------

extern "C" int rus_lora_down_rows(const rus_lora_rows* q, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_down_rows";
  if (!q) return fail(RUS_ERR_INVALID, "%s: null argument", fn);
  DownRows a;
  if (int e = lora_rows_args(fn, *q, a)) return e;
  if (q->n_tokens == 0) return RUS_OK;
  const dim3 grid(static_cast<uint32_t>((q->n_tokens + kDownRows - 1) / kDownRows));
  hipLaunchKernelGGL(lora_down_rows_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  return check_launch(fn);
}

// ---------------------------------------------------------------------------------------------
// The step's fp16 LoRA factors in both layouts, one launch: the flat fp32 parameter buffer
// (n_layers x [segment 0 | segment 1 | ...], segment s row-major [rows_s, cols_s]) cast to fp16
// in the same layout, and each segment transposed into out_t region s = [n_layers, cols_s,
// rows_s] (regions back to back). Replaces the reference's per-layer fp16 casts of the factors
// (solution/ops.py:776, 778, and the backward's q_B_fp16 / q_A_fp16, ops.py:979-987); the
// transposed copies are the rank-major layout the fused LoRA backward kernels read.
// ---------------------------------------------------------------------------------------------

namespace rus {
namespace {

constexpr int kCastSegs = 4;

struct CastSegs {
  int64_t off[kCastSegs + 1];  // segment starts within a layer (off[n_seg] = per-layer size)
  int64_t base_t[kCastSegs];   // start of each segment's region in out_t
  int64_t cols[kCastSegs];
  int64_t rows[kCastSegs];
  int n_seg;
};

__global__ __launch_bounds__(256) void lora_cast_t_kernel(const float* __restrict__ flat,
                                                          int64_t n, CastSegs s,
                                                          f16* __restrict__ out,
                                                          f16* __restrict__ out_t) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n) return;
  const f16 h = from_f32<f16>(flat[e]);
  out[e] = h;
  if (out_t == nullptr) return;
  const int64_t per = s.off[s.n_seg];
  const int64_t l = e / per, rem = e - l * per;
  int j = 0;
#pragma unroll
  for (int k = 1; k < kCastSegs; ++k) j += (k < s.n_seg && rem >= s.off[k]) ? 1 : 0;
  const int64_t in_seg = rem - s.off[j];
  const int64_t r = in_seg / s.cols[j], c = in_seg - r * s.cols[j];
  out_t[s.base_t[j] + l * (s.off[j + 1] - s.off[j]) + c * s.rows[j] + r] = h;
}

}  // namespace
}  // namespace rus

extern "C" int rus_lora_cast_t(const float* flat, int64_t n_layers, int32_t n_seg,
                               const int64_t* seg_rows, const int64_t* seg_cols, void* out,
                               void* out_t, void* stream) {
  using namespace rus;
  const char* fn = "rus_lora_cast_t";
  if (n_seg < 1 || n_seg > kCastSegs || n_layers < 0 || !seg_rows || !seg_cols)
    return fail(RUS_ERR_INVALID, "%s: n_seg=%d outside [1, %d] or bad shape arguments", fn,
                n_seg, kCastSegs);
  if (!flat || !out) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  CastSegs s{};
  s.n_seg = n_seg;
  int64_t per = 0;
  for (int j = 0; j < n_seg; ++j) {
    if (seg_rows[j] <= 0 || seg_cols[j] <= 0 || seg_rows[j] >= (int64_t(1) << 31) ||
        seg_cols[j] >= (int64_t(1) << 31))
      return fail(RUS_ERR_INVALID, "%s: segment %d has shape %lld x %lld", fn, j,
                  (long long)seg_rows[j], (long long)seg_cols[j]);
    s.off[j] = per;
    s.rows[j] = seg_rows[j];
    s.cols[j] = seg_cols[j];
    per += seg_rows[j] * seg_cols[j];
  }
  s.off[n_seg] = per;
  for (int j = 0; j < n_seg; ++j) s.base_t[j] = n_layers * s.off[j];
  const int64_t n = n_layers * per;
  if (n >= (int64_t(1) << 40)) return fail(RUS_ERR_INVALID, "%s: %lld values", fn, (long long)n);
  if (n == 0) return RUS_OK;
  hipLaunchKernelGGL(lora_cast_t_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                     0, static_cast<hipStream_t>(stream), flat, n, s, static_cast<f16*>(out),
                     static_cast<f16*>(out_t));
  return check_launch(fn);
}
