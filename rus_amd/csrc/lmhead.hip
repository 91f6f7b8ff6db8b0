// Vocab-tiled lm_head cross-entropy on fp16 MFMA for gfx950.
//
// Behaviour follows the reference's chunked lm_head (solution/ops.py:174-349 with
// lm_head_piece_kernel / lm_head_finish_kernel, solution/kernels.py:453-565): logits are the fp16
// rounding of H.W^T (fp32 accumulation), per token the forward keeps an online max m,
// s = sum e^{z-m}, w = sum e^{z-m} z, the first-index argmax and the target logit, and finishes
// lse = m + ln s, entropy = lse - w/s, nll = lse - z[label]. The backward forms
// G = fp16((e^{z-lse} - 1[v=label]) * 2^16/denom) and dH = sum_v G[:, v] W[v, :].
// Two layouts share these kernels; neither holds the logits of a whole batch (CDNA4, wave64,
// 160 KiB LDS):
//   * token-blocked head (the default with a device-resident W): the tokens go in blocks of whole
//     256-token tiles, at least two per batch; per block lmhead_logits_kernel writes the block's
//     fp16 logits into a [block, round_up(V, 64)] buffer (at most 256 MiB: 768 tokens at
//     V = 151,936), lmhead_rows_kernel (one workgroup per token row) forms lse / nll / entropy /
//     first argmax and rewrites the row in place as G, and lmhead_grad_hidden_kernel forms
//     G . (W^T)^T split-K over the vocabulary into fp32 partials that dh_reduce_kernel sums;
//   * single pass over vocabulary chunks (a head streamed from the host, or v_chunk given):
//     lmhead_stats_kernel<KEEP> keeps per-token online statistics per 256 vocab rows in
//     registers and the chunk's logits; lmhead_chunk_scale_kernel turns them into
//     P = e^{z - M} (M the running maximum) and the same split-K GEMM adds P . W_chunk into fp32
//     partials rescaled when M grows; lmhead_dh_finish_kernel divides by s and subtracts the
//     label rows.
// The GEMMs run the mainloops of mfma_gemm.h: 256 x 256 block tiles on v_mfma_f32_32x32x16_f16
// filled by direct global -> LDS copies. The logits, statistics and hidden-gradient kernels run
// eight waves of 128 x 64 (two per SIMD) with K staged 64 deep through two 64 KiB buffers; the
// logit-gradient kernel (the recomputing backward) runs four waves of 128 x 128 with K staged 32
// deep through four 32 KiB buffers. In the statistics epilogue each lane holds 64 vocabulary
// entries of one token (W is the M operand) and the two 128-row halves of a tile meet in the LDS.
// Blocks are numbered XCD-aware (block b on XCD b % 8, each XCD a contiguous range of tiles), so
// blocks that share a W tile share an L2. LDS rows are XOR-swizzled per 16-byte chunk, so the
// copies and the MFMA fragment reads are bank-conflict free. The hidden gradient accumulates in
// fp32 partials (the reference accumulates in fp16, solution/ops.py:320).
#include <math.h>

#include "common.h"
#include "mfma_gemm.h"

namespace rus {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kPrescale = 65536.0f;  // solution/ops.py:171

__device__ __forceinline__ float round16(float x) {
  return static_cast<float>(from_f32<f16>(x));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Writes the block's 256 (vocab) x 256 (token) tile, held in the accumulator layout, as fp16
// out[token][vocab - tile base]: value(mt, nt, r, row) is the element of accumulator (mt, nt, r),
// whose vocab row local to A is row; rows >= g.M are written as 0. Staged through the LDS as
// [token][vocab] with 8-byte quads XOR-swizzled by row (pairs kept adjacent) so every lane stores
// 16 contiguous bytes of one token's row: out[tok][tl.m0 + c] for tok < g.N, c < kpad.
// NW waves in the mainloop's layout (4: 128 x 128 each, 8: 128 x 64).
template <int NW = 4, class F>
__device__ __forceinline__ void store_tile_tv(char* smem, const GemmArgs& g, const Tile& tl,
                                              f16* out, int64_t ld, int kpad, F value) {
  constexpr int NT = 16 / NW, RW = kBN / (NW / 2);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / (NW / 2), wn = wave % (NW / 2), h = lane >> 5;
  const int vrow0 = tl.m0 + wm * kWM;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int trow = wn * RW + nt * 32 + (lane & 31);  // token row within the block tile
    char* srow = smem + trow * 512;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = vrow0 + mt * 32 + 8 * q + 4 * h + e;
          v[e] = from_f32<f16>(row < g.M ? value(mt, nt, q * 4 + e, row) : 0.0f);
        }
        const int col = wm * kWM + mt * 32 + 8 * q + 4 * h;  // vocab column within the tile
        const int pq = (col >> 2) ^ ((trow & 31) << 1);
        *reinterpret_cast<f16x4*>(srow + pq * 8) = v;
      }
  }
  __syncthreads();
  const int t = threadIdx.x;
  const int c = t & 31;
#pragma unroll 4
  for (int it = 0; it < kBN / (2 * NW); ++it) {
    const int trow = it * 2 * NW + (t >> 5);
    const int tok = tl.n0 + trow;
    const int col = tl.m0 + c * 8;
    if (tok < g.N && col < kpad) {
      const int pq = (2 * c) ^ ((trow & 31) << 1);
      const uint4 v = *reinterpret_cast<const uint4*>(smem + trow * 512 + pq * 8);
      *reinterpret_cast<uint4*>(out + static_cast<int64_t>(tok) * ld + col) = v;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Forward statistics: A = W rows (vocab), B = H rows (tokens).
// ---------------------------------------------------------------------------------------------

struct StatsParams {
  const int64_t* labels;
  float* part_m;
  float* part_s;
  float* part_w;
  int32_t* part_idx;
  float* target;
  int64_t part_stride;  // entries per partial row (>= n_tok)
  int part_base;        // partial row of A's first 256-row tile
  int vocab_start;      // global vocabulary index of A's row 0
  f16* z;               // KEEP: the fp16 logits [n_tok][ld_z], columns up to kpad (0 past M)
  int64_t ld_z;
  int kpad;
};

// The statistics epilogue of a block's 256 (vocab) x 256 (token) tile of logits, on NW waves in
// the mainloop's layout (4: 128 x 128 each, 8: 128 x 64): per token, the maximum, the sums of e^{z-m}
// and e^{z-m} z, the first argmax and the target logit over the tile's vocab rows (the two 128-row
// halves merged through the LDS); with KEEP the fp16 logits are stored first.
template <int NW, bool KEEP>
__device__ __forceinline__ void stats_epilogue(char* smem, const GemmArgs& g, const Tile& tl,
                                               const StatsParams& p,
                                               f32x16 (&acc)[kMT][16 / NW]) {
  constexpr int NT = 16 / NW, RW = kBN / (NW / 2);  // token columns per wave: 128 or 64
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave / (NW / 2), wn = wave % (NW / 2), h = lane >> 5;
  const int vrow0 = tl.m0 + wm * kWM;  // local vocab row of this wave's first accumulator row
  const bool full = tl.m0 + kBM <= g.M;
  float rm[NT], rs[NT], rw[NT];
  int ri[NT];
  // Logits as the reference's fp16 GEMM output: rounded once, in place.
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = round16(acc[mt][nt][r]);
  if constexpr (KEEP)
    store_tile_tv<NW>(smem, g, tl, p.z, p.ld_z, p.kpad,
                      [&](int mt, int nt, int r, int) { return acc[mt][nt][r]; });
  // Accumulator row of (mt, r) for this lane: mt*32 + 8*(r/4) + 4*h + r%4 (local to vrow0).
  const int rows_left = g.M - vrow0;  // rows at or past this are padding (edge tile only)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int tok = tl.n0 + wn * RW + nt * 32 + (lane & 31);
    int lab_adj = -1000;  // label row local to vrow0, minus 4h (compared with the r/mt part)
    if (tok < g.N) {
      const int64_t l = p.labels[tok] - p.vocab_start - vrow0;
      lab_adj = (l >= 0 && l < kWM) ? static_cast<int>(l) - 4 * h : -1000;
    }
    float m = -INFINITY, tgt = 0.0f;
    int idx = 0x7fffffff;  // local row minus 4h until the end
    if (full) {
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rl = mt * 32 + 8 * (r >> 2) + (r & 3);
          const float z = acc[mt][nt][r];
          idx = z > m ? rl : idx;  // rows ascend: strict > keeps the first index
          m = fmaxf(m, z);
          tgt = rl == lab_adj ? z : tgt;
        }
    } else {
#pragma unroll
      for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int rl = mt * 32 + 8 * (r >> 2) + (r & 3);
          const float z = acc[mt][nt][r];
          if (rl + 4 * h < rows_left && z > m) {
            m = z;
            idx = rl;
          }
          tgt = rl == lab_adj ? z : tgt;
        }
    }
    idx = idx == 0x7fffffff ? idx : vrow0 + idx + 4 * h;
    // The lane pair (l, l^32) holds the two interleaved halves of the wave's 128 rows.
    const float m2 = __shfl_xor(m, 32, kWave);
    const int i2 = __shfl_xor(idx, 32, kWave);
    if (m2 > m || (m2 == m && i2 < idx)) {
      m = m2;
      idx = i2;
    }
    float s = 0.0f, w = 0.0f;
    if (m > -INFINITY) {
      const float mb = m * kLog2e;
      if (full) {
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float z = acc[mt][nt][r];
            const float e = exp2_fast(__builtin_fmaf(z, kLog2e, -mb));
            s += e;
            w = __builtin_fmaf(e, z, w);
          }
      } else {
#pragma unroll
        for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int rl = mt * 32 + 8 * (r >> 2) + (r & 3);
            if (rl + 4 * h < rows_left) {
              const float z = acc[mt][nt][r];
              const float e = exp2_fast(__builtin_fmaf(z, kLog2e, -mb));
              s += e;
              w = __builtin_fmaf(e, z, w);
            }
          }
      }
    }
    s += __shfl_xor(s, 32, kWave);
    w += __shfl_xor(w, 32, kWave);
    rm[nt] = m;
    rs[nt] = s;
    rw[nt] = w;
    ri[nt] = idx;
    // The label's row lives in exactly one lane of one block: that lane writes the target.
    if (lab_adj + 4 * h >= 0 && ((lab_adj + 4 * h) >> 2 & 1) == h) p.target[tok] = tgt;
  }

  // Merge the two vocab halves (wm = 0, 1) of the block through LDS; wm = 0 writes the partial.
  if constexpr (KEEP) __syncthreads();  // the logits' staging reads of the LDS are done
  float* xm = reinterpret_cast<float*>(smem);  // [token column of the tile] x (m, s, w, idx)
  if (wm == 1 && h == 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int o = wn * RW + nt * 32 + lane;
      xm[o] = rm[nt];
      xm[kBN + o] = rs[nt];
      xm[2 * kBN + o] = rw[nt];
      reinterpret_cast<int*>(xm)[3 * kBN + o] = ri[nt];
    }
  }
  __syncthreads();
  if (wm == 0 && h == 0) {
    const int part = p.part_base + tl.m0 / kBM;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int tok = tl.n0 + wn * RW + nt * 32 + lane;
      const int o = wn * RW + nt * 32 + lane;
      const float mB = xm[o], sB = xm[kBN + o], wB = xm[2 * kBN + o];
      const int iB = reinterpret_cast<int*>(xm)[3 * kBN + o];
      float m = rm[nt], s = rs[nt], w = rw[nt];
      int idx = ri[nt];
      const float M = fmaxf(m, mB);
      if (M > -INFINITY) {
        const float ca = exp2_fast((m - M) * kLog2e), cb = exp2_fast((mB - M) * kLog2e);
        s = s * ca + sB * cb;
        w = w * ca + wB * cb;
      }
      if (mB > m) idx = iB;  // the second half's rows all follow the first half's
      m = M;
      if (tok < g.N && idx != 0x7fffffff) {
        const int64_t o2 = static_cast<int64_t>(part) * p.part_stride + tok;
        p.part_m[o2] = m;
        p.part_s[o2] = s;
        p.part_w[o2] = w;
        p.part_idx[o2] = idx + p.vocab_start;
      }
    }
  }
}

template <bool KEEP>
__global__ __launch_bounds__(kThreads8) __attribute__((amdgpu_waves_per_eu(2, 2))) void
lmhead_stats_kernel(GemmArgs g, StatsParams p) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  Tile tl;
  if (!tile_of(g, tl)) return;
  f32x16 acc[kMT][2];
  mainloop(g, tl, smem, acc);
  stats_epilogue<8, KEEP>(smem, g, tl, p, acc);
}

// ---------------------------------------------------------------------------------------------
// Logits only: A = W rows (vocab), B = H rows (tokens) -> z[token][vocab] = fp16(H.W^T), the
// mainloop followed by the tile's store (no statistics in the epilogue: lmhead_rows_kernel forms
// them from the stored row, at full occupancy, beside other rows' HBM traffic).
// ---------------------------------------------------------------------------------------------

struct LogitsParams {
  f16* z;  // [n_tok][ld_z], columns up to kpad (0 past M)
  int64_t ld_z;
  int kpad;
};


__global__ __launch_bounds__(kThreads8) __attribute__((amdgpu_waves_per_eu(2, 2))) void
lmhead_logits_kernel(GemmArgs g, LogitsParams p) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  Tile tl;
  if (!tile_of(g, tl)) return;
  f32x16 acc[kMT][2];
  mainloop(g, tl, smem, acc);
  store_tile_tv<8>(smem, g, tl, p.z, p.ld_z, p.kpad,
                   [&](int mt, int nt, int r, int) { return acc[mt][nt][r]; });
}

// ---------------------------------------------------------------------------------------------
// Logit gradient: A = W rows (vocab chunk), B = H rows (tokens) -> G[token][vocab] fp16.
// ---------------------------------------------------------------------------------------------

struct GradParams {
  const int64_t* labels;
  const float* lse;
  const float* denom;  // device scalar: loss denominator (clamped to >= 1 here)
  f16* g;              // [n_tok][ld_g]
  int64_t ld_g;
  int kpad;            // columns written: round_up(n_vocab, 64); rows >= n_vocab get zeros
  int vocab_start;
};

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void
lmhead_grad_logits_kernel(GemmArgs g, GradParams p) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  Tile tl;
  if (!tile_of(g, tl)) return;
  f32x16 acc[kMT][kNT];
  mainloop(g, tl, smem, acc);

  const float scale_all = kPrescale / fmaxf(*p.denom, 1.0f);
  const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) & 1;
  int lab[kNT];
  float scale[kNT], l2[kNT];
#pragma unroll
  for (int nt = 0; nt < kNT; ++nt) {
    const int tok = tl.n0 + wn * kWN + nt * 32 + (lane & 31);
    lab[nt] = -1;
    scale[nt] = 0.0f;
    l2[nt] = 0.0f;
    if (tok < g.N) {
      const int64_t lg = p.labels[tok];
      if (lg != -100) {
        scale[nt] = scale_all;
        const int64_t l = lg - p.vocab_start;
        lab[nt] = (l >= 0 && l < g.M) ? static_cast<int>(l) : -1;
      }
      l2[nt] = p.lse[tok] * kLog2e;
    }
  }
  store_tile_tv(smem, g, tl, p.g, p.ld_g, p.kpad, [&](int mt, int nt, int r, int row) {
    const float z = round16(acc[mt][nt][r]);
    const float pr = exp2_fast(__builtin_fmaf(z, kLog2e, -l2[nt]));
    return (pr - (row == lab[nt] ? 1.0f : 0.0f)) * scale[nt];
  });
}

// ---------------------------------------------------------------------------------------------
// Logit gradient in place from the logits the statistics pass kept: per element the formula of
// lmhead_grad_logits_kernel's epilogue on the same fp16 logit, so both give the same bits.
// Block = (token, kZgCols columns); each thread loads its kZgUnroll 16-byte packs before any math.
// ---------------------------------------------------------------------------------------------

constexpr int kZgThreads = 256, kZgUnroll = 2, kZgCols = kZgThreads * kZgUnroll * 8;

__global__ __launch_bounds__(kZgThreads) void lmhead_grad_from_logits_kernel(
    f16* zg, int64_t ld, int n_vocab, int kpad, const int64_t* labels, const float* lse,
    const float* denom, int vocab_start) {
  const int tok = blockIdx.x;
  const int64_t lg = labels[tok];
  float scale = 0.0f;
  int lab = -1;
  if (lg != -100) {
    scale = kPrescale / fmaxf(*denom, 1.0f);
    const int64_t l = lg - vocab_start;
    lab = (l >= 0 && l < n_vocab) ? static_cast<int>(l) : -1;
  }
  const float l2 = lse[tok] * kLog2e;
  f16* row = zg + static_cast<int64_t>(tok) * ld;
  const int c0 = blockIdx.y * kZgCols + threadIdx.x * 8;
  f16x8 v[kZgUnroll];
#pragma unroll
  for (int u = 0; u < kZgUnroll; ++u) {
    const int c = c0 + u * kZgThreads * 8;
    if (c < kpad) v[u] = *reinterpret_cast<const f16x8*>(row + c);
  }
#pragma unroll
  for (int u = 0; u < kZgUnroll; ++u) {
    const int c = c0 + u * kZgThreads * 8;
    if (c >= kpad) continue;
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = static_cast<float>(v[u][e]);
      const float pr = exp2_fast(__builtin_fmaf(z, kLog2e, -l2));
      const float gv = (pr - (c + e == lab ? 1.0f : 0.0f)) * scale;
      o[e] = from_f32<f16>(c + e < n_vocab ? gv : 0.0f);
    }
    *reinterpret_cast<f16x8*>(row + c) = o;
  }
}

// ---------------------------------------------------------------------------------------------
// Hidden gradient: A = G rows (tokens), B = W^T rows (hidden dims), split-K over vocab.
// ---------------------------------------------------------------------------------------------

struct StoreParams {
  float* parts;  // [splits][M][N] fp32
  int accumulate;
  const float* alpha;  // accumulate: parts = parts * alpha[row] + acc (alpha null: factor 1)
};

__global__ __launch_bounds__(kThreads8) __attribute__((amdgpu_waves_per_eu(2, 2))) void
lmhead_grad_hidden_kernel(GemmArgs g, StoreParams p) {
  __shared__ __attribute__((aligned(16))) char smem[kSmemBytes];
  Tile tl;
  if (!tile_of(g, tl)) return;
  f32x16 acc[kMT][2];
  mainloop(g, tl, smem, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 2, wn = wave & 3, h = lane >> 5;
  float* base = p.parts + static_cast<int64_t>(tl.split) * g.M * g.N;
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int col = tl.n0 + wn * 64 + nt * 32 + (lane & 31);
    if (col >= g.N) continue;
#pragma unroll
    for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = tl.m0 + wm * kWM + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < g.M) {
          float* dst = base + static_cast<int64_t>(row) * g.N + col;
          if (!p.accumulate)
            *dst = acc[mt][nt][r];
          else
            *dst = (p.alpha ? *dst * p.alpha[row] : *dst) + acc[mt][nt][r];
        }
      }
  }
}

// ---------------------------------------------------------------------------------------------
// Online single pass: one vocabulary chunk's kept logits z become P = fp16(e^{z - M}) in place,
// where M = max(M_run, the chunk's maximum) is the running maximum over the chunks so far; the
// hidden-gradient GEMM then accumulates P . W_chunk into partials rescaled by
// alpha = e^{M_run - M}. Block = (token, kZgCols columns). Every block of a token forms M itself
// from the chunk's partial maxima (max(M_run, chunk max) is the same whether it reads M_run before
// or after block (token, 0) stores the new value); block (token, 0) writes M_run and alpha.
// ---------------------------------------------------------------------------------------------

__global__ __launch_bounds__(kZgThreads) void lmhead_chunk_scale_kernel(
    f16* zg, int64_t ld, int n_vocab, int kpad, const float* __restrict__ part_m,
    int64_t part_stride, int part_base, int n_parts, float* m_run, float* alpha, int first) {
  __shared__ float red[kZgThreads / kWave];
  const int tok = blockIdx.x;
  float cm = -INFINITY;
  for (int q = threadIdx.x; q < n_parts; q += kZgThreads)
    cm = fmaxf(cm, part_m[static_cast<int64_t>(part_base + q) * part_stride + tok]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off, kWave));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = cm;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kZgThreads / kWave; ++w) cm = fmaxf(cm, red[w]);
  const float mo = first ? -INFINITY : m_run[tok];
  const float mn = fmaxf(mo, cm);
  __syncthreads();  // every thread has read m_run before it is replaced
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    m_run[tok] = mn;
    alpha[tok] = first ? 0.0f : exp2_fast((mo - mn) * kLog2e);
  }
  const float mb = mn * kLog2e;
  f16* row = zg + static_cast<int64_t>(tok) * ld;
  const int c0 = blockIdx.y * kZgCols + threadIdx.x * 8;
  f16x8 v[kZgUnroll];
#pragma unroll
  for (int u = 0; u < kZgUnroll; ++u) {
    const int c = c0 + u * kZgThreads * 8;
    if (c < kpad) v[u] = *reinterpret_cast<const f16x8*>(row + c);
  }
#pragma unroll
  for (int u = 0; u < kZgUnroll; ++u) {
    const int c = c0 + u * kZgThreads * 8;
    if (c >= kpad) continue;
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pr = exp2_fast(__builtin_fmaf(static_cast<float>(v[u][e]), kLog2e, -mb));
      o[e] = from_f32<f16>(c + e < n_vocab ? pr : 0.0f);
    }
    *reinterpret_cast<f16x8*>(row + c) = o;
  }
}

// dH (times 2^16 / denom, times scale) from the online accumulation:
//   out[t][c] = (sum_s parts[s][t][c] * e^{M[t] - lse[t]} - W[y_t][c]) * 2^16 / denom * scale
// for labelled tokens (y_t != -100; the W row term only when y_t indexes the vocabulary), 0 for
// the others. w_rows may be device memory or device-mapped pinned host memory. Four columns per
// thread.
template <typename T>
__global__ __launch_bounds__(256) void lmhead_dh_finish_kernel(
    const float* __restrict__ parts, int n_parts, int n_tok, int d, const float* __restrict__ m_run,
    const float* __restrict__ lse, const int64_t* __restrict__ labels,
    const f16* __restrict__ w_rows, int64_t ld_w, int64_t n_vocab, const float* __restrict__ denom,
    float scale_h, const float* __restrict__ scale_d, T* __restrict__ out) {
  const int64_t n = static_cast<int64_t>(n_tok) * d;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  const int t = static_cast<int>(i / d), c = static_cast<int>(i % d);
  const int64_t y = labels[t];
  float o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (y != -100) {
    f32x4 a = *reinterpret_cast<const f32x4*>(parts + i);
    for (int q = 1; q < n_parts; ++q) a += *reinterpret_cast<const f32x4*>(parts + q * n + i);
    const float f = exp2_fast((m_run[t] - lse[t]) * kLog2e);
    float scale = kPrescale / fmaxf(*denom, 1.0f) * scale_h;
    if (scale_d) scale *= *scale_d;
    float wy[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (y >= 0 && y < n_vocab) load_f32<f16, 4>(w_rows + y * ld_w + c, wy);
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (a[e] * f - wy[e]) * scale;
  }
  store_from_f32<T, 4>(out + i, o);
}

// ---------------------------------------------------------------------------------------------
// One token's row of kept logits z[0 .. n_vocab): its statistics (first-index argmax, max m,
// s = sum e^{z-m}, w = sum e^{z-m} z, the label's logit) in one pass, lse = m + ln s,
// entropy = lse - w/s, nll = lse - z[label]; then, when a denominator is given, the logit
// gradient G = fp16((e^{z-lse} - 1[v=label]) 2^16 / denom) in place (the formula of
// lmhead_grad_logits_kernel's epilogue; 0 in the padding columns up to kpad, and for label -100).
// Block = one row, kRowThreads threads, each taking 16-byte packs kRowThreads * 8 apart and
// keeping kRowDepth of them in flight.
// ---------------------------------------------------------------------------------------------

constexpr int kRowThreads = 512, kRowDepth = 8;

__device__ __forceinline__ void merge_row(float& m, float& s, float& w, float& bv, int& bi, float m2,
                                          float s2, float w2, float bv2, int bi2) {
  const float M = fmaxf(m, m2);
  if (M > -INFINITY) {
    const float c1 = exp2_fast((m - M) * kLog2e), c2 = exp2_fast((m2 - M) * kLog2e);
    s = s * c1 + s2 * c2;
    w = w * c1 + w2 * c2;
  }
  m = M;
  if (bv2 > bv || (bv2 == bv && bi2 < bi)) {
    bv = bv2;
    bi = bi2;
  }
}

__global__ __launch_bounds__(kRowThreads) void lmhead_rows_kernel(
    f16* zg, int64_t ld, int n_vocab, int kpad, const int64_t* __restrict__ labels,
    const float* __restrict__ denom, float* __restrict__ lse_out, float* __restrict__ nll_out,
    float* __restrict__ ent_out, int64_t* __restrict__ amax_out) {
  __shared__ float red[5][kRowThreads / kWave];
  const int tok = blockIdx.x, tid = threadIdx.x;
  f16* row = zg + static_cast<int64_t>(tok) * ld;
  float m = -INFINITY, s = 0.0f, w = 0.0f, bv = -INFINITY;
  int bi = 0x7fffffff;
  const int n_packs = (n_vocab + 7) / 8;
  for (int p0 = tid; p0 < n_packs; p0 += kRowThreads * kRowDepth) {
    f16x8 v[kRowDepth];
#pragma unroll
    for (int u = 0; u < kRowDepth; ++u) {
      const int p = p0 + u * kRowThreads;
      if (p < n_packs) v[u] = *reinterpret_cast<const f16x8*>(row + 8 * p);
    }
#pragma unroll
    for (int u = 0; u < kRowDepth; ++u) {
      const int p = p0 + u * kRowThreads;
      if (p >= n_packs) break;
      float z[8];
      float mc = -INFINITY;
      int ic = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        z[e] = 8 * p + e < n_vocab ? static_cast<float>(v[u][e]) : -INFINITY;
        if (z[e] > mc) {  // strict: the first index of the pack's maximum
          mc = z[e];
          ic = e;
        }
      }
      if (mc > bv) {  // packs ascend within a thread: strict keeps the first index
        bv = mc;
        bi = 8 * p + ic;
      }
      if (mc > m) {
        const float c = exp2_fast((m - mc) * kLog2e);
        s *= c;
        w *= c;
        m = mc;
      }
      if (mc == -INFINITY) continue;  // only padding in this pack
      const float mb = m * kLog2e;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (8 * p + e < n_vocab) {  // the padding's -inf would make 0 * -inf in w
          const float t = exp2_fast(__builtin_fmaf(z[e], kLog2e, -mb));
          s += t;
          w = __builtin_fmaf(t, z[e], w);
        }
      }
    }
  }
  // wave, then block: merge (m, s, w) and the argmax (ties: the smaller index)
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off, kWave), s2 = __shfl_xor(s, off, kWave);
    const float w2 = __shfl_xor(w, off, kWave), bv2 = __shfl_xor(bv, off, kWave);
    const int bi2 = __shfl_xor(bi, off, kWave);
    merge_row(m, s, w, bv, bi, m2, s2, w2, bv2, bi2);
  }
  const int wave = tid >> 6;
  if ((tid & 63) == 0) {
    red[0][wave] = m;
    red[1][wave] = s;
    red[2][wave] = w;
    red[3][wave] = bv;
    red[4][wave] = __int_as_float(bi);
  }
  __syncthreads();
  m = red[0][0];
  s = red[1][0];
  w = red[2][0];
  bv = red[3][0];
  bi = __float_as_int(red[4][0]);
  for (int k = 1; k < kRowThreads / kWave; ++k)
    merge_row(m, s, w, bv, bi, red[0][k], red[1][k], red[2][k], red[3][k],
              __float_as_int(red[4][k]));
  const float L = m + logf(s);
  const int64_t y = labels[tok];
  const bool in_range = y >= 0 && y < n_vocab;
  if (tid == 0) {
    const float tgt = in_range ? static_cast<float>(row[y]) : 0.0f;
    lse_out[tok] = L;
    ent_out[tok] = L - w / s;
    nll_out[tok] = y != -100 ? L - tgt : 0.0f;
    amax_out[tok] = bi;
  }
  if (!denom) return;
  __syncthreads();  // the label's logit is read before it is overwritten
  const float scale = y != -100 ? kPrescale / fmaxf(*denom, 1.0f) : 0.0f;
  const int lab = in_range ? static_cast<int>(y) : -1;
  const float l2 = L * kLog2e;
  const int k_packs = kpad / 8;
  // Last chunk first: the row's tail, read last by the statistics pass, is the part most likely
  // still in L2 (every element's G depends only on its own logit, so the order leaves the bits).
  constexpr int kChunk = kRowThreads * kRowDepth;
  for (int ch = (k_packs - 1) / kChunk; ch >= 0; --ch) {
    const int p0 = ch * kChunk + tid;
    f16x8 v[kRowDepth];
#pragma unroll
    for (int u = 0; u < kRowDepth; ++u) {
      const int p = p0 + u * kRowThreads;
      if (p < k_packs) v[u] = *reinterpret_cast<const f16x8*>(row + 8 * p);
    }
#pragma unroll
    for (int u = 0; u < kRowDepth; ++u) {
      const int p = p0 + u * kRowThreads;
      if (p >= k_packs) break;
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 8 * p + e;
        const float pr = exp2_fast(__builtin_fmaf(static_cast<float>(v[u][e]), kLog2e, -l2));
        const float gv = (pr - (c == lab ? 1.0f : 0.0f)) * scale;
        o[e] = from_f32<f16>(c < n_vocab ? gv : 0.0f);
      }
      *reinterpret_cast<f16x8*>(row + 8 * p) = o;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Combine partial statistics: one lane per token, 16 waves per 64 tokens, each wave merging a
// contiguous range of partials eight loads at a time, then wave 0 merging the 16 results in
// wave order (deterministic; ties keep the smallest vocabulary index).
// ---------------------------------------------------------------------------------------------

constexpr int kCombWaves = 16, kCombDepth = 8;

struct Stat {
  float m, s, w;
  int i;
};

__device__ __forceinline__ void merge_stat(Stat& a, float m, float s, float w, int i) {
  if (m > a.m) {
    const float c = exp2_fast((a.m - m) * kLog2e);
    a.s = a.s * c + s;
    a.w = a.w * c + w;
    a.m = m;
    a.i = i;
  } else if (m > -INFINITY) {
    const float c = exp2_fast((m - a.m) * kLog2e);
    a.s += s * c;
    a.w += w * c;
    if (m == a.m && i < a.i) a.i = i;
  }
}

__global__ __launch_bounds__(kCombWaves * 64) void lmhead_combine_kernel(
    const float* __restrict__ pm, const float* __restrict__ ps, const float* __restrict__ pw,
    const int32_t* __restrict__ pi, int n_parts, int64_t stride, const float* __restrict__ target,
    const int64_t* __restrict__ labels, int n_tok, float* __restrict__ lse,
    float* __restrict__ nll, float* __restrict__ ent, int64_t* __restrict__ amax) {
  __shared__ float sm[kCombWaves][64], ss[kCombWaves][64], sw[kCombWaves][64];
  __shared__ int si[kCombWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tok = blockIdx.x * 64 + lane;
  Stat st{-INFINITY, 0.0f, 0.0f, 0x7fffffff};
  const int per = (n_parts + kCombWaves - 1) / kCombWaves;
  const int q0 = wave * per, q1 = min(q0 + per, n_parts);
  if (tok < n_tok) {
    for (int q = q0; q < q1; q += kCombDepth) {
      float m[kCombDepth], s[kCombDepth], w[kCombDepth];
      int ix[kCombDepth];
#pragma unroll
      for (int j = 0; j < kCombDepth; ++j) {
        const int64_t o = static_cast<int64_t>(min(q + j, q1 - 1)) * stride + tok;
        m[j] = pm[o];
        s[j] = ps[o];
        w[j] = pw[o];
        ix[j] = pi[o];
      }
#pragma unroll
      for (int j = 0; j < kCombDepth; ++j)
        if (q + j < q1) merge_stat(st, m[j], s[j], w[j], ix[j]);
    }
  }
  sm[wave][lane] = st.m;
  ss[wave][lane] = st.s;
  sw[wave][lane] = st.w;
  si[wave][lane] = st.i;
  __syncthreads();
  if (wave != 0 || tok >= n_tok) return;
  Stat t{-INFINITY, 0.0f, 0.0f, 0x7fffffff};
  for (int k = 0; k < kCombWaves; ++k)
    merge_stat(t, sm[k][lane], ss[k][lane], sw[k][lane], si[k][lane]);
  const float L = t.m + logf(t.s);
  lse[tok] = L;
  ent[tok] = L - t.w / t.s;
  nll[tok] = labels[tok] != -100 ? L - target[tok] : 0.0f;
  amax[tok] = t.i;
}

// out[i] = T( scale * sum_p parts[p][i] ), four elements per thread (16-byte accesses when every
// partial starts 16-byte aligned, i.e. n % 4 == 0).
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void dh_reduce_kernel(const float* __restrict__ parts,
                                                        int n_parts, int64_t n, float scale_h,
                                                        const float* __restrict__ scale_d,
                                                        T* __restrict__ out) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  const float scale = scale_d ? scale_h * *scale_d : scale_h;
  if (VEC && i + 4 <= n) {
    f32x4 s = *reinterpret_cast<const f32x4*>(parts + i);
    for (int q = 1; q < n_parts; ++q) s += *reinterpret_cast<const f32x4*>(parts + q * n + i);
    float o[4] = {s[0] * scale, s[1] * scale, s[2] * scale, s[3] * scale};
    store_from_f32<T, 4>(out + i, o);
  } else {
    for (int64_t j = i; j < n && j < i + 4; ++j) {
      float s = parts[j];
      for (int q = 1; q < n_parts; ++q) s += parts[q * n + j];
      out[j] = from_f32<T>(s * scale);
    }
  }
}

// dst[c][r] = src[r][c] for r < rows, c < cols, and dst[c][r] = 0 for rows <= r < rows_pad:
// 64x64 tiles through LDS (row pitch 66 halves, so the column reads of the write phase spread
// over the banks); each thread moves 16 elements in and 16 out.
__global__ __launch_bounds__(256) void transpose_f16_kernel(const f16* __restrict__ src,
                                                            int64_t rows, int64_t cols,
                                                            int64_t ld_src, f16* __restrict__ dst,
                                                            int64_t ld_dst, int64_t rows_pad) {
  __shared__ f16 tile[64][66];
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64, c0 = static_cast<int64_t>(blockIdx.y) * 64;
  const int t = threadIdx.x;
  {
    const int rr = t >> 2, cc = (t & 3) * 16;
    const int64_t r = r0 + rr;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int64_t c = c0 + cc + e;
      tile[rr][cc + e] = (r < rows && c < cols) ? src[r * ld_src + c] : static_cast<f16>(0.0f);
    }
  }
  __syncthreads();
  const int cc = t >> 2, rr = (t & 3) * 16;
  const int64_t c = c0 + cc;
  if (c >= cols) return;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int64_t r = r0 + rr + e;
    if (r < rows_pad) dst[c * ld_dst + r] = tile[rr + e][cc];
  }
}

}  // namespace
}  // namespace rus

using namespace rus;

static int lmhead_fwd(const char* fn, const void* hidden, const void* weight,
                      const int64_t* labels, int64_t n_tok, int64_t d, int64_t ld_h, int64_t ld_w,
                      int64_t n_vocab, int64_t vocab_start, float* part_m, float* part_s,
                      float* part_w, int32_t* part_idx, int64_t part_base, int64_t part_stride,
                      float* target, void* logits, int64_t ld_z, void* stream) {
  if (n_tok < 0 || n_tok >= (1 << 30) || n_vocab < 0 || n_vocab >= (1 << 30) || d <= 0 ||
      d % kBK || vocab_start < 0 || vocab_start + n_vocab >= (int64_t(1) << 31))
    return fail(RUS_ERR_INVALID,
                "%s: bad sizes n_tok=%lld n_vocab=%lld d=%lld (d must be a multiple of %d)", fn,
                (long long)n_tok, (long long)n_vocab, (long long)d, kBK);
  if (n_tok == 0 || n_vocab == 0) return RUS_OK;
  if (ld_h < d || ld_w < d) return fail(RUS_ERR_INVALID, "%s: row strides smaller than d", fn);
  if (int e = check_operand(fn, hidden, ld_h, "hidden")) return e;
  if (int e = check_operand(fn, weight, ld_w, "weight")) return e;
  if (!labels || !part_m || !part_s || !part_w || !part_idx || !target || part_base < 0 ||
      part_stride < n_tok)
    return fail(RUS_ERR_INVALID, "%s: null output or bad partial layout", fn);
  if (logits) {
    const int64_t kpad = (n_vocab + kBK - 1) / kBK * kBK;
    if (ld_z < kpad)
      return fail(RUS_ERR_INVALID, "%s: ld_z must be >= %lld", fn, (long long)kpad);
    if (int e = check_operand(fn, logits, ld_z, "logits")) return e;
  }
  GemmArgs g;
  g.A = static_cast<const f16*>(weight);
  g.lda = ld_w;
  g.M = static_cast<int>(n_vocab);
  g.B = static_cast<const f16*>(hidden);
  g.ldb = ld_h;
  g.N = static_cast<int>(n_tok);
  g.K = static_cast<int>(d);
  g.k_per_split = g.K;
  g.splits = 1;
  g.tiles_m = (g.M + kBM - 1) / kBM;
  g.tiles_n = (g.N + kBN - 1) / kBN;
  StatsParams p{labels,      part_m,      part_s, part_w,  part_idx,
                target,      part_stride, static_cast<int>(part_base),
                static_cast<int>(vocab_start), static_cast<f16*>(logits), ld_z,
                static_cast<int>((n_vocab + kBK - 1) / kBK * kBK)};
  if (logits)
    hipLaunchKernelGGL(lmhead_stats_kernel<true>, dim3(launch_grid(g)), dim3(kThreads8), 0,
                       static_cast<hipStream_t>(stream), g, p);
  else
    hipLaunchKernelGGL(lmhead_stats_kernel<false>, dim3(launch_grid(g)), dim3(kThreads8), 0,
                       static_cast<hipStream_t>(stream), g, p);
  return check_launch(fn);
}

extern "C" int rus_lmhead_ce_fwd(const void* hidden, const void* weight, const int64_t* labels,
                                 int64_t n_tok, int64_t d, int64_t ld_h, int64_t ld_w,
                                 int64_t n_vocab, int64_t vocab_start, float* part_m,
                                 float* part_s, float* part_w, int32_t* part_idx,
                                 int64_t part_base, int64_t part_stride, float* target,
                                 void* stream) {
  return lmhead_fwd("rus_lmhead_ce_fwd", hidden, weight, labels, n_tok, d, ld_h, ld_w, n_vocab,
                    vocab_start, part_m, part_s, part_w, part_idx, part_base, part_stride, target,
                    nullptr, 0, stream);
}

extern "C" int rus_lmhead_ce_fwd_keep(const void* hidden, const void* weight,
                                      const int64_t* labels, int64_t n_tok, int64_t d,
                                      int64_t ld_h, int64_t ld_w, int64_t n_vocab,
                                      int64_t vocab_start, float* part_m, float* part_s,
                                      float* part_w, int32_t* part_idx, int64_t part_base,
                                      int64_t part_stride, float* target, void* logits,
                                      int64_t ld_z, void* stream) {
  const char* fn = "rus_lmhead_ce_fwd_keep";
  if (!logits) return fail(RUS_ERR_INVALID, "%s: null logits buffer", fn);
  return lmhead_fwd(fn, hidden, weight, labels, n_tok, d, ld_h, ld_w, n_vocab, vocab_start,
                    part_m, part_s, part_w, part_idx, part_base, part_stride, target, logits,
                    ld_z, stream);
}

extern "C" int rus_lmhead_ce_grad_from_logits(void* logits_grad, int64_t ld_g,
                                              const int64_t* labels, const float* lse,
                                              const float* denom, int64_t n_tok,
                                              int64_t n_vocab, int64_t vocab_start,
                                              void* stream) {
  const char* fn = "rus_lmhead_ce_grad_from_logits";
  if (n_tok < 0 || n_tok >= (1 << 30) || n_vocab < 0 || n_vocab >= (1 << 30) || vocab_start < 0 ||
      vocab_start + n_vocab >= (int64_t(1) << 31))
    return fail(RUS_ERR_INVALID, "%s: bad sizes n_tok=%lld n_vocab=%lld", fn, (long long)n_tok,
                (long long)n_vocab);
  if (n_tok == 0 || n_vocab == 0) return RUS_OK;
  const int64_t kpad = (n_vocab + kBK - 1) / kBK * kBK;
  if (ld_g < kpad)
    return fail(RUS_ERR_INVALID, "%s: ld_g must be >= %lld", fn, (long long)kpad);
  if (int e = check_operand(fn, logits_grad, ld_g, "logits_grad")) return e;
  if (!labels || !lse || !denom) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  const int64_t col_blocks = (kpad + kZgCols - 1) / kZgCols;
  if (col_blocks > 65535) return fail(RUS_ERR_INVALID, "%s: n_vocab too large", fn);
  hipLaunchKernelGGL(lmhead_grad_from_logits_kernel,
                     dim3(static_cast<unsigned>(n_tok), static_cast<unsigned>(col_blocks)),
                     dim3(kZgThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<f16*>(logits_grad), ld_g, static_cast<int>(n_vocab),
                     static_cast<int>(kpad), labels, lse, denom, static_cast<int>(vocab_start));
  return check_launch(fn);
}

extern "C" int rus_lmhead_ce_combine(const float* part_m, const float* part_s, const float* part_w,
                                     const int32_t* part_idx, int64_t n_parts,
                                     int64_t part_stride, const float* target,
                                     const int64_t* labels, int64_t n_tok, float* lse,
                                     float* nll, float* entropy, int64_t* argmax, void* stream) {
  const char* fn = "rus_lmhead_ce_combine";
  if (n_tok < 0 || n_tok >= (1 << 30) || n_parts <= 0 || n_parts >= (1 << 30) ||
      part_stride < n_tok)
    return fail(RUS_ERR_INVALID, "%s: bad sizes", fn);
  if (n_tok == 0) return RUS_OK;
  if (!part_m || !part_s || !part_w || !part_idx || !target || !labels || !lse || !nll ||
      !entropy || !argmax)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  const dim3 grid(static_cast<unsigned>((n_tok + 63) / 64));
  hipLaunchKernelGGL(lmhead_combine_kernel, grid, dim3(kCombWaves * 64), 0,
                     static_cast<hipStream_t>(stream), part_m, part_s, part_w, part_idx,
                     static_cast<int>(n_parts), part_stride, target, labels,
                     static_cast<int>(n_tok), lse, nll, entropy, argmax);
  return check_launch(fn);
}

namespace rus {
namespace {

// loss = sum(nll) / denom, denom = max(*num_items, 1) if given, else max(#(labels != -100), 1).
// One workgroup of 1024 threads (16 waves); fixed summation order, so repeated calls agree bitwise.
__global__ __launch_bounds__(1024) void lmhead_loss_kernel(const float* __restrict__ nll,
                                                           const int64_t* __restrict__ labels,
                                                           int n_tok,
                                                           const float* __restrict__ num_items,
                                                           float* __restrict__ loss,
                                                           float* __restrict__ denom) {
  __shared__ float s_sum[16], s_cnt[16];
  float sum = 0.0f, cnt = 0.0f;
  for (int i = threadIdx.x; i < n_tok; i += 1024) {
    if (nll) sum += nll[i];
    cnt += labels[i] != -100 ? 1.0f : 0.0f;
  }
  sum = wave_sum(sum);
  cnt = wave_sum(cnt);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) {
    s_sum[wave] = sum;
    s_cnt[wave] = cnt;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.0f, c = 0.0f;
    for (int w = 0; w < 16; ++w) {
      t += s_sum[w];
      c += s_cnt[w];
    }
    const float d = fmaxf(num_items ? *num_items : c, 1.0f);
    denom[0] = d;
    if (loss) loss[0] = t / d;
  }
}

}  // namespace
}  // namespace rus

extern "C" int rus_lmhead_ce_loss(const float* nll, const int64_t* labels, int64_t n_tok,
                                  const float* num_items, float* loss, float* denom,
                                  void* stream) {
  using namespace rus;
  const char* fn = "rus_lmhead_ce_loss";
  if (n_tok < 0 || n_tok >= (int64_t(1) << 31))
    return fail(RUS_ERR_INVALID, "%s: n_tok=%lld outside [0, 2^31)", fn, (long long)n_tok);
  if ((n_tok > 0 && !labels) || (nll && !loss) || !denom)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  hipLaunchKernelGGL(lmhead_loss_kernel, dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream),
                     nll, labels, static_cast<int>(n_tok), num_items, loss, denom);
  return check_launch(fn);
}

extern "C" int rus_lmhead_ce_grad_logits(const void* hidden, const void* weight,
                                         const int64_t* labels, const float* lse,
                                         const float* denom, int64_t n_tok, int64_t d,
                                         int64_t ld_h, int64_t ld_w, int64_t n_vocab,
                                         int64_t vocab_start, void* grad_logits, int64_t ld_g,
                                         void* stream) {
  const char* fn = "rus_lmhead_ce_grad_logits";
  if (n_tok < 0 || n_tok >= (1 << 30) || n_vocab < 0 || n_vocab >= (1 << 30) || d <= 0 ||
      d % kBK || vocab_start < 0 || vocab_start + n_vocab >= (int64_t(1) << 31))
    return fail(RUS_ERR_INVALID, "%s: bad sizes (d must be a multiple of %d)", fn, kBK);
  if (n_tok == 0 || n_vocab == 0) return RUS_OK;
  const int64_t kpad = (n_vocab + kBK - 1) / kBK * kBK;
  if (ld_h < d || ld_w < d || ld_g < kpad)
    return fail(RUS_ERR_INVALID, "%s: row strides too small (ld_g must be >= %lld)", fn,
                (long long)kpad);
  if (int e = check_operand(fn, hidden, ld_h, "hidden")) return e;
  if (int e = check_operand(fn, weight, ld_w, "weight")) return e;
  if (int e = check_operand(fn, grad_logits, ld_g, "grad_logits")) return e;
  if (!labels || !lse || !denom) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  GemmArgs g;
  g.A = static_cast<const f16*>(weight);
  g.lda = ld_w;
  g.M = static_cast<int>(n_vocab);
  g.B = static_cast<const f16*>(hidden);
  g.ldb = ld_h;
  g.N = static_cast<int>(n_tok);
  g.K = static_cast<int>(d);
  g.k_per_split = g.K;
  g.splits = 1;
  g.tiles_m = (g.M + kBM - 1) / kBM;
  g.tiles_n = (g.N + kBN - 1) / kBN;
  GradParams p{labels, lse, denom, static_cast<f16*>(grad_logits), ld_g, static_cast<int>(kpad),
               static_cast<int>(vocab_start)};
  hipLaunchKernelGGL(lmhead_grad_logits_kernel, dim3(launch_grid(g)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), g, p);
  return check_launch(fn);
}

// allow_empty: splits past the last non-empty one still run (empty K range, so their epilogue
// only rescales: parts = parts * alpha + 0).
static int grad_hidden(const char* fn, const void* grad_logits, int64_t ld_g, const void* weight_t,
                       int64_t ld_wt, int64_t n_tok, int64_t d, int64_t n_vocab, float* parts,
                       int32_t n_split, int32_t accumulate, const float* alpha, bool allow_empty,
                       void* stream) {
  if (n_tok < 0 || n_tok >= (1 << 30) || d <= 0 || d >= (1 << 30) || n_vocab < 0 ||
      n_vocab >= (1 << 30) || n_split <= 0 || n_split > 64)
    return fail(RUS_ERR_INVALID, "%s: bad sizes or n_split=%d (1..64)", fn, n_split);
  if (n_tok == 0) return RUS_OK;
  const int64_t kpad = (n_vocab + kBK - 1) / kBK * kBK;
  if (ld_g < kpad || ld_wt < kpad)
    return fail(RUS_ERR_INVALID,
                "%s: grad_logits / weight_t rows must hold round_up(n_vocab, 64)=%lld columns",
                fn, (long long)kpad);
  if (int e = check_operand(fn, grad_logits, ld_g, "grad_logits")) return e;
  if (int e = check_operand(fn, weight_t, ld_wt, "weight_t")) return e;
  if (!parts) return fail(RUS_ERR_INVALID, "%s: parts is null", fn);
  if (kpad == 0) return RUS_OK;
  GemmArgs g;
  g.A = static_cast<const f16*>(grad_logits);
  g.lda = ld_g;
  g.M = static_cast<int>(n_tok);
  g.B = static_cast<const f16*>(weight_t);
  g.ldb = ld_wt;
  g.N = static_cast<int>(d);
  g.K = static_cast<int>(kpad);
  const int64_t per = (kpad + n_split - 1) / n_split;
  g.k_per_split = static_cast<int>((per + kBK - 1) / kBK * kBK);
  g.splits = static_cast<int>((kpad + g.k_per_split - 1) / g.k_per_split);
  if (allow_empty) g.splits = n_split;
  if (g.splits != n_split)
    return fail(RUS_ERR_INVALID, "%s: n_split=%d does not divide K=%lld into 64-wide pieces", fn,
                n_split, (long long)kpad);
  g.tiles_m = (g.M + kBM - 1) / kBM;
  g.tiles_n = (g.N + kBN - 1) / kBN;
  StoreParams p{parts, accumulate, alpha};
  hipLaunchKernelGGL(lmhead_grad_hidden_kernel, dim3(launch_grid(g)), dim3(kThreads8), 0,
                     static_cast<hipStream_t>(stream), g, p);
  return check_launch(fn);
}

extern "C" int rus_lmhead_ce_grad_hidden(const void* grad_logits, int64_t ld_g,
                                         const void* weight_t, int64_t ld_wt, int64_t n_tok,
                                         int64_t d, int64_t n_vocab, float* parts,
                                         int32_t n_split, int32_t accumulate, void* stream) {
  return grad_hidden("rus_lmhead_ce_grad_hidden", grad_logits, ld_g, weight_t, ld_wt, n_tok, d,
                     n_vocab, parts, n_split, accumulate, nullptr, false, stream);
}

extern "C" int rus_lmhead_ce_grad_hidden_scaled(const void* probs, int64_t ld_p,
                                                const void* weight_t, int64_t ld_wt,
                                                int64_t n_tok, int64_t d, int64_t n_vocab,
                                                float* parts, int32_t n_split,
                                                int32_t accumulate, const float* alpha,
                                                void* stream) {
  const char* fn = "rus_lmhead_ce_grad_hidden_scaled";
  if (accumulate && !alpha) return fail(RUS_ERR_INVALID, "%s: alpha is null", fn);
  return grad_hidden(fn, probs, ld_p, weight_t, ld_wt, n_tok, d, n_vocab, parts, n_split,
                     accumulate, alpha, true, stream);
}

extern "C" int rus_lmhead_ce_chunk_scale(void* logits, int64_t ld_z, int64_t n_tok,
                                         int64_t n_vocab, const float* part_m,
                                         int64_t part_stride, int64_t part_base, float* m_run,
                                         float* alpha, int32_t first, void* stream) {
  const char* fn = "rus_lmhead_ce_chunk_scale";
  if (n_tok < 0 || n_tok >= (1 << 30) || n_vocab < 0 || n_vocab >= (1 << 30) || part_base < 0 ||
      part_base >= (1 << 30) || part_stride < n_tok)
    return fail(RUS_ERR_INVALID, "%s: bad sizes", fn);
  if (n_tok == 0 || n_vocab == 0) return RUS_OK;
  const int64_t kpad = (n_vocab + kBK - 1) / kBK * kBK;
  if (ld_z < kpad) return fail(RUS_ERR_INVALID, "%s: ld_z must be >= %lld", fn, (long long)kpad);
  if (int e = check_operand(fn, logits, ld_z, "logits")) return e;
  if (!part_m || !m_run || !alpha) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  const int64_t col_blocks = (kpad + kZgCols - 1) / kZgCols;
  if (col_blocks > 65535) return fail(RUS_ERR_INVALID, "%s: n_vocab too large", fn);
  const int n_parts = static_cast<int>((n_vocab + kBM - 1) / kBM);
  hipLaunchKernelGGL(lmhead_chunk_scale_kernel,
                     dim3(static_cast<unsigned>(n_tok), static_cast<unsigned>(col_blocks)),
                     dim3(kZgThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<f16*>(logits), ld_z, static_cast<int>(n_vocab),
                     static_cast<int>(kpad), part_m, part_stride, static_cast<int>(part_base),
                     n_parts, m_run, alpha, first ? 1 : 0);
  return check_launch(fn);
}

extern "C" int rus_lmhead_ce_dh_finish(const float* parts, int32_t n_parts, int64_t n_tok,
                                       int64_t d, const float* m_run, const float* lse,
                                       const int64_t* labels, const void* w_rows, int64_t ld_w,
                                       int64_t n_vocab, int32_t w_on_host, const float* denom,
                                       float scale, const float* scale_dev, void* out,
                                       int32_t out_dtype, void* stream) {
  const char* fn = "rus_lmhead_ce_dh_finish";
  if (n_parts <= 0 || n_tok < 0 || n_tok >= (1 << 30) || d <= 0 || d % 4 || d >= (1 << 30) ||
      n_vocab < 0 || ld_w < d || (out_dtype != RUS_DTYPE_F16 && out_dtype != RUS_DTYPE_F32))
    return fail(RUS_ERR_INVALID, "%s: bad arguments (d must be a multiple of 4)", fn);
  if (n_tok == 0) return RUS_OK;
  if (!parts || !m_run || !lse || !labels || !w_rows || !denom || !out || !aligned(parts, 16) ||
      !aligned(out, 16) || !aligned(w_rows, 8) || ld_w % 4)
    return fail(RUS_ERR_INVALID, "%s: null or misaligned pointer", fn);
  const void* w = w_rows;
  if (w_on_host) {  // pinned host rows are read through their device mapping
    void* mapped = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&mapped, const_cast<void*>(w_rows), 0);
    if (e != hipSuccess || !mapped)
      return fail(RUS_ERR_INVALID, "%s: w_rows is not page-locked, device-mapped host memory (%s)",
                  fn, hipGetErrorString(e));
    w = mapped;
  }
  const int64_t n = n_tok * d;
  const dim3 grid(static_cast<unsigned>((n / 4 + 255) / 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (out_dtype == RUS_DTYPE_F16)
    hipLaunchKernelGGL(lmhead_dh_finish_kernel<f16>, grid, dim3(256), 0, st, parts, n_parts,
                       static_cast<int>(n_tok), static_cast<int>(d), m_run, lse, labels,
                       static_cast<const f16*>(w), ld_w, n_vocab, denom, scale, scale_dev,
                       static_cast<f16*>(out));
  else
    hipLaunchKernelGGL(lmhead_dh_finish_kernel<float>, grid, dim3(256), 0, st, parts, n_parts,
                       static_cast<int>(n_tok), static_cast<int>(d), m_run, lse, labels,
                       static_cast<const f16*>(w), ld_w, n_vocab, denom, scale, scale_dev,
                       static_cast<float*>(out));
  return check_launch(fn);
}

extern "C" int rus_lmhead_dh_reduce(const float* parts, int32_t n_parts, int64_t n_elem,
                                    float scale, const float* scale_dev, void* out,
                                    int32_t out_dtype, void* stream) {
  const char* fn = "rus_lmhead_dh_reduce";
  if (n_parts <= 0 || n_elem < 0 || (out_dtype != RUS_DTYPE_F16 && out_dtype != RUS_DTYPE_F32))
    return fail(RUS_ERR_INVALID, "%s: bad arguments", fn);
  if (n_elem == 0) return RUS_OK;
  if (!parts || !out || !aligned(parts, 16) || !aligned(out, 16))
    return fail(RUS_ERR_INVALID, "%s: parts/out must be non-null and 16-byte aligned", fn);
  const dim3 grid(static_cast<unsigned>((n_elem + 1023) / 1024));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = n_elem % 4 == 0;
  if (out_dtype == RUS_DTYPE_F16) {
    if (vec)
      hipLaunchKernelGGL((dh_reduce_kernel<f16, true>), grid, dim3(256), 0, st, parts, n_parts,
                         n_elem, scale, scale_dev, static_cast<f16*>(out));
    else
      hipLaunchKernelGGL((dh_reduce_kernel<f16, false>), grid, dim3(256), 0, st, parts, n_parts,
                         n_elem, scale, scale_dev, static_cast<f16*>(out));
  } else {
    if (vec)
      hipLaunchKernelGGL((dh_reduce_kernel<float, true>), grid, dim3(256), 0, st, parts, n_parts,
                         n_elem, scale, scale_dev, static_cast<float*>(out));
    else
      hipLaunchKernelGGL((dh_reduce_kernel<float, false>), grid, dim3(256), 0, st, parts, n_parts,
                         n_elem, scale, scale_dev, static_cast<float*>(out));
  }
  return check_launch(fn);
}

extern "C" int rus_transpose_f16(const void* src, int64_t rows, int64_t cols, int64_t ld_src,
                                 void* dst, int64_t ld_dst, int64_t rows_pad, void* stream) {
  const char* fn = "rus_transpose_f16";
  if (rows < 0 || cols < 0 || rows_pad < rows || ld_src < cols || ld_dst < rows_pad)
    return fail(RUS_ERR_INVALID, "%s: bad sizes or strides", fn);
  if (rows_pad == 0 || cols == 0) return RUS_OK;
  if (!src || !dst) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  const int64_t gx = (rows_pad + 63) / 64, gy = (cols + 63) / 64;
  if (gx >= (int64_t(1) << 31) || gy > 65535)
    return fail(RUS_ERR_INVALID, "%s: matrix too large", fn);
  hipLaunchKernelGGL(transpose_f16_kernel, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                     dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<const f16*>(src),
                     rows, cols, ld_src, static_cast<f16*>(dst), ld_dst, rows_pad);
  return check_launch(fn);
}

extern "C" int rus_lmhead_ce_logits(const void* hidden, const void* weight, int64_t n_tok,
                                    int64_t d, int64_t ld_h, int64_t ld_w, int64_t n_vocab,
                                    void* logits, int64_t ld_z, void* stream) {
  const char* fn = "rus_lmhead_ce_logits";
  if (n_tok < 0 || n_tok >= (1 << 30) || n_vocab < 0 || n_vocab >= (1 << 30) || d <= 0 ||
      d % kBK)
    return fail(RUS_ERR_INVALID, "%s: bad sizes (d must be a multiple of %d)", fn, kBK);
  if (n_tok == 0 || n_vocab == 0) return RUS_OK;
  const int64_t kpad = (n_vocab + kBK - 1) / kBK * kBK;
  if (ld_h < d || ld_w < d || ld_z < kpad)
    return fail(RUS_ERR_INVALID, "%s: row strides too small (ld_z must be >= %lld)", fn,
                (long long)kpad);
  if (int e = check_operand(fn, hidden, ld_h, "hidden")) return e;
  if (int e = check_operand(fn, weight, ld_w, "weight")) return e;
  if (int e = check_operand(fn, logits, ld_z, "logits")) return e;
  GemmArgs g;
  g.A = static_cast<const f16*>(weight);
  g.lda = ld_w;
  g.M = static_cast<int>(n_vocab);
  g.B = static_cast<const f16*>(hidden);
  g.ldb = ld_h;
  g.N = static_cast<int>(n_tok);
  g.K = static_cast<int>(d);
  g.k_per_split = g.K;
  g.splits = 1;
  g.tiles_m = (g.M + kBM - 1) / kBM;
  g.tiles_n = (g.N + kBN - 1) / kBN;
  LogitsParams p{static_cast<f16*>(logits), ld_z, static_cast<int>(kpad)};
  hipLaunchKernelGGL(lmhead_logits_kernel, dim3(launch_grid(g)), dim3(kThreads8), 0,
                     static_cast<hipStream_t>(stream), g, p);
  return check_launch(fn);
}

extern "C" int rus_lmhead_ce_rows(void* logits, int64_t ld_z, int64_t n_tok, int64_t n_vocab,
                                  const int64_t* labels, const float* denom, float* lse,
                                  float* nll, float* entropy, int64_t* argmax, void* stream) {
  const char* fn = "rus_lmhead_ce_rows";
  if (n_tok < 0 || n_tok >= (1 << 30) || n_vocab <= 0 || n_vocab >= (1 << 30))
    return fail(RUS_ERR_INVALID, "%s: bad sizes", fn);
  if (n_tok == 0) return RUS_OK;
  const int64_t kpad = (n_vocab + kBK - 1) / kBK * kBK;
  if (ld_z < kpad) return fail(RUS_ERR_INVALID, "%s: ld_z must be >= %lld", fn, (long long)kpad);
  if (int e = check_operand(fn, logits, ld_z, "logits")) return e;
  if (!labels || !lse || !nll || !entropy || !argmax)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  hipLaunchKernelGGL(lmhead_rows_kernel, dim3(static_cast<unsigned>(n_tok)), dim3(kRowThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<f16*>(logits), ld_z,
                     static_cast<int>(n_vocab), static_cast<int>(kpad), labels, denom, lse, nll,
                     entropy, argmax);
  return check_launch(fn);
}
