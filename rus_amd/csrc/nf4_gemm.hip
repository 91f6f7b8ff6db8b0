// NF4 W4A16 products for gfx950: GEMMs against a frozen NF4 double-quant weight whose
// dequantisation runs inside the MFMA main loop, so no fp16 copy of the weight is written to or
// read from HBM.
//
// Reference: the F.linear / torch.mm calls on the dequantised layer weights of the packed stack
// (solution/ops.py:759-807 forward, 898-966 backward), each on the fp16 output of
// nf4_dequant_turing_kernel (solution/kernels.py:27-118):
//   trans = 0 (forward):  Y[m, n] = fp16( sum_k X[m, k] W[n, k] )   X [M, Kw], W [Nw, Kw], Y [M, Nw]
//   trans = 1 (backward): Y[m, k] = fp16( sum_n X[m, n] W[n, k] )   X [M, Nw],             Y [M, Kw]
// W[n, k] = fp16(NF4[code] * scale(block)) is exactly what rus_nf4_dequant writes (same code
// order, same scale = code2[absmax] * absmax2[super] + segment offset with two roundings); the
// sums are fp32 (MFMA) and rounded once.
//
// Design (CDNA4, wave64, v_mfma_f32_32x32x16_f16):
//   * block tile: 256 tokens x BN output columns (BN = 128 or 64), 4 waves as 2 (columns) x 2
//     (tokens), each wave 128 tokens x BN/2 columns; the reduction runs in steps of 64 = one NF4
//     block along a weight row;
//   * per step the block stages the activation tile (256 x 64 fp16, loaded 8 lanes per 128-byte
//     row) and the dequantised weight tile (BN x 64, transposed on the way in for trans = 1) in
//     LDS, double buffered: a step's global loads are issued two steps ahead, its decode runs
//     beside the previous step's MFMAs, one barrier per step; each weight element is decoded
//     once per 256-token tile;
//   * MFMAs compute C[column][token] (weights as the A operand), so a lane's accumulators hold 4
//     runs of 4 consecutive output columns of one token: 8-byte fp16 stores;
//   * narrow outputs split the reduction over blocks (fp32 partials in a caller workspace); the
//     last block of a tile to finish (arrival counter, left at zero) adds the partials in split
//     order and rounds once: deterministic, one launch;
//   * blocks are numbered XCD-major, so the token tiles that share a weight tile run on one XCD
//     (one L2) and the packed weight is read from HBM about once.

#include "common.h"

namespace rus {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// NF4 code points in nibble order (QLoRA normal-float-4 table; solution/kernels.py:76-83).
__constant__ float kNF4Codes[16] = {
    -1.0f,
    -0.6961928009986877f,
    -0.5250730514526367f,
    -0.39491748809814453f,
    -0.28444138169288635f,
    -0.18477343022823334f,
    -0.09105003625154495f,
    0.0f,
    0.07958029955625534f,
    0.16093020141124725f,
    0.24611230194568634f,
    0.33791524171829224f,
    0.44070982933044434f,
    0.5626170039176941f,
    0.7229568362236023f,
    1.0f,
};

constexpr int kBM = 256;       // tokens per tile
constexpr int kBK = 64;        // reduction step (= NF4 blocksize)
constexpr int kLd = 72;        // LDS row stride in halfs (144 B: conflict-free 16-byte reads)
constexpr int kThreads = 512;  // 4 MFMA waves + 4 loader waves: one of each per SIMD
constexpr int kHalf = 256;     // threads per role
constexpr int kTJ = 4;         // 32-token MFMA tiles per MFMA wave (128 tokens)
constexpr int kARows = kHalf / 8;  // activation rows per coalesced load (8 lanes per row)

struct GemmArgs {
  const f16* x;
  int64_t sx;
  int m;
  const uint8_t* packed;
  const uint8_t* absmax;
  const float* absmax2;
  const float* code2;
  float off0, off1, off2;
  int64_t row1, row2;      // first weight row of segment 1 / 2 (w_rows: segment absent)
  int64_t blk0_1, blk0_2;  // first absmax block of segment 1 / 2
  int64_t sbase1, sbase2;  // first absmax2 entry of segment 1 / 2
  int sb_shift;            // log2(super_blocksize)
  int64_t w_cols;          // Kw
  const f16* bias;  // [n_out] added to the fp32 sums before rounding (trans = 0; nullptr: none)
  f16* y;
  int64_t sy;
  int mt, nt, ks;        // token tiles, column tiles, reduction splits
  int steps, per_split;  // reduction steps in total / per split
  float* part;
  int* counters;
};

__device__ __forceinline__ f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// One reduction step's global operands of this thread, loaded one step ahead of their use:
// 8 activation chunks of 16 bytes (rows r0 + 32 i, coalesced: 8 lanes cover a 128-byte row) and
// the packed codes this thread decodes into the shared weight tile.
template <int EPT>
struct Stage {
  u32x4 a[kBM / kARows];
  uint32_t w[EPT / 8];  // EPT packed NF4 codes
  uint32_t code;        // absmax byte of the weight block
  float a2, off;        // absmax2 entry and segment offset
};

// TI: 32-column MFMA tiles per MFMA wave (BN = 64 TI); TRANS: contraction over weight rows.
// Waves 0-3 (one per SIMD) run the MFMAs of a step from one LDS buffer while waves 4-7 (the
// loaders, one per SIMD) fill the other: global loads two steps ahead, NF4 decode, LDS stores.
// The two roles share each SIMD, so decode and load issue overlap the matrix-core work.
template <int TI, bool TRANS>
__global__ __launch_bounds__(kThreads) void nf4_gemm_kernel(GemmArgs a) {
  constexpr int BN = 2 * TI * 32;
  constexpr int EPT = BN * kBK / kHalf;  // weight elements decoded per loader thread per step
  __shared__ __attribute__((aligned(16))) f16 sA[2][kBM * kLd];  // tokens x reduction
  // Weight tile: output column c at c * kLd + 16 (c / EPT) halfs. The per-group shift puts the
  // transposed stores of the 4 column groups that one wave writes (trans = 1) on distinct banks.
  constexpr int kBsz = BN * kLd + 16 * (BN / EPT);
  __shared__ __attribute__((aligned(16))) f16 sB[2][kBsz];  // output columns x reduction
  __shared__ float s_code2[256];
  __shared__ float2 s_pair[256];  // code points of the high and low nibble of each byte value

  // XCD-major block numbering (blocks are dispatched to the 8 XCDs round robin); the grid is a
  // multiple of 8 and the spare blocks exit before any barrier.
  const int nb = gridDim.x, b = blockIdx.x;
  const int idx = (b & 7) * (nb >> 3) + (b >> 3);
  if (idx >= a.mt * a.nt * a.ks) return;
  const int mtile = idx % a.mt, ntile = (idx / a.mt) % a.nt, split = idx / (a.mt * a.nt);
  const int s_begin = split * a.per_split;
  const int s_end = min(s_begin + a.per_split, a.steps);
  const int tid = threadIdx.x, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform role
  const bool mfma_wave = wave < 4;
  const int64_t m0 = static_cast<int64_t>(mtile) * kBM;
  const int64_t c0 = static_cast<int64_t>(ntile) * BN;  // first output column

  for (int i = tid; i < 256; i += kThreads) {
    s_code2[i] = a.code2[i];
    s_pair[i] = float2{kNF4Codes[i >> 4], kNF4Codes[i & 15]};
  }

  f32x16 acc[TI][kTJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < kTJ; ++j) acc[i][j] = f32x16{};
  const int wn = wave & 1, wm = (wave >> 1) & 1;

  if (mfma_wave) {
    // MFMAs of one step from LDS buffer `buf`: weight fragments (A operand, columns
    // wn*32TI + 32i) and activation fragments (B operand, tokens wm*128 + 32j); C[column][token].
    __syncthreads();  // tables
    __syncthreads();  // first step stored
    const int col = wn * TI * 32 + l32;  // + 32 i
    for (int s = s_begin; s < s_end; ++s) {
      const int buf = (s - s_begin) & 1;
      const f16* bw = sB[buf] + col * kLd + 16 * (col / EPT) + 8 * h;
      const f16* bt = sA[buf] + (wm * kTJ * 32 + l32) * kLd + 8 * h;
#pragma unroll
      for (int kk = 0; kk < kBK / 16; ++kk) {
        f16x8 fw[TI], ft[kTJ];
#pragma unroll
        for (int i = 0; i < TI; ++i)  // 32 i columns further: 32 i kLd + 16 (32 i / EPT) halfs
          fw[i] = *reinterpret_cast<const f16x8*>(bw + i * 32 * kLd + 16 * (i * 32 / EPT) + kk * 16);
#pragma unroll
        for (int j = 0; j < kTJ; ++j)
          ft[j] = *reinterpret_cast<const f16x8*>(bt + j * 32 * kLd + kk * 16);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < kTJ; ++j) acc[i][j] = mfma(fw[i], ft[j], acc[i][j]);
      }
      __syncthreads();  // buffer `buf` free; the other one stored
    }
  } else {
    const int lt = tid - kHalf;  // loader thread index
    // Activation loads: chunk lt % 8 (16 bytes) of rows lt / 8 + 32 i; rows past the end read
    // row m - 1 and are not stored.
    const int a_row = lt >> 3, a_chunk = lt & 7;
    const f16* ap[kBM / kARows];
#pragma unroll
    for (int i = 0; i < kBM / kARows; ++i) {
      const int64_t t = m0 + a_row + kARows * i;
      ap[i] = a.x + (t < a.m ? t : a.m - 1) * a.sx + 8 * a_chunk;
    }
    // Weight codes this thread decodes per step. trans = 0: row c0 + wr, EPT codes at wq * EPT
    // of the step (64 / EPT threads per row). trans = 1: step row wr = lt / (BN / EPT), EPT
    // columns at c0 + wq * EPT (BN / EPT threads per row: a wave reads whole row segments).
    constexpr int kPerRow = TRANS ? BN / EPT : kBK / EPT;
    const int wr = lt / kPerRow, wq = lt % kPerRow;

    // Segment constants of the weight rows this thread decodes. trans = 0: the row (c0 + wr) is
    // fixed for the whole loop. trans = 1: the step's 64 rows share one segment (segment starts
    // are multiples of 64 rows), chosen per step by integer arithmetic (selects of loaded values
    // would become loads of selected addresses and keep the captures in scratch memory).
    const int64_t kb1 = a.blk0_1, kb2 = a.blk0_2, kbs1 = a.sbase1, kbs2 = a.sbase2;
    const int64_t krow1 = a.row1, krow2 = a.row2, w_cols = a.w_cols;
    const int sb_shift = a.sb_shift;
    const uint8_t* __restrict__ absmax = a.absmax;
    const float* __restrict__ absmax2 = a.absmax2;
    const uint8_t* __restrict__ packed = a.packed;
    const float ko0 = a.off0, ko1 = a.off1, ko2 = a.off2;
    const uint32_t ob0 = __builtin_bit_cast(uint32_t, ko0),
                   ob1 = __builtin_bit_cast(uint32_t, ko1),
                   ob2 = __builtin_bit_cast(uint32_t, ko2);
    int64_t fix_blk0 = 0, fix_base = 0;
    float fix_off = ko0;
    if constexpr (!TRANS) {
      const int64_t n = c0 + wr;
      fix_blk0 = n >= krow2 ? kb2 : (n >= krow1 ? kb1 : 0);
      fix_base = n >= krow2 ? kbs2 : (n >= krow1 ? kbs1 : 0);
      fix_off = n >= krow2 ? ko2 : (n >= krow1 ? ko1 : ko0);
    }

    auto prefetch = [=](int s, Stage<EPT>& p) __attribute__((always_inline)) {
      int64_t e, blk0, base;
      if constexpr (!TRANS) {
        e = (c0 + wr) * w_cols + static_cast<int64_t>(s) * kBK + wq * EPT;
        blk0 = fix_blk0;
        base = fix_base;
        p.off = fix_off;
      } else {
        const int64_t r0 = static_cast<int64_t>(s) * kBK;  // first row of the step (uniform)
        e = (r0 + wr) * w_cols + c0 + wq * EPT;
        const int64_t in1 = r0 >= krow1, in2 = r0 >= krow2;
        blk0 = in1 * kb1 + in2 * (kb2 - kb1);
        base = in1 * kbs1 + in2 * (kbs2 - kbs1);
        p.off = __builtin_bit_cast(float, ob0 + static_cast<uint32_t>(in1) * (ob1 - ob0) +
                                              static_cast<uint32_t>(in2) * (ob2 - ob1));
      }
      const int64_t blk = e >> 6;
      p.code = absmax[blk];
      p.a2 = absmax2[base + ((blk - blk0) >> sb_shift)];
      const uint32_t* wp = reinterpret_cast<const uint32_t*>(packed + (e >> 1));
#pragma unroll
      for (int i = 0; i < EPT / 8; ++i) p.w[i] = wp[i];
#pragma unroll
      for (int i = 0; i < kBM / kARows; ++i)
        p.a[i] = *reinterpret_cast<const u32x4*>(ap[i] + static_cast<int64_t>(s) * kBK);
    };

    // Decodes a prefetched step into LDS buffer `buf`: the code2 entry and, per packed byte,
    // the code points of both nibbles (LDS tables), scaled and rounded; the activation chunks
    // copied.
    auto produce = [=](const Stage<EPT>& p, int buf) __attribute__((always_inline)) {
      const float cv = s_code2[p.code];
      float2 lv[EPT / 2];
#pragma unroll
      for (int i = 0; i < EPT / 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) lv[4 * i + j] = s_pair[(p.w[i] >> (8 * j)) & 0xffu];
#pragma unroll
      for (int i = 0; i < kBM / kARows; ++i)
        *reinterpret_cast<u32x4*>(sA[buf] + (a_row + kARows * i) * kLd + 8 * a_chunk) = p.a[i];
      const float c = cv * p.a2;  // two roundings (no contraction in this library)
      const float scale = c + p.off;
      f16 v[EPT];
#pragma unroll
      for (int q = 0; q < EPT / 2; ++q) {  // byte q: high nibble = even element
        v[2 * q] = from_f32<f16>(lv[q].x * scale);
        v[2 * q + 1] = from_f32<f16>(lv[q].y * scale);
      }
      if constexpr (!TRANS) {
        f16* db = sB[buf] + wr * kLd + 16 * (wr / EPT) + wq * EPT;
#pragma unroll
        for (int i = 0; i < EPT / 8; ++i) {
          f16x8 t;
#pragma unroll
          for (int k = 0; k < 8; ++k) t[k] = v[8 * i + k];
          *reinterpret_cast<f16x8*>(db + 8 * i) = t;
        }
      } else {
        f16* db = sB[buf] + (wq * EPT) * kLd + 16 * wq + wr;  // transposed: row = column
#pragma unroll
        for (int i = 0; i < EPT; ++i) db[i * kLd] = v[i];
      }
    };

    // Two register stages, each loaded two steps before it is decoded. Steps past the end
    // reload the last step (in range) and are never used.
    Stage<EPT> pf[2];
    prefetch(s_begin, pf[0]);
    prefetch(min(s_begin + 1, s_end - 1), pf[1]);
    __syncthreads();  // tables
    produce(pf[0], 0);
    prefetch(min(s_begin + 2, s_end - 1), pf[0]);
    __syncthreads();  // first step stored
    int s = s_begin;
    // Iteration s: decode step s + 1 (stage (s+1) % 2) into the idle buffer, refill that stage
    // with step s + 3.
    auto iter = [&](int s, Stage<EPT>& st) __attribute__((always_inline)) {
      produce(st, ((s - s_begin) & 1) ^ 1);
      prefetch(min(s + 3, s_end - 1), st);
      __syncthreads();
    };
    for (; s + 2 <= s_end; s += 2) {
      iter(s, pf[1]);
      iter(s + 1, pf[0]);
    }
    if (s < s_end) iter(s, pf[1]);
  }

  // Epilogue (MFMA waves): lane holds token m0 + wm*128 + 32 j + l32 and, per accumulator, the
  // 16 columns 8 (r / 4) + 4 h + r % 4 of its 32-column tile (4 runs of 4 consecutive columns).
  const int cw_wave = mfma_wave ? wave : 0;
  if (a.ks > 1) {
    constexpr int kTile = kBM * BN;  // floats per partial tile
    const int tile = mtile + a.mt * ntile;
    float* mine = a.part + (static_cast<int64_t>(split) * a.mt * a.nt + tile) * kTile;
    if (mfma_wave) {
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < kTJ; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            store_partial(mine + (((cw_wave * TI + i) * kTJ + j) * 16 + r) * 64 + lane,
                          acc[i][j][r]);
    }
    if (!arrive_last(a.counters + tile, a.ks)) return;
    if (!mfma_wave) return;
    // Sum every split's partial in split order.
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < kTJ; ++j) acc[i][j] = f32x16{};
    for (int c = 0; c < a.ks; ++c) {
      const float* pc = a.part + (static_cast<int64_t>(c) * a.mt * a.nt + tile) * kTile;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < kTJ; ++j) {
          f32x16 v;
#pragma unroll
          for (int r = 0; r < 16; ++r)
            v[r] = load_partial(pc + (((cw_wave * TI + i) * kTJ + j) * 16 + r) * 64 + lane);
          acc[i][j] += v;
        }
    }
  }
  if (!mfma_wave) return;
  const int64_t cw = c0 + wn * TI * 32 + 4 * h;  // this lane's first output column
#pragma unroll
  for (int j = 0; j < kTJ; ++j) {
    const int64_t m = m0 + wm * kTJ * 32 + 32 * j + l32;
    if (m >= a.m) continue;
    f16* yrow = a.y + m * a.sy + cw;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f16x4 bv = a.bias ? *reinterpret_cast<const f16x4*>(a.bias + cw + i * 32 + 8 * r4)
                                : f16x4{0, 0, 0, 0};
        f16x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
          o[k] = from_f32<f16>(acc[i][j][4 * r4 + k] + static_cast<float>(bv[k]));
        *reinterpret_cast<f16x4*>(yrow + i * 32 + 8 * r4) = o;
      }
  }
}

// Launch plan: column tile (TI), splits and scratch for a product shape.
struct Plan {
  int ti, mt, nt, ks, steps, per_split, grid;
  int64_t floats, counters;
};

constexpr int kMaxSplits = 8;
constexpr int kTargetBlocks = 256;  // one block per CU

Plan make_plan(int64_t m, int64_t n_out, int64_t n_red, int split) {
  Plan p{};
  const int mt = static_cast<int>((m + kBM - 1) / kBM);
  // 128-column tiles (each activation fragment feeds 4 MFMAs) when they give most CUs a block
  // without splitting the reduction, else 64-column tiles.
  p.ti = (n_out % 128 == 0 && mt * (n_out / 128) >= kTargetBlocks * 3 / 4) ? 2 : 1;
  const int bn = 2 * p.ti * 32;
  p.mt = mt;
  p.nt = static_cast<int>(n_out / bn);
  p.steps = static_cast<int>(n_red / kBK);
  int ks = split;
  if (ks <= 0) {
    const int tiles = p.mt * p.nt;
    ks = (kTargetBlocks + tiles - 1) / tiles;
    ks = ks < 1 ? 1 : (ks > kMaxSplits ? kMaxSplits : ks);
    const int min_steps = 4;  // keep the pipeline busy between the split boundaries
    if (ks > p.steps / min_steps) ks = p.steps / min_steps > 0 ? p.steps / min_steps : 1;
  }
  if (ks > p.steps) ks = p.steps;
  p.per_split = (p.steps + ks - 1) / ks;
  p.ks = (p.steps + p.per_split - 1) / p.per_split;  // no empty split
  const int64_t blocks = static_cast<int64_t>(p.mt) * p.nt * p.ks;
  p.grid = static_cast<int>((blocks + 7) / 8 * 8);
  p.floats = p.ks > 1 ? blocks * kBM * bn : 0;
  p.counters = p.ks > 1 ? static_cast<int64_t>(p.mt) * p.nt : 0;
  return p;
}

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << r) < v) ++r;
  return r;
}

int check_shape(const char* fn, int64_t m, int64_t w_rows, int64_t w_cols, int32_t trans) {
  if (trans != 0 && trans != 1) return fail(RUS_ERR_INVALID, "%s: trans must be 0 or 1", fn);
  if (m < 0 || m >= (int64_t(1) << 31) || w_rows <= 0 || w_cols <= 0)
    return fail(RUS_ERR_INVALID, "%s: bad sizes m=%lld w=[%lld, %lld]", fn, (long long)m,
                (long long)w_rows, (long long)w_cols);
  if (w_rows % 64 || w_cols % 64)
    return fail(RUS_ERR_UNSUPPORTED, "%s: weight dims must be multiples of 64, got [%lld, %lld]",
                fn, (long long)w_rows, (long long)w_cols);
  if (w_rows * w_cols / 2 >= (int64_t(1) << 31))
    return fail(RUS_ERR_UNSUPPORTED, "%s: weight of 2^32 or more elements", fn);
  return RUS_OK;
}

}  // namespace
}  // namespace rus

using rus::f16;

extern "C" int rus_nf4_gemm_plan(int64_t m, int64_t w_rows, int64_t w_cols, int32_t trans,
                                 int32_t* split, int64_t* workspace_floats, int64_t* n_counters) {
  using namespace rus;
  const char* fn = "rus_nf4_gemm_plan";
  if (!split || !workspace_floats || !n_counters) return fail(RUS_ERR_INVALID, "%s: null output", fn);
  if (int e = check_shape(fn, m, w_rows, w_cols, trans)) return e;
  const Plan p = make_plan(m, trans ? w_cols : w_rows, trans ? w_rows : w_cols, *split);
  *split = p.ks;
  *workspace_floats = p.floats;
  *n_counters = p.counters;
  return RUS_OK;
}

extern "C" int rus_nf4_gemm(const void* x, int64_t m, int64_t stride_x, const rus_nf4_job* w,
                            const float* code2, int64_t w_rows, int64_t w_cols, int32_t blocksize,
                            int32_t super_blocksize, int32_t trans, const void* bias, void* y,
                            int64_t stride_y,
                            int32_t split, float* workspace, int64_t workspace_floats,
                            int32_t* counters, int64_t n_counters, void* stream) {
  using namespace rus;
  const char* fn = "rus_nf4_gemm";
  if (int e = check_shape(fn, m, w_rows, w_cols, trans)) return e;
  if (!x || !w || !code2 || !y) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (!w->packed || !w->absmax || !w->absmax2)
    return fail(RUS_ERR_INVALID, "%s: null weight pointer", fn);
  if (blocksize != 64)
    return fail(RUS_ERR_UNSUPPORTED, "%s: blocksize %d (the fused product decodes 64-element "
                "blocks)", fn, blocksize);
  if (!is_pow2(super_blocksize))
    return fail(RUS_ERR_INVALID, "%s: super_blocksize %d is not a power of two", fn,
                super_blocksize);
  const int64_t n_in = trans ? w_rows : w_cols, n_out = trans ? w_cols : w_rows;
  if (stride_x < n_in || stride_x % 8 || stride_y < n_out || stride_y % 4)
    return fail(RUS_ERR_INVALID, "%s: need stride_x >= %lld (multiple of 8) and stride_y >= %lld "
                "(multiple of 4)", fn, (long long)n_in, (long long)n_out);
  if (!aligned(x, 16) || !aligned(y, 8) || !aligned(w->packed, 8) || !aligned(bias, 8))
    return fail(RUS_ERR_INVALID, "%s: x must be 16-, y, bias and packed 8-byte aligned", fn);
  if (bias && trans)
    return fail(RUS_ERR_INVALID, "%s: a bias applies to the forward product (trans = 0) only", fn);
  const int64_t n_bytes = w_rows * w_cols / 2;
  if (w->n_bytes != n_bytes)
    return fail(RUS_ERR_INVALID, "%s: job has %lld bytes, the [%lld, %lld] weight %lld", fn,
                (long long)w->n_bytes, (long long)w_rows, (long long)w_cols, (long long)n_bytes);
  const int64_t row_bytes = w_cols / 2;
  const int64_t s1 = w->split_byte_1, s2 = w->split_byte_2;
  if (s1 < 0 || s2 < s1 || s2 > n_bytes || s1 % row_bytes || s2 % row_bytes)
    return fail(RUS_ERR_INVALID, "%s: segment starts (%lld, %lld) must be ordered whole rows", fn,
                (long long)s1, (long long)s2);
  if (trans && ((s1 / row_bytes) % 64 || (s2 / row_bytes) % 64))
    return fail(RUS_ERR_UNSUPPORTED, "%s: trans = 1 needs segment starts at multiples of 64 "
                "rows", fn);
  if (w->absmax2_base_1 < 0 || w->absmax2_base_2 < w->absmax2_base_1)
    return fail(RUS_ERR_INVALID, "%s: absmax2 bases must be non-negative, ordered", fn);
  const int64_t n_blocks = n_bytes / 32;
  if (w->n_absmax < n_blocks)
    return fail(RUS_ERR_INVALID, "%s: absmax has %lld entries, needs %lld", fn,
                (long long)w->n_absmax, (long long)n_blocks);
  const int sb = ilog2(super_blocksize);
  const int64_t starts[3] = {0, s1, s2}, ends[3] = {s1, s2, n_bytes};
  const int64_t bases[3] = {0, w->absmax2_base_1, w->absmax2_base_2};
  for (int s = 0; s < 3; ++s) {
    if (ends[s] <= starts[s]) continue;
    const int64_t sup_last = bases[s] + (((ends[s] - 1) / 32 - starts[s] / 32) >> sb);
    if (sup_last >= w->n_absmax2)
      return fail(RUS_ERR_INVALID, "%s: absmax2 has %lld entries, segment %d needs index %lld",
                  fn, (long long)w->n_absmax2, s, (long long)sup_last);
  }
  if (m == 0) return RUS_OK;
  const Plan p = make_plan(m, n_out, n_in, split);
  if (split > 0 && p.ks != split)
    return fail(RUS_ERR_INVALID, "%s: split %d does not divide %d steps into non-empty parts "
                "(use rus_nf4_gemm_plan)", fn, split, p.steps);
  if (p.ks > 1) {
    if (!workspace || !counters || !aligned(workspace, 16) || !aligned(counters, 4))
      return fail(RUS_ERR_INVALID, "%s: split products need an aligned workspace and counters",
                  fn);
    if (workspace_floats < p.floats || n_counters < p.counters)
      return fail(RUS_ERR_INVALID, "%s: workspace holds %lld floats and %lld counters, needs "
                  "%lld and %lld", fn, (long long)workspace_floats, (long long)n_counters,
                  (long long)p.floats, (long long)p.counters);
  }
  if (static_cast<int64_t>(p.grid) >= (int64_t(1) << 31) / 2)
    return fail(RUS_ERR_UNSUPPORTED, "%s: grid too large", fn);
  GemmArgs a{};
  a.x = static_cast<const f16*>(x);
  a.sx = stride_x;
  a.m = static_cast<int>(m);
  a.packed = w->packed;
  a.absmax = w->absmax;
  a.absmax2 = w->absmax2;
  a.code2 = code2;
  a.off0 = w->off0;
  a.off1 = w->off1;
  a.off2 = w->off2;
  a.row1 = s1 / row_bytes;
  a.row2 = s2 / row_bytes;
  a.blk0_1 = s1 / 32;
  a.blk0_2 = s2 / 32;
  a.sbase1 = w->absmax2_base_1;
  a.sbase2 = w->absmax2_base_2;
  a.sb_shift = sb;
  a.w_cols = w_cols;
  a.bias = static_cast<const f16*>(bias);
  a.y = static_cast<f16*>(y);
  a.sy = stride_y;
  a.mt = p.mt;
  a.nt = p.nt;
  a.ks = p.ks;
  a.steps = p.steps;
  a.per_split = p.per_split;
  a.part = workspace;
  a.counters = counters;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(p.grid), block(kThreads);
  if (p.ti == 2) {
    if (trans)
      hipLaunchKernelGGL((nf4_gemm_kernel<2, true>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((nf4_gemm_kernel<2, false>), grid, block, 0, st, a);
  } else {
    if (trans)
      hipLaunchKernelGGL((nf4_gemm_kernel<1, true>), grid, block, 0, st, a);
    else
      hipLaunchKernelGGL((nf4_gemm_kernel<1, false>), grid, block, 0, st, a);
  }
  return check_launch(fn);
}
