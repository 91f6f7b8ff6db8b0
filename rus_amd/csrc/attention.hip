// Varlen causal GQA attention (forward and backward) on packed tokens for gfx950, head_dim 128.
//
// Reference behaviour (solution/ops.py:669-696, _run_packed_sdpa): per packed row, causal scaled
// dot-product attention with softmax scale 1/sqrt(head_dim) and K/V shared by h_q / h_kv query
// heads; its backward is torch's. Layout here: q [N, h_q, 128], k / v [N, h_kv, 128] token-major
// (the RoPE kernel's outputs), rows delimited by cu_seqlens [n_seq + 1] (int32, on the device).
//
// Design (CDNA4, v_mfma_f32_32x32x16_f16; operand / accumulator lane layouts as in mfma_gemm.h):
//   * one block of 4 waves per (row, 32-token block, query head); the waves split the loop over
//     the other operand's 32-token blocks and merge their partials through LDS at the end in a
//     fixed order (softmax partials rescaled by their running maxima);
//   * every operand tile (32 tokens x 128 dims) is copied straight into LDS by
//     global_load_lds_dwordx4 (whole 256-byte rows per 16 lanes; the block's own query tile
//     once, the waves' key / value tiles per loop step) and read from there as 16-byte row
//     fragments or, through ds_read_b64_tr_b16, as transposed fragments: no tile is held in
//     registers in flight, no transposed copy is written, and blocks fit two per CU;
//   * forward computes S^T = K Q^T, so a lane owns one query (column) and 16 of the block's 32
//     keys: the running max / sum and the O rescale are per-lane scalars, and P^T feeds the
//     O^T += V^T P^T product straight from the accumulator registers. An accumulator tile used
//     as an MFMA operand carries its reduction index in the order
//         k(h, i) = 16 s + 8 (i / 4) + 4 h + i % 4      (lane half h, slot i of step s),
//     which the transposed reads produce (two reads of 4 consecutive tokens per fragment);
//   * P and dS are rounded to fp16 for their MFMAs, as flash attention does; O, LSE, dQ, dK, dV
//     accumulate in fp32;
//   * backward: one launch runs the dK / dV blocks (row, key block, query head; fp32 dK / dV
//     partials per query head) and the dQ blocks (row, query block, head); each block forms
//     D = rowsum(dO o O) of the query rows it visits from the dO tile in LDS and O rows loaded
//     with that tile (no separate launch, no D array). The h_q / h_kv partials of a KV group are summed in head order
//     and rounded once, either by the last of the group's blocks to finish a key block (arrival
//     counter; no atomics on data) or, in the engine's path, by the RoPE backward that packs
//     them (rus_qkv_rope_bwd_mid_parts).
#include <math.h>

#include "common.h"

namespace rus {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kHD = 128;       // head_dim
constexpr int kBlk = 32;       // tokens per block
constexpr int kW = 4;          // waves per block (one 32x32 head-dim tile each in the merges)
constexpr int kMaxGroup = 8;   // query heads per KV head (GQA group) the backward supports
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazy = 8.0f;  // lazy-rescale threshold (log2 units)

struct AttnArgs {
  const f16* q;
  const f16* k;
  const f16* v;
  const f16* o;    // forward output (backward input)
  const f16* dout;
  const int32_t* cu;
  f16* out;        // forward: O; backward kernel 1: dQ
  float* lse;      // [h_q, n_tok], natural log
  float* dk_part;  // [h_q, n_tok, 128]
  float* dv_part;
  f16* dk;         // [n_tok, h_kv, 128]
  f16* dv;
  int* counters;   // [max_blocks, h_kv] arrival counters (zero on entry, left zero)
  int64_t n_tok;
  int n_seq, h_q, h_kv;
  int max_blocks;  // backward: blocks per pass (grid y of each pass)
  int group_sum;   // backward: 1 = sum each KV group's dK / dV partials into dk / dv
  float scale, scale_log2;
};

// 2^x by the hardware instruction (v_exp_f32): 2^-inf = 0; results below the normal range
// flush to zero, far below what the fp16 operands they feed can hold.
__device__ __forceinline__ float exp2_raw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Row bounds of row s (clamped to [0, n_tok] and non-decreasing, so a malformed cu_seqlens
// cannot send an access outside the token arrays) and its number of 32-token blocks.
struct RowInfo {
  int a, e, nb;
};

__device__ __forceinline__ RowInfo row_info(const int32_t* cu, int s, int n_seq, int n_tok) {
  RowInfo r{0, 0, 0};
  if (s < n_seq) {
    r.a = min(max(cu[s], 0), n_tok);
    r.e = min(max(cu[s + 1], r.a), n_tok);
    r.nb = (r.e - r.a + kBlk - 1) / kBlk;
  }
  return r;
}

// Index of the n-th set bit of m (n < popcount(m)).
__device__ __forceinline__ int nth_bit(uint64_t m, int n) {
  for (int i = 0; i < n; ++i) m &= m - 1;
  return __ffsll(static_cast<unsigned long long>(m)) - 1;
}

// Block id -> (row start, row end, block start), heaviest blocks first. A row of nb blocks has
// one block of each work level w = 1 .. nb (the number of 32-token blocks on the other side of
// the causal loop): block w - 1 when the work grows towards the row's end (kDiagLast: forward
// and dQ, which loop over the keys up to the diagonal), block nb - w otherwise (dK/dV, which loop
// over the queries from the diagonal on). Ids run over levels from the highest down, rows in
// order within a level, so the longest blocks are dispatched first. Each lane holds one row of
// a 64-row chunk; false if blk is past the last block. Uniform over the block.
template <bool kDiagLast>
__device__ __forceinline__ bool find_block(const int32_t* cu, int n_seq, int n_tok, int blk,
                                           int& start, int& end, int& b0) {
  const int lane = threadIdx.x & 63;
  const int n_chunks = (n_seq + 63) / 64;
  const RowInfo r0 = row_info(cu, lane, n_seq, n_tok);
  int max_nb = r0.nb;
  for (int c = 1; c < n_chunks; ++c) max_nb = max(max_nb, row_info(cu, 64 * c + lane, n_seq, n_tok).nb);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) max_nb = max(max_nb, __shfl_xor(max_nb, off, 64));
  for (int w = max_nb; w >= 1; --w) {
    for (int c = 0; c < n_chunks; ++c) {
      const RowInfo r = c == 0 ? r0 : row_info(cu, 64 * c + lane, n_seq, n_tok);
      const uint64_t mask = __ballot(r.nb >= w);
      const int cnt = __popcll(mask);
      if (blk < cnt) {
        const int src = nth_bit(mask, blk);
        start = __shfl(r.a, src, 64);
        end = __shfl(r.e, src, 64);
        const int nb = __shfl(r.nb, src, 64);
        b0 = start + (kDiagLast ? w - 1 : nb - w) * kBlk;
        return true;
      }
      blk -= cnt;
    }
  }
  return false;
}

// fp16 operand of k-step s from accumulator registers 8s .. 8s+7.
__device__ __forceinline__ f16x8 frag_acc(const f32x16& c, int s) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = from_f32<f16>(c[8 * s + i]);
  return r;
}

// Accumulator row of register r for lane half h.
__device__ __forceinline__ int acc_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// Partial accumulators of the block's kW waves, summed in a fixed order: every wave stores its
// four 32x32 tiles (the accumulator layout, lane-contiguous), then thread (wave w, lane) reads
// tile w of every wave. buf holds kW * 64 * 64 floats.
__device__ __forceinline__ void park(float* buf, const f32x16 (&acc)[4], int wave, int lane) {
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) buf[(wave * 64 + d * 16 + r) * 64 + lane] = acc[d][r];
}

__device__ __forceinline__ float parked(const float* buf, int w, int tile, int r, int lane) {
  return buf[(w * 64 + tile * 16 + r) * 64 + lane];
}

// fp16 store of the 16 accumulator values of tile d (head dims d*32 + 8 r4 + 4 h + i) of one
// query's row.
__device__ __forceinline__ void store_tile_row(f16* row, const float (&x)[16], int d, int h) {
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) {
    f16x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = from_f32<f16>(x[4 * r4 + i]);
    *reinterpret_cast<f16x4*>(row + d * 32 + 8 * r4 + 4 * h) = w;
  }
}

constexpr int kParkBytes = kW * 64 * 64 * 4;             // 64 KiB
constexpr int kMax(int x, int y) { return x > y ? x : y; }

// ---------------------------------------------------------------------------------------------
// Operand tiles (32 tokens x 128 head dims of Q, dO, K or V) are copied straight from global
// memory into LDS (global_load_lds_dwordx4: 4 rows x 256 contiguous bytes per wave instruction,
// no registers in flight) and read from there both ways: 16-byte row fragments (ds_read_b128)
// and transposed fragments (ds_read_b64_tr_b16), so each tile is loaded once per use.
// ---------------------------------------------------------------------------------------------
constexpr int kTile = kBlk * kHD * 2;  // one 32 x 128 fp16 tile: 8 KiB
typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// Tiles are row-major, 256 bytes per token row, with the 16-byte chunk c of row r stored at chunk
// c ^ swz(r): a quarter wave's 16-byte fragment reads (16 consecutive rows, one chunk) and a
// half wave's transposing reads (4 consecutive rows x 64 bytes) each cover the 64 banks once.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Issues copies i0 .. i0 + n - 1 of the 8 that fill a tile with token rows r0 .. r0 + 31 of a
// [*, stride] head slice (rows clamped into [lo, hi): rows past a row's end repeat its last token,
// finite values that the masks discard). Copy i fills tile rows 4 i .. 4 i + 3; lane l lands at
// row 4 i + l / 16, position l % 16, so it loads the chunk (l % 16) ^ swz(row).
__device__ __forceinline__ void tile_copy(char* tile, const f16* x, int64_t stride, int r0,
                                          int lo, int hi, int i0, int n) {
  const int lane = threadIdx.x & 63;
  for (int i = i0; i < i0 + n; ++i) {
    const int r = 4 * i + (lane >> 4);
    int t = r0 + r;
    t = t < hi ? t : hi - 1;
    t = t < lo ? lo : t;
    const int c = (lane & 15) ^ swz(r);
    __builtin_amdgcn_global_load_lds(x + static_cast<int64_t>(t) * stride + c * 8,
                                     (lds_void_ptr)(tile + i * 1024), 16, 0, 0);
  }
}

// s_waitcnt vmcnt(0): this wave's tile copies have landed (expcnt / lgkmcnt not waited on).
__device__ __forceinline__ void wait_copies() {
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

// This wave's LDS reads have returned: a copy may now overwrite the tiles they read.
__device__ __forceinline__ void wait_tile_reads() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt / expcnt not waited on
  asm volatile("" ::: "memory");
}

// 16-byte fragment: head dims 8 c .. 8 c + 7 of tile row r.
__device__ __forceinline__ f16x8 tile_frag(const char* tile, int r, int c) {
  return *reinterpret_cast<const f16x8*>(tile + r * 256 + ((c ^ swz(r)) << 4));
}

// Transposed fragment of k-step s in the accumulator order k(h, i) = 16 s + 8 (i / 4) + 4 h +
// i % 4, head-dim tile d: lane l holds x[k(h, i)][32 d + l % 32], i = 0..7. ds_read_b64_tr_b16
// gives lane i of each 16-lane group element i % 4 of the 8 bytes read by lanes i / 4 + 4 e of
// the group, so lane j of a group reads row k0 + j / 4, head dims n0 + 4 (j % 4) .. +4, and lane i
// receives x[k0 + e][n0 + i], e = 0..3 (k0 = 16 s + 4 h, then + 8).
__device__ __forceinline__ f16x8 tile_frag_t(const char* tile, int s, int d) {
  const int lane = threadIdx.x & 63, j = lane & 15;
  const int col = 32 * d + (lane & 16) + 4 * (j & 3);
  const int r0 = 16 * s + 4 * (lane >> 5) + (j >> 2), r1 = r0 + 8;
  const int cb = (col & 7) * 2;
  const v4i16 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(tile + r0 * 256 + (((col >> 3) ^ swz(r0)) << 4) + cb));
  const v4i16 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16*)(tile + r1 * 256 + (((col >> 3) ^ swz(r1)) << 4) + cb));
  const f16x4 a = __builtin_bit_cast(f16x4, x0), b = __builtin_bit_cast(f16x4, x1);
  return f16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}


// ---------------------------------------------------------------------------------------------
// Forward: O = softmax(Q K^T * scale, causal) V and LSE. Block = (row, query block, head); its
// kW waves take key blocks w, w + kW, ... with their own running max / sum, merged at the end.
// ---------------------------------------------------------------------------------------------
// At most 256 registers per lane (no spills) and 72 KiB of LDS (the block's Q tile, each wave's
// K and V tiles): two blocks share a CU, so the grid of (query block, head) blocks fits the chip
// in one round and one block's loads overlap another's MFMAs.
__global__ __launch_bounds__(64 * kW) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_fwd_kernel(AttnArgs a) {
  constexpr int kBytes = kMax((1 + 2 * kW) * kTile, kParkBytes + kW * 64 * 4);
  __shared__ __attribute__((aligned(16))) char smem[kBytes];
  int start, end, q0;
  if (!find_block<true>(a.cu, a.n_seq, static_cast<int>(a.n_tok), blockIdx.y, start, end, q0)) return;
  const int head = blockIdx.x, g = head / (a.h_q / a.h_kv);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const int64_t sq = static_cast<int64_t>(a.h_q) * kHD, skv = static_cast<int64_t>(a.h_kv) * kHD;
  const f16* kh = a.k + g * kHD;
  const f16* vh = a.v + g * kHD;
  char* qt = smem;
  char* kt = smem + (1 + 2 * wave) * kTile;
  char* vt = kt + kTile;

  const int qi = q0 + col;  // this lane's query
  const int nk = (q0 - start) / kBlk + 1;  // key blocks up to and including the diagonal
  tile_copy(qt, a.q + head * kHD, sq, q0, start, end, 2 * wave, 2);  // the 8 copies, 2 per wave
  if (wave < nk) {
    const int k0 = start + wave * kBlk;
    tile_copy(kt, kh, skv, k0, start, end, 0, 8);
    tile_copy(vt, vh, skv, k0, start, end, 0, 8);
  }
  wait_copies();
  __syncthreads();  // every wave's share of the Q tile has landed
  f16x8 qf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) qf[s] = tile_frag(qt, col, 2 * s + h);
  f32x16 o[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) o[d] = f32x16{};
  float m = -INFINITY, l = 0.0f;
  for (int kb = wave; kb < nk; kb += kW) {
    const int k0 = start + kb * kBlk;
    f32x16 st = f32x16{};  // S^T = K Q^T: rows keys, columns queries
#pragma unroll
    for (int s = 0; s < 8; ++s) st = mfma(tile_frag(kt, col, 2 * s + h), qf[s], st);
    // Only the diagonal block holds keys past the query or past the row's end.
    float mx = -INFINITY;
    if (kb == nk - 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + acc_row(r, h);
        st[r] = (key <= qi && key < end) ? st[r] * a.scale_log2 : -INFINITY;
        mx = fmaxf(mx, st[r]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        st[r] *= a.scale_log2;
        mx = fmaxf(mx, st[r]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // finite: key k0 <= q0 <= qi is always allowed
    // Lazy rescaling: the reference point m moves only when a block's maximum exceeds it by
    // more than 8 (log2 units), so p = 2^(s - m) <= 256 (exact in range for fp16) and O and l
    // share one reference, leaving O / l unchanged; the rescale of O is a wave-uniform branch
    // that is rarely taken after the first block.
    const bool bump = mx > m + kLazy;
    if (__ballot(bump)) {
      const float mn = bump ? mx : m;
      const float alpha = exp2_raw(m - mn);  // 0 on the first block (m = -inf)
      l *= alpha;
      m = mn;
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
    }
    float rs = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = exp2_raw(st[r] - m);
      st[r] = p;
      rs += p;
    }
    rs += __shfl_xor(rs, 32, 64);
    l += rs;
    const f16x8 p0 = frag_acc(st, 0), p1 = frag_acc(st, 1);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      o[d] = mfma(tile_frag_t(vt, 0, d), p0, o[d]);  // O^T += V^T P^T
      o[d] = mfma(tile_frag_t(vt, 1, d), p1, o[d]);
    }
    if (kb + kW < nk) {  // the wave's next key block into its tiles
      wait_tile_reads();
      const int k1 = k0 + kW * kBlk;
      tile_copy(kt, kh, skv, k1, start, end, 0, 8);
      tile_copy(vt, vh, skv, k1, start, end, 0, 8);
      wait_copies();
    }
  }
  __syncthreads();  // all waves are done with their V^T tiles; the space is reused below
  float* buf = reinterpret_cast<float*>(smem);
  float* ml = buf + kW * 64 * 64;  // per wave: m of columns 0..31, then l
  park(buf, o, wave, lane);
  if (h == 0) {
    ml[wave * 64 + col] = m;
    ml[wave * 64 + 32 + col] = l;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kW; ++w) M = fmaxf(M, ml[w * 64 + col]);
  float f[kW], L = 0.0f;
#pragma unroll
  for (int w = 0; w < kW; ++w) {
    const float mw = ml[w * 64 + col];
    f[w] = exp2_raw(mw - M);  // 0 for a wave without key blocks (mw = -inf)
    L += ml[w * 64 + 32 + col] * f[w];
  }
  if (qi < end) {
    const float inv = 1.0f / L;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < kW; ++w) acc += parked(buf, w, wave, r, lane) * f[w];
      x[r] = acc * inv;
    }
    store_tile_row(a.out + qi * sq + head * kHD, x, wave, h);
    if (wave == 0 && h == 0) a.lse[head * a.n_tok + qi] = (M + log2f(L)) * kLn2;
  }
}

// ---------------------------------------------------------------------------------------------
// Backward, on the LDS tiles: row fragments for S = Q K^T and dP = dO V^T, transposed fragments
// for dV += P^T dO, dK += dS^T Q and dQ^T += K^T dS^T. D = rowsum(dO o O) is formed once per
// (head, query) by a small kernel before the main launch.
// ---------------------------------------------------------------------------------------------
// Waves per backward block: 4 (80 KiB of LDS and at most 256 registers, so two blocks share a
// CU and one block's waits overlap the other's work; 8 waves in one block per CU ran 13% slower).
constexpr int kWB = 4;
static_assert(kWB == 4 || kWB == 8, "4 or 8 waves per backward block");
constexpr int kCopiesPerWave = 8 / kWB;  // a shared tile's 8 copies over the block's waves
constexpr int kRegsPerWave = 64 / kWB;   // accumulator registers each wave sums in the merge
// LDS of a backward block: 2 shared tiles + 2 per wave; the merge reuses it as a buffer of every
// wave's four 32x32 fp32 accumulator tiles.
constexpr int kBwdBytes = (2 + 2 * kWB) * kTile;
static_assert(kWB * 64 * 64 * 4 <= kBwdBytes, "the merge buffer fits the tiles' LDS");

// Every wave's four 32x32 fp32 tiles into the merge buffer (the accumulator layout,
// lane-contiguous); thread (wave w, lane) then sums tile w % 4, registers kRegsPerWave (w / 4)
// .. + kRegsPerWave, over the waves in wave order.
__device__ __forceinline__ void park_b(float* buf, const f32x16 (&acc)[4], int wave, int lane) {
#pragma unroll
  for (int d = 0; d < 4; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) buf[(wave * 64 + d * 16 + r) * 64 + lane] = acc[d][r];
}

__device__ __forceinline__ void merge_b(const float* buf, int wave, int lane,
                                        float (&x)[kRegsPerWave]) {
  const int tile = wave & 3, r0 = kRegsPerWave * (wave >> 2);
#pragma unroll
  for (int r = 0; r < kRegsPerWave; ++r) {
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < kWB; ++w) acc += buf[(w * 64 + tile * 16 + r0 + r) * 64 + lane];
    x[r] = acc;
  }
}

// D = rowsum(dO o O) of the 32 query rows of a block, formed where it is used: the dO tile is in
// LDS and the O rows come in registers (ORows, loaded with the tiles). Pass p covers rows 4 p ..
// 4 p + 3: lane l takes row 4 p + l / 16, head dims 8 (l % 16) .. + 8, sums their 8 fp32 products
// of fp16 values in dim order, then the 16 lanes of a row add by a butterfly (xor 8, 4, 2, 1);
// every lane of the group then holds the row's D. Rows past the row's end repeat its last token
// (as the tiles do), so they hold that token's D.
struct ORows {
  f16x8 v[8];
};

__device__ __forceinline__ void load_o_rows(ORows& o, const f16* oh, int64_t stride, int r0,
                                            int lo, int hi) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    int t = r0 + 4 * p + (lane >> 4);
    t = t < hi ? t : hi - 1;
    t = t < lo ? lo : t;
    o.v[p] = *reinterpret_cast<const f16x8*>(oh + static_cast<int64_t>(t) * stride +
                                             8 * (lane & 15));
  }
}

// x of the lane N places further round its 16-lane row (DPP row_ror: a VALU move, no LDS).
template <int N>
__device__ __forceinline__ float row_ror(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               0x120 + N, 0xF, 0xF, false));
}

// The butterfly adds lane c's sum to lane c ^ 8's, then c ^ 4's, c ^ 2's, c ^ 1's. After the
// step with 8 a lane's sum depends on c mod 8 only, so the lane c + 4 (mod 16) holds what c ^ 4
// holds; likewise for 2 and 1: rotations give the same sums as the xor exchanges.
__device__ __forceinline__ float row_dsum(const ORows& o, const char* dt, int p) {
  const int lane = threadIdx.x & 63;
  const f16x8 y = tile_frag(dt, 4 * p + (lane >> 4), lane & 15);
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc += static_cast<float>(o.v[p][e]) * static_cast<float>(y[e]);
  acc += row_ror<8>(acc);
  acc += row_ror<4>(acc);
  acc += row_ror<2>(acc);
  acc += row_ror<1>(acc);
  return acc;
}

// D of the rows this lane's accumulator registers cover (register r: row acc_row(r, h)).
__device__ __forceinline__ void dsum_acc_rows(const ORows& o, const char* dt, int h,
                                              float (&d)[16]) {
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const float s = row_dsum(o, dt, p);
    // rows 4 p + g sit in lanes 16 g .. 16 g + 15; acc_row(4 j + g, h) = 4 (2 j + h) + g, so
    // the lanes of half h = p % 2 take them as registers 4 (p / 2) + g
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float v = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), 16 * g));
      if ((p & 1) == h) d[4 * (p >> 1) + g] = v;
    }
  }
}

// D of tile row c (this lane's query column in the dQ blocks).
__device__ __forceinline__ float dsum_row(const ORows& o, const char* dt, int c) {
  float d = 0.0f;
#pragma unroll
  for (int p = 0; p < 8; ++p) {
    const float s = __shfl(row_dsum(o, dt, p), 16 * (c & 3), 64);
    if ((c >> 2) == p) d = s;
  }
  return d;
}

// dQ = scale * dS K. Block = (row, query block, head): the Q and dO tiles of its 32 queries are
// shared; the kWB waves take key blocks w, w + kWB, ... (K and V tiles of their own) and their
// dQ partials are summed in wave order at the end.
__device__ __forceinline__ void attn_bwd_dq_block(const AttnArgs& a, int blk, char* smem) {
  int start, end, q0;
  if (!find_block<true>(a.cu, a.n_seq, static_cast<int>(a.n_tok), blk, start, end, q0)) return;
  const int head = blockIdx.x, g = head / (a.h_q / a.h_kv);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const int64_t sq = static_cast<int64_t>(a.h_q) * kHD, skv = static_cast<int64_t>(a.h_kv) * kHD;
  const f16* kh = a.k + g * kHD;
  const f16* vh = a.v + g * kHD;
  char* qt = smem;
  char* dt = smem + kTile;
  char* kt = smem + (2 + 2 * wave) * kTile;
  char* vt = kt + kTile;
  const int nk = (q0 - start) / kBlk + 1;
  tile_copy(qt, a.q + head * kHD, sq, q0, start, end, kCopiesPerWave * wave, kCopiesPerWave);
  tile_copy(dt, a.dout + head * kHD, sq, q0, start, end, kCopiesPerWave * wave, kCopiesPerWave);
  if (wave < nk) {
    const int k0 = start + wave * kBlk;
    tile_copy(kt, kh, skv, k0, start, end, 0, 8);
    tile_copy(vt, vh, skv, k0, start, end, 0, 8);
  }
  ORows orow;
  load_o_rows(orow, a.o + head * kHD, sq, q0, start, end);
  const int qi = q0 + col, qr = qi < end ? qi : end - 1;
  const float lse2 = a.lse[head * a.n_tok + qr] * kLog2e;
  wait_copies();
  __syncthreads();  // every wave's share of the Q and dO tiles has landed
  const float dsum = dsum_row(orow, dt, col);  // D of this lane's query (tile row col)

  f32x16 dq[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) dq[d] = f32x16{};
  for (int kb = wave; kb < nk; kb += kWB) {
    const int k0 = start + kb * kBlk;
    f32x16 st = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      st = mfma(tile_frag(kt, col, 2 * s + h), tile_frag(qt, col, 2 * s + h), st);  // S^T = K Q^T
      dp = mfma(tile_frag(vt, col, 2 * s + h), tile_frag(dt, col, 2 * s + h), dp);  // dP^T = V dO^T
    }
    if (kb == nk - 1) {  // diagonal block: causal and row-end mask
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + acc_row(r, h);
        const float p = exp2_raw(st[r] * a.scale_log2 - lse2);
        st[r] = (key <= qi && key < end) ? p * (dp[r] - dsum) : 0.0f;  // dS^T
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) st[r] = exp2_raw(st[r] * a.scale_log2 - lse2) * (dp[r] - dsum);
    }
    const f16x8 s0 = frag_acc(st, 0), s1 = frag_acc(st, 1);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      dq[d] = mfma(tile_frag_t(kt, 0, d), s0, dq[d]);  // dQ^T += K^T dS^T
      dq[d] = mfma(tile_frag_t(kt, 1, d), s1, dq[d]);
    }
    if (kb + kWB < nk) {  // the wave's next key block into its tiles
      wait_tile_reads();
      const int k1 = k0 + kWB * kBlk;
      tile_copy(kt, kh, skv, k1, start, end, 0, 8);
      tile_copy(vt, vh, skv, k1, start, end, 0, 8);
      wait_copies();
    }
  }
  __syncthreads();  // every wave is done with the tiles; the space becomes the merge buffer
  float* buf = reinterpret_cast<float*>(smem);
  park_b(buf, dq, wave, lane);
  __syncthreads();
  if (qi < end) {
    float x[kRegsPerWave];
    merge_b(buf, wave, lane, x);
    // Register 4 r4 + i of tile d holds head dim 32 d + 8 r4 + 4 h + i.
    const int d = wave & 3, r4b = (kRegsPerWave / 4) * (wave >> 2);
    f16* row = a.out + qi * sq + head * kHD;
#pragma unroll
    for (int r4 = 0; r4 < kRegsPerWave / 4; ++r4) {
      f16x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = from_f32<f16>(x[4 * r4 + i] * a.scale);
      *reinterpret_cast<f16x4*>(row + d * 32 + 8 * (r4b + r4) + 4 * h) = w;
    }
  }
}

// This query head's dK = scale * dS^T Q and dV = P^T dO for one 32-key block, fp32. Block = (row,
// key block, head): the K and V tiles are shared; the kWB waves take query blocks (Q and dO tiles
// of their own). The h_q / h_kv heads of a KV group store fp32 partials; the last of them to
// finish sums the group in head order and writes dK and dV once (no atomics on data, no separate
// reduce launch).
__device__ __forceinline__ void attn_bwd_dkdv_block(const AttnArgs& a, int blk, char* smem) {
  int start, end, k0;
  if (!find_block<false>(a.cu, a.n_seq, static_cast<int>(a.n_tok), blk, start, end, k0)) return;
  const int head = blockIdx.x, g = head / (a.h_q / a.h_kv);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, col = lane & 31;
  const int64_t sq = static_cast<int64_t>(a.h_q) * kHD, skv = static_cast<int64_t>(a.h_kv) * kHD;
  const f16* qh = a.q + head * kHD;
  const f16* doh = a.dout + head * kHD;
  const float* lse = a.lse + head * a.n_tok;
  const f16* oh = a.o + head * kHD;
  char* kt = smem;
  char* vt = smem + kTile;
  char* qt = smem + (2 + 2 * wave) * kTile;
  char* dt = qt + kTile;
  const int nq = (end - k0 + kBlk - 1) / kBlk;  // query blocks from the diagonal to the row end
  tile_copy(kt, a.k + g * kHD, skv, k0, start, end, kCopiesPerWave * wave, kCopiesPerWave);
  tile_copy(vt, a.v + g * kHD, skv, k0, start, end, kCopiesPerWave * wave, kCopiesPerWave);
  ORows orow;  // the O rows of the wave's next query block, loaded with its tiles
  if (wave < nq) {
    const int q0 = k0 + wave * kBlk;
    tile_copy(qt, qh, sq, q0, start, end, 0, 8);
    tile_copy(dt, doh, sq, q0, start, end, 0, 8);
    load_o_rows(orow, oh, sq, q0, start, end);
  }
  const int kj = k0 + col;  // this lane's key (column of S = Q K^T)
  wait_copies();
  __syncthreads();  // every wave's share of the K and V tiles has landed
  // D of the query rows of this lane's registers, for the wave's current query block; formed
  // once its dO tile and O rows have landed, so the O rows are not held across the products
  float dsum[16] = {};
  if (wave < nq) dsum_acc_rows(orow, dt, h, dsum);

  f32x16 dk[4], dv[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    dk[d] = f32x16{};
    dv[d] = f32x16{};
  }
  for (int qb = wave; qb < nq; qb += kWB) {
    const int q0 = k0 + qb * kBlk;
    f32x16 st = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      st = mfma(tile_frag(qt, col, 2 * s + h), tile_frag(kt, col, 2 * s + h), st);  // S = Q K^T
      dp = mfma(tile_frag(dt, col, 2 * s + h), tile_frag(vt, col, 2 * s + h), dp);  // dP = dO V^T
    }
    // Query rows past the row's end (last block) and before the key (diagonal block) are
    // masked; key columns past the row's end only feed dK / dV rows that are not written.
    const bool edge = q0 == k0 || q0 + kBlk > end;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = q0 + acc_row(r, h);
      const int qc = qi < end ? qi : end - 1;
      float p = exp2_raw(st[r] * a.scale_log2 - lse[qc] * kLog2e);
      if (edge) p = (kj <= qi && qi < end) ? p : 0.0f;
      st[r] = p;                         // P
      dp[r] = p * (dp[r] - dsum[r]);     // dS
    }
    const f16x8 p0 = frag_acc(st, 0), p1 = frag_acc(st, 1);
    const f16x8 s0 = frag_acc(dp, 0), s1 = frag_acc(dp, 1);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      dv[d] = mfma(p0, tile_frag_t(dt, 0, d), dv[d]);  // dV += P^T dO
      dv[d] = mfma(p1, tile_frag_t(dt, 1, d), dv[d]);
      dk[d] = mfma(s0, tile_frag_t(qt, 0, d), dk[d]);  // dK += dS^T Q
      dk[d] = mfma(s1, tile_frag_t(qt, 1, d), dk[d]);
    }
    if (qb + kWB < nq) {  // the wave's next query block into its tiles
      wait_tile_reads();
      const int q1 = q0 + kWB * kBlk;
      tile_copy(qt, qh, sq, q1, start, end, 0, 8);
      tile_copy(dt, doh, sq, q1, start, end, 0, 8);
      load_o_rows(orow, oh, sq, q1, start, end);
      wait_copies();
      dsum_acc_rows(orow, dt, h, dsum);
    }
  }
  // Sum the waves' partials (dK, then dV through the same buffer) and store this head's fp32
  // partial. Rows are keys (accumulator rows), columns head dims (lanes); thread (wave w, lane)
  // writes head-dim tile w % 4, key rows of registers kRegsPerWave (w / 4) .. + kRegsPerWave.
  float* buf = reinterpret_cast<float*>(smem);
  const int dt4 = wave & 3, rb = kRegsPerWave * (wave >> 2);
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    __syncthreads();
    park_b(buf, pass == 0 ? dk : dv, wave, lane);
    __syncthreads();
    float x[kRegsPerWave];
    merge_b(buf, wave, lane, x);
    float* dst = pass == 0 ? a.dk_part : a.dv_part;
    const float sc = pass == 0 ? a.scale : 1.0f;
#pragma unroll
    for (int r = 0; r < kRegsPerWave; ++r) {
      const int key = k0 + acc_row(rb + r, h);
      if (key < end)
        store_partial(dst + (static_cast<int64_t>(head) * a.n_tok + key) * kHD + dt4 * 32 + col,
                      x[r] * sc);
    }
  }
  if (!a.group_sum) return;  // the partials are the output (summed by the RoPE backward)
  const int grp = a.h_q / a.h_kv;
  // The verdict goes through the first word of the merge buffer, which every thread is done
  // reading once arrive_last_at's first barrier has passed.
  if (!arrive_last_at(a.counters + static_cast<int64_t>(blk) * a.h_kv + g, grp,
                      reinterpret_cast<int*>(smem)))
    return;
  // Last head of the group: dk[key, g, :] = fp16(sum over the group's heads in head order).
  // Thread (wave, lane) owns head dims (wave % 4) * 32 + col of its keys, as in the stores.
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const float* src = pass == 0 ? a.dk_part : a.dv_part;
    f16* out = pass == 0 ? a.dk : a.dv;
    // Every head's loads are issued together (the partials are read device-coherently, from
    // beyond this XCD's L2: one latency instead of one per head), then added in head order;
    // slots past the group re-read its last head and are not added.
    float v[kMaxGroup][kRegsPerWave];
#pragma unroll
    for (int j = 0; j < kMaxGroup; ++j) {
      const int jj = min(j, grp - 1);
      const float* hsrc =
          src + static_cast<int64_t>(g * grp + jj) * a.n_tok * kHD + dt4 * 32 + col;
#pragma unroll
      for (int r = 0; r < kRegsPerWave; ++r) {
        const int key = min(k0 + acc_row(rb + r, h), end - 1);  // past the end: read, not stored
        v[j][r] = load_partial(hsrc + static_cast<int64_t>(key) * kHD);
      }
    }
#pragma unroll
    for (int r = 0; r < kRegsPerWave; ++r) {
      float acc = v[0][r];
#pragma unroll
      for (int j = 1; j < kMaxGroup; ++j)
        if (j < grp) acc += v[j][r];
      const int key = k0 + acc_row(rb + r, h);
      if (key < end)
        out[(static_cast<int64_t>(key) * a.h_kv + g) * kHD + dt4 * 32 + col] = from_f32<f16>(acc);
    }
  }
}

// Both backward passes in one launch: blocks y < max_blocks are dK/dV blocks (the heavier ones,
// dispatched first), the rest dQ blocks.
__global__ __launch_bounds__(64 * kWB) __attribute__((amdgpu_waves_per_eu(2, 2))) void
attn_bwd_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) char smem[kBwdBytes];
  if (static_cast<int>(blockIdx.y) < a.max_blocks)
    attn_bwd_dkdv_block(a, blockIdx.y, smem);
  else
    attn_bwd_dq_block(a, blockIdx.y - a.max_blocks, smem);
}

int check(const char* fn, const void* q, const void* k, const void* v, const int32_t* cu,
          int64_t n_tok, int32_t n_seq, int32_t h_q, int32_t h_kv, int32_t head_dim,
          int32_t max_blocks) {
  if (!q || !k || !v || !cu) return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (head_dim != kHD) return fail(RUS_ERR_UNSUPPORTED, "%s: head_dim %d (only 128)", fn, head_dim);
  if (h_q <= 0 || h_kv <= 0 || h_q % h_kv)
    return fail(RUS_ERR_INVALID, "%s: h_q=%d must be a multiple of h_kv=%d", fn, h_q, h_kv);
  if (n_tok <= 0 || n_tok >= (int64_t(1) << 31) || n_seq <= 0 || max_blocks <= 0 ||
      max_blocks > 65535)
    return fail(RUS_ERR_INVALID, "%s: n_tok=%lld n_seq=%d max_blocks=%d", fn, (long long)n_tok,
                n_seq, max_blocks);
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16))
    return fail(RUS_ERR_INVALID, "%s: q/k/v must be 16-byte aligned", fn);
  return RUS_OK;
}

}  // namespace
}  // namespace rus

using rus::f16;

extern "C" int rus_attn_varlen_fwd(const void* q, const void* k, const void* v,
                                   const int32_t* cu_seqlens, int32_t n_seq, int64_t n_tokens,
                                   int32_t max_blocks, int32_t h_q, int32_t h_kv,
                                   int32_t head_dim, float scale, void* out, float* lse,
                                   void* stream) {
  using namespace rus;
  const char* fn = "rus_attn_varlen_fwd";
  if (int e = check(fn, q, k, v, cu_seqlens, n_tokens, n_seq, h_q, h_kv, head_dim, max_blocks))
    return e;
  if (!out || !lse || !aligned(out, 16)) return fail(RUS_ERR_INVALID, "%s: bad output", fn);
  AttnArgs a{};
  a.q = static_cast<const f16*>(q);
  a.k = static_cast<const f16*>(k);
  a.v = static_cast<const f16*>(v);
  a.cu = cu_seqlens;
  a.out = static_cast<f16*>(out);
  a.lse = lse;
  a.n_tok = n_tokens;
  a.n_seq = n_seq;
  a.h_q = h_q;
  a.h_kv = h_kv;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(h_q, max_blocks), dim3(64 * kW), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch(fn);
}

static int attn_bwd(const char* fn, const void* q, const void* k, const void* v,
                    const void* out, const void* dout, const float* lse,
                    const int32_t* cu_seqlens, int32_t n_seq, int64_t n_tokens,
                    int32_t max_blocks, int32_t h_q, int32_t h_kv, int32_t head_dim, float scale,
                    void* dq, void* dk, void* dv, float* workspace, int32_t* counters,
                    int64_t n_counters, bool group_sum, void* stream) {
  using namespace rus;
  if (int e = check(fn, q, k, v, cu_seqlens, n_tokens, n_seq, h_q, h_kv, head_dim, max_blocks))
    return e;
  if (!out || !dout || !lse || !dq || !workspace || !aligned(out, 16) || !aligned(dout, 16) ||
      !aligned(dq, 16) || !aligned(workspace, 16))
    return fail(RUS_ERR_INVALID, "%s: null or misaligned argument", fn);
  if (group_sum) {
    if (!dk || !dv || !aligned(dk, 16) || !aligned(dv, 16) || !counters || !aligned(counters, 4))
      return fail(RUS_ERR_INVALID, "%s: null or misaligned argument", fn);
    if (h_q / h_kv > kMaxGroup)
      return fail(RUS_ERR_UNSUPPORTED, "%s: %d query heads per KV head (at most %d)", fn,
                  h_q / h_kv, kMaxGroup);
    if (n_counters < static_cast<int64_t>(max_blocks) * h_kv)
      return fail(RUS_ERR_INVALID, "%s: %lld counters, need max_blocks * h_kv = %lld", fn,
                  static_cast<long long>(n_counters),
                  static_cast<long long>(max_blocks) * h_kv);
  }
  AttnArgs a{};
  a.q = static_cast<const f16*>(q);
  a.k = static_cast<const f16*>(k);
  a.v = static_cast<const f16*>(v);
  a.o = static_cast<const f16*>(out);
  a.dout = static_cast<const f16*>(dout);
  a.cu = cu_seqlens;
  a.lse = const_cast<float*>(lse);
  a.n_tok = n_tokens;
  a.n_seq = n_seq;
  a.h_q = h_q;
  a.h_kv = h_kv;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  // workspace: dk_part [h_q, n_tok, 128] | dv_part (alike)
  if (2 * static_cast<int64_t>(max_blocks) > 65535)
    return fail(RUS_ERR_UNSUPPORTED, "%s: max_blocks=%d (at most 32767)", fn, max_blocks);
  a.dk_part = workspace;
  a.dv_part = a.dk_part + static_cast<int64_t>(h_q) * n_tokens * kHD;
  hipStream_t st = static_cast<hipStream_t>(stream);
  a.out = static_cast<f16*>(dq);
  a.dk = static_cast<f16*>(dk);
  a.dv = static_cast<f16*>(dv);
  a.counters = counters;
  a.max_blocks = max_blocks;
  a.group_sum = group_sum ? 1 : 0;
  hipLaunchKernelGGL(attn_bwd_kernel, dim3(h_q, 2 * max_blocks), dim3(64 * kWB), 0, st, a);
  return check_launch(fn);
}

extern "C" int rus_attn_varlen_bwd(const void* q, const void* k, const void* v, const void* out,
                                   const void* dout, const float* lse,
                                   const int32_t* cu_seqlens, int32_t n_seq, int64_t n_tokens,
                                   int32_t max_blocks, int32_t h_q, int32_t h_kv,
                                   int32_t head_dim, float scale, void* dq, void* dk, void* dv,
                                   float* workspace, int32_t* counters, int64_t n_counters,
                                   void* stream) {
  return attn_bwd("rus_attn_varlen_bwd", q, k, v, out, dout, lse, cu_seqlens, n_seq, n_tokens,
                  max_blocks, h_q, h_kv, head_dim, scale, dq, dk, dv, workspace, counters,
                  n_counters, true, stream);
}

extern "C" int rus_attn_varlen_bwd_parts(const void* q, const void* k, const void* v,
                                         const void* out, const void* dout, const float* lse,
                                         const int32_t* cu_seqlens, int32_t n_seq,
                                         int64_t n_tokens, int32_t max_blocks, int32_t h_q,
                                         int32_t h_kv, int32_t head_dim, float scale, void* dq,
                                         float* workspace, void* stream) {
  return attn_bwd("rus_attn_varlen_bwd_parts", q, k, v, out, dout, lse, cu_seqlens, n_seq,
                  n_tokens, max_blocks, h_q, h_kv, head_dim, scale, dq, nullptr, nullptr,
                  workspace, nullptr, 0, false, stream);
}
