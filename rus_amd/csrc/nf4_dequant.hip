// NF4 double-quant dequantisation for gfx950.
//
// Behaviour follows solution/kernels.py:27-118 (nf4_dequant_turing_kernel) and the launcher
// solution/kernels.py:572-619: one packed byte holds two NF4 codes (high nibble = even element),
// the per-block scale is code2[absmax[blk]] * absmax2[super] + segment offset, and the output is
// fp16 stored as fp16x2 words. Layout and design (CDNA4, wave64):
//   * one thread decodes one 4-byte unit of packed codes = 8 fp16 = one 16-byte store, so a wave
//     reads 256 contiguous bytes and writes 1 KiB contiguous per access (coalesced 128-bit stores);
//     UNROLL units per thread are loaded before any is decoded to keep several loads in flight;
//   * the NF4 codebook (16 floats) and the 256-entry code2 table live in LDS: the codebook index
//     differs per lane, and a 16-entry table hits 16 distinct banks (broadcast, conflict free),
//     which costs ~1 LDS read per element instead of a 15-select mux tree per element;
//   * the file is built with -ffp-contract=off so scale = (code2*absmax2) + off keeps two
//     roundings, matching an eager mul-then-add (bitsandbytes dequantize_blockwise + offset);
//   * the super-block (absmax2) index is taken relative to each segment's first block, so fused
//     segments whose block counts are not multiples of super_blocksize stay correct.
#include <type_traits>

#include "common.h"
#include "rmsnorm_rows.h"
#include "lora_rows.h"

namespace rus {
namespace {

// NF4 code points in nibble order (QLoRA normal-float-4 table; solution/kernels.py:76-83).
__constant__ float kNF4[16] = {
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

constexpr int kThreads = 256;
constexpr int kUnrollTab = 4;  // 4-byte units per thread on the table path

struct Nf4Args {
  const uint32_t* packed;  // packed codes viewed as 32-bit units
  const uint8_t* packed_bytes;
  const uint8_t* absmax;
  const float* code2;
  const float* absmax2;
  uint32_t* out;  // one fp16x2 word per packed byte
  float off0, off1, off2;
  uint32_t split1, split2;  // first byte of segment 1 / 2
  uint32_t blk0_1, blk0_2;  // first absmax block of segment 1 / 2
  uint32_t sbase1, sbase2;  // first absmax2 entry of segment 1 / 2
  uint32_t n_units;         // complete 4-byte units
  uint32_t n_bytes;
  int wide;                 // table path (blocksize >= 32)
  int hb_shift;  // log2(blocksize / 2): bytes per absmax block
  int sb_shift;  // log2(super_blocksize): absmax blocks per absmax2 entry
};

// The global inputs of the scale of the absmax block holding `byte`: its absmax code, its
// absmax2 entry and its segment's offset (all bytes of a 4-byte unit share one block because
// blocksize/2 >= 4 and segment starts are block aligned).
struct ScaleIn {
  uint32_t code;
  float a2, off;
};

__device__ __forceinline__ ScaleIn scale_inputs(const Nf4Args& a, uint32_t byte) {
  const uint32_t blk = byte >> a.hb_shift;
  uint32_t sup;
  float off;
  if (byte >= a.split2) {
    sup = a.sbase2 + ((blk - a.blk0_2) >> a.sb_shift);
    off = a.off2;
  } else if (byte >= a.split1) {
    sup = a.sbase1 + ((blk - a.blk0_1) >> a.sb_shift);
    off = a.off1;
  } else {
    sup = blk >> a.sb_shift;
    off = a.off0;
  }
  return ScaleIn{a.absmax[blk], a.absmax2[sup], off};
}

// code2[absmax] * absmax2 + offset, two roundings (no contraction in this file).
__device__ __forceinline__ float finish_scale(const ScaleIn& in, const float* __restrict__ s_code2) {
  const float s = s_code2[in.code] * in.a2;
  return s + in.off;
}

__device__ __forceinline__ float block_scale(const Nf4Args& a, uint32_t byte,
                                             const float* __restrict__ s_code2) {
  return finish_scale(scale_inputs(a, byte), s_code2);
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// One 16-byte store of four decoded words (a vector access, which the compiler keeps whole).
__device__ __forceinline__ void store16(uint32_t* p, const uint4& w) {
  *static_cast<u32x4s*>(__builtin_assume_aligned(p, 16)) = u32x4s{w.x, w.y, w.z, w.w};
}

// Decode one packed byte into the fp16x2 word (even element in the low half).
__device__ __forceinline__ uint32_t decode_byte(uint32_t b, float scale,
                                                const float* __restrict__ s_nf4) {
  const float vh = s_nf4[(b >> 4) & 15u] * scale;
  const float vl = s_nf4[b & 15u] * scale;
  h2 r;
  r.x = from_f32<f16>(vh);
  r.y = from_f32<f16>(vl);
  return __builtin_bit_cast(uint32_t, r);
}

// Dequantises block `blk` (of `nblk`) of one segment job; the LDS tables are already loaded.
template <int UNROLL>
__device__ __forceinline__ void dequant_block(const Nf4Args& a, uint32_t blk, uint32_t nblk,
                                              const float* __restrict__ s_code2,
                                              const float* __restrict__ s_nf4) {
  const uint32_t t = threadIdx.x;
  const uint32_t base = blk * (kThreads * UNROLL) + t;
  uint32_t p[UNROLL];
  float sc[UNROLL];
  if ((blk + 1) * (kThreads * UNROLL) <= a.n_units) {
    // Whole block in range (all but the last block): no per-unit checks, all loads issued first.
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) p[u] = a.packed[base + u * kThreads];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) sc[u] = block_scale(a, (base + u * kThreads) * 4u, s_code2);
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      uint4 w;
      w.x = decode_byte(p[u] & 0xffu, sc[u], s_nf4);
      w.y = decode_byte((p[u] >> 8) & 0xffu, sc[u], s_nf4);
      w.z = decode_byte((p[u] >> 16) & 0xffu, sc[u], s_nf4);
      w.w = decode_byte(p[u] >> 24, sc[u], s_nf4);
      store16(a.out + 4 * (base + u * kThreads), w);
    }
  } else {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const uint32_t idx = base + u * kThreads;
      p[u] = idx < a.n_units ? a.packed[idx] : 0u;
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const uint32_t idx = base + u * kThreads;
      sc[u] = idx < a.n_units ? block_scale(a, idx * 4u, s_code2) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const uint32_t idx = base + u * kThreads;
      if (idx < a.n_units) {
        uint4 w;
        w.x = decode_byte(p[u] & 0xffu, sc[u], s_nf4);
        w.y = decode_byte((p[u] >> 8) & 0xffu, sc[u], s_nf4);
        w.z = decode_byte((p[u] >> 16) & 0xffu, sc[u], s_nf4);
        w.w = decode_byte(p[u] >> 24, sc[u], s_nf4);
        store16(a.out + 4 * idx, w);
      }
    }
  }

  // Trailing bytes that do not fill a 4-byte unit (n_bytes % 4 != 0): the last block does them.
  if (blk == nblk - 1) {
    const uint32_t byte = a.n_units * 4u + t;
    if (byte < a.n_bytes) {
      const float s = block_scale(a, byte, s_code2);
      a.out[byte] = decode_byte(a.packed_bytes[byte], s, s_nf4);
    }
  }
}

// Table path (blocksize >= 32): a block's 4 KiB of packed bytes span at most 128 absmax blocks;
// their 16 products NF4[i] * scale (the fp32 values the reference rounds to fp16) are formed
// once in LDS, so each output is one LDS read and one conversion, with no global scale loads in
// the streaming loop. Same coalesced 4-byte loads / 16-byte stores as dequant_block.
constexpr int kTabMaxBlocks = kThreads * kUnrollTab * 4 / 16;  // 4 KiB / (blocksize/2 >= 16)

template <int UNROLL>
__device__ __forceinline__ void dequant_block_tab(const Nf4Args& a, uint32_t blk, uint32_t nblk,
                                                  float* __restrict__ s_code2,
                                                  float* __restrict__ s_nf4,
                                                  float* __restrict__ s_scale,
                                                  float* __restrict__ s_tab) {
  static_assert(UNROLL == kUnrollTab, "table sized for kUnrollTab units per thread");
  const uint32_t t = threadIdx.x;
  const uint32_t base = blk * (kThreads * UNROLL) + t;
  // 1. Every global read of the block issued at once: its packed words, the code2 table and the
  // absmax / absmax2 entries of its first kThreads absmax blocks (one per thread), so one
  // memory latency precedes the decode.
  uint32_t p[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const uint32_t idx = base + u * kThreads;
    p[u] = idx < a.n_units ? a.packed[idx] : 0u;
  }
  const uint32_t byte0 = blk * (kThreads * UNROLL * 4u);
  // The last block also covers the (< 4) bytes past the last whole unit: one more absmax block
  // at most, hence the table's spare row.
  const uint32_t byte_end =
      blk == nblk - 1 ? a.n_bytes : min(byte0 + kThreads * UNROLL * 4u, a.n_bytes);
  const uint32_t ab0 = byte0 >> a.hb_shift;
  const uint32_t n_ab = ((byte_end - 1u) >> a.hb_shift) - ab0 + 1u;
  ScaleIn mine{0u, 0.0f, 0.0f};
  if (t < n_ab) mine = scale_inputs(a, (ab0 + t) << a.hb_shift);
  // 2. Lookup tables, then one scale per absmax block of the block's range.
  s_code2[t] = a.code2[t];
  if (t < 16) s_nf4[t] = kNF4[t];
  __syncthreads();
  if (t < n_ab) s_scale[t] = finish_scale(mine, s_code2);
  for (uint32_t i = t + kThreads; i < n_ab; i += kThreads)  // blocksize 32 only: 257 blocks
    s_scale[i] = block_scale(a, (ab0 + i) << a.hb_shift, s_code2);
  __syncthreads();
  // 3. The 16 products per absmax block.
  for (uint32_t e = t; e < n_ab * 16u; e += kThreads)
    s_tab[e] = s_nf4[e & 15u] * s_scale[e >> 4];  // rounded product (no contraction here)
  __syncthreads();
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const uint32_t idx = base + u * kThreads;
    if (idx < a.n_units) {
      const float* row = s_tab + (((idx * 4u) >> a.hb_shift) - ab0) * 16u;
      uint4 w;
      uint32_t* ww = reinterpret_cast<uint32_t*>(&w);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t b = (p[u] >> (8 * k)) & 0xffu;
        h2 r;
        r.x = static_cast<_Float16>(row[b >> 4]);
        r.y = static_cast<_Float16>(row[b & 15u]);
        ww[k] = __builtin_bit_cast(uint32_t, r);
      }
      store16(a.out + 4 * idx, w);
    }
  }
  // Trailing bytes past the last 4-byte unit (n_bytes % 4 != 0): the last block does them.
  if (blk == nblk - 1) {
    const uint32_t byte = a.n_units * 4u + t;
    if (byte < a.n_bytes) {
      const float* row = s_tab + ((byte >> a.hb_shift) - ab0) * 16u;
      const uint32_t b = a.packed_bytes[byte];
      h2 r;
      r.x = static_cast<_Float16>(row[b >> 4]);
      r.y = static_cast<_Float16>(row[b & 15u]);
      a.out[byte] = __builtin_bit_cast(uint32_t, r);
    }
  }
}

__device__ __forceinline__ void load_tables(const float* __restrict__ code2, float* s_code2,
                                            float* s_nf4) {
  const uint32_t t = threadIdx.x;
  s_code2[t] = code2[t];
  if (t < 16) s_nf4[t] = kNF4[t];
  __syncthreads();
}

template <int UNROLL>
__global__ __launch_bounds__(kThreads) void nf4_dequant_kernel(Nf4Args a) {
  __shared__ float s_code2[256];
  __shared__ float s_nf4[16];
  __shared__ float s_scale[kTabMaxBlocks + 1];
  __shared__ float s_tab[(kTabMaxBlocks + 1) * 16];
  if (a.wide) {
    dequant_block_tab<UNROLL>(a, blockIdx.x, gridDim.x, s_code2, s_nf4, s_scale, s_tab);
  } else {
    load_tables(a.code2, s_code2, s_nf4);
    dequant_block<UNROLL>(a, blockIdx.x, gridDim.x, s_code2, s_nf4);
  }
}

constexpr int kMaxJobs = 4;

// Up to four segment jobs in one launch: blocks [start[j], start[j+1]) belong to job j.
struct Nf4Multi {
  Nf4Args job[kMaxJobs];
  uint32_t start[kMaxJobs + 1];
  int n_jobs;
};

template <int UNROLL>
__global__ __launch_bounds__(kThreads) void nf4_dequant_multi_kernel(Nf4Multi m) {
  __shared__ float s_code2[256];
  __shared__ float s_nf4[16];
  __shared__ float s_scale[kTabMaxBlocks + 1];
  __shared__ float s_tab[(kTabMaxBlocks + 1) * 16];
  int j = 0;
#pragma unroll
  for (int k = 1; k < kMaxJobs; ++k) j += (k < m.n_jobs && blockIdx.x >= m.start[k]) ? 1 : 0;
  if (m.job[j].wide) {  // uniform over the block; every job shares one code2 table
    dequant_block_tab<UNROLL>(m.job[j], blockIdx.x - m.start[j], m.start[j + 1] - m.start[j],
                              s_code2, s_nf4, s_scale, s_tab);
  } else {
    load_tables(m.job[0].code2, s_code2, s_nf4);
    dequant_block<UNROLL>(m.job[j], blockIdx.x - m.start[j], m.start[j + 1] - m.start[j],
                          s_code2, s_nf4);
  }
}

// A layer's dequant with one RMSNorm (forward or backward, fp16 activations) in the same launch:
// blocks [0, norm_blocks) run the norm, four rows each (one per wave), the rest the segment
// jobs as nf4_dequant_multi_kernel. The norm's rows do not depend on the weights, so the
// latency-bound norm blocks run beside the bandwidth-bound decode instead of in a launch of
// their own. Each block's role is uniform (the decode's barriers involve only its blocks).
struct NormSide {
  const f16* x;    // forward: x; backward: dy
  const f16* res;  // forward: residual; backward: dresidual (either may be null)
  const f16* h;    // backward: the norm input
  const void* w;
  float* rstd;     // forward: written; backward: read
  f16* sum_out;    // forward with residual
  f16* out;        // forward: y; backward: dx
  int n_rows, n_cols;
  int64_t stride;
  float eps;
  uint32_t blocks;
  int has_down;   // forward: the same blocks then form the LoRA-down of their rows' output
                  // (nf4_dequant_norm_down_kernel)
  DownRows down;
};

constexpr int kTabFloats = (kTabMaxBlocks + 1) * 16;
// The LoRA-down variant's s_tab also holds the down's wave sums and its staged rows (d <= 2048,
// the carried norm's limit).
constexpr int kTabFloatsDown = kDownParkFloats + down_stage_bytes(2048) / 4 > kTabFloats
                                   ? kDownParkFloats + down_stage_bytes(2048) / 4
                                   : kTabFloats;
constexpr int kDownStageU = 2;  // A fragments of 2 K steps in flight per lane

// DOWN: the forward norm's blocks then form the LoRA-down of their rows (lora_rows.h): the four
// rows and their keep bits are staged in LDS by one coalesced pass, so each wave's K loop waits
// on global memory once per kDownStageU steps (for the A fragments) instead of at every step.
// Its MFMA code needs registers the decode does not, so it is a kernel of its own (80 VGPRs,
// 6 waves per SIMD; the plain variant keeps the decode at 8). Batches of 4 or 6 steps hold
// 88-96 VGPRs (5 waves) and ran 0.5-0.9 us slower per launch at 744 tokens.
template <int UNROLL, bool BWD, typename W, int NIT, bool DOWN>
__device__ __forceinline__ void dequant_norm_body(const Nf4Multi& m, const NormSide& s) {
  __shared__ float s_code2[256];
  __shared__ float s_nf4[16];
  __shared__ float s_scale[kTabMaxBlocks + 1];
  __shared__ __attribute__((aligned(16))) float s_tab[DOWN ? kTabFloatsDown : kTabFloats];
  if (blockIdx.x < s.blocks) {
    const int row = blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
    const W* w = static_cast<const W*>(s.w);
    if constexpr (BWD) {
      if (s.res)
        rmsnorm_bwd_row<f16, W, NIT, true>(s.x, s.h, w, s.rstd, s.res, s.out, row, s.n_rows,
                                           s.n_cols, s.stride);
      else
        rmsnorm_bwd_row<f16, W, NIT, false>(s.x, s.h, w, s.rstd, s.res, s.out, row, s.n_rows,
                                            s.n_cols, s.stride);
    } else {
      if (s.res)
        rmsnorm_fwd_row<f16, W, NIT, true>(s.x, s.res, w, s.sum_out, s.out, s.rstd, row,
                                           s.n_rows, s.n_cols, s.stride, s.eps);
      else
        rmsnorm_fwd_row<f16, W, NIT, false>(s.x, s.res, w, s.sum_out, s.out, s.rstd, row,
                                            s.n_rows, s.n_cols, s.stride, s.eps);
      if constexpr (DOWN) {  // the block's four output rows are its LoRA-down tokens
        __syncthreads();  // every wave's row is stored
        const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kDownRows;
        f16* xs = reinterpret_cast<f16*>(s_tab + kDownParkFloats);
        uint32_t* bq = reinterpret_cast<uint32_t*>(xs + kDownRows * s.down.d);
        uint32_t* bv = bq + kDownRows * s.down.words;
        stage_down_rows(s.down, t0, xs, bq, bv);
        lora_down_rows4_staged<kDownStageU>(s.down, t0, xs, bq, bv, s_tab);
      }
    }
    return;
  }
  const uint32_t b = blockIdx.x - s.blocks;
  int j = 0;
#pragma unroll
  for (int k = 1; k < kMaxJobs; ++k) j += (k < m.n_jobs && b >= m.start[k]) ? 1 : 0;
  if (m.job[j].wide) {
    dequant_block_tab<UNROLL>(m.job[j], b - m.start[j], m.start[j + 1] - m.start[j], s_code2,
                              s_nf4, s_scale, s_tab);
  } else {
    load_tables(m.job[0].code2, s_code2, s_nf4);
    dequant_block<UNROLL>(m.job[j], b - m.start[j], m.start[j + 1] - m.start[j], s_code2,
                          s_nf4);
  }
}

template <int UNROLL, bool BWD, typename W, int NIT>
__global__ __launch_bounds__(kThreads) void nf4_dequant_norm_kernel(Nf4Multi m, NormSide s) {
  dequant_norm_body<UNROLL, BWD, W, NIT, false>(m, s);
}

template <int UNROLL, typename W, int NIT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(6))) void
nf4_dequant_norm_down_kernel(Nf4Multi m, NormSide s) {
  dequant_norm_body<UNROLL, false, W, NIT, true>(m, s);
}

bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

int ilog2(int64_t v) {
  int r = 0;
  while ((int64_t(1) << r) < v) ++r;
  return r;
}

}  // namespace
}  // namespace rus

namespace rus {
namespace {

constexpr int kUnrollMain = 4;
static_assert(kUnrollMain == kUnrollTab, "both paths cover 4 KiB of packed bytes per block");

// Validates one segment job and fills its kernel arguments (see rus_nf4_dequant).
int make_job(const char* fn, const uint8_t* packed, const uint8_t* absmax, const float* code2,
             const float* absmax2, float off0, float off1, float off2, int64_t split_byte_1,
             int64_t split_byte_2, int64_t absmax2_base_1, int64_t absmax2_base_2,
             int64_t n_bytes, int64_t n_absmax, int64_t n_absmax2, int32_t blocksize,
             int32_t super_blocksize, uint32_t* out_u32, Nf4Args& a) {
  if (n_bytes <= 0 || n_bytes >= (int64_t(1) << 31))
    return fail(RUS_ERR_UNSUPPORTED, "%s: n_bytes=%lld outside [1, 2^31)", fn, (long long)n_bytes);
  if (!packed || !absmax || !code2 || !absmax2 || !out_u32)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (!is_pow2(blocksize) || blocksize < 8 || !is_pow2(super_blocksize))
    return fail(RUS_ERR_INVALID,
                "%s: blocksize=%d (power of two >= 8) / super_blocksize=%d (power of two) invalid",
                fn, blocksize, super_blocksize);
  if (!aligned(packed, 4) || !aligned(out_u32, 16))
    return fail(RUS_ERR_INVALID, "%s: packed must be 4-byte and out 16-byte aligned", fn);
  const int64_t half_block = blocksize / 2;
  if (split_byte_1 < 0 || split_byte_2 < split_byte_1 || split_byte_2 > n_bytes)
    return fail(RUS_ERR_INVALID, "%s: splits (%lld, %lld) not ordered in [0, %lld]", fn,
                (long long)split_byte_1, (long long)split_byte_2, (long long)n_bytes);
  if ((split_byte_1 < n_bytes && split_byte_1 % half_block) ||
      (split_byte_2 < n_bytes && split_byte_2 % half_block))
    return fail(RUS_ERR_INVALID,
                "%s: segment starts (%lld, %lld) must be multiples of blocksize/2=%lld", fn,
                (long long)split_byte_1, (long long)split_byte_2, (long long)half_block);
  if (absmax2_base_1 < 0 || absmax2_base_2 < absmax2_base_1)
    return fail(RUS_ERR_INVALID, "%s: absmax2 bases must be non-negative, ordered", fn);
  // Every absmax / absmax2 index the kernel can form must be in range.
  const int hb = ilog2(half_block), sb = ilog2(super_blocksize);
  const int64_t last_blk = (n_bytes - 1) >> hb;
  if (last_blk >= n_absmax)
    return fail(RUS_ERR_INVALID, "%s: absmax has %lld entries, needs %lld", fn,
                (long long)n_absmax, (long long)(last_blk + 1));
  const int64_t starts[3] = {0, split_byte_1, split_byte_2};
  const int64_t ends[3] = {split_byte_1, split_byte_2, n_bytes};
  const int64_t bases[3] = {0, absmax2_base_1, absmax2_base_2};
  for (int s = 0; s < 3; ++s) {
    if (ends[s] <= starts[s]) continue;
    const int64_t blk_first = starts[s] >> hb, blk_last = (ends[s] - 1) >> hb;
    const int64_t sup_last = bases[s] + ((blk_last - blk_first) >> sb);
    if (sup_last >= n_absmax2)
      return fail(RUS_ERR_INVALID, "%s: absmax2 has %lld entries, segment %d needs index %lld",
                  fn, (long long)n_absmax2, s, (long long)sup_last);
  }
  a.packed = reinterpret_cast<const uint32_t*>(packed);
  a.packed_bytes = packed;
  a.absmax = absmax;
  a.code2 = code2;
  a.absmax2 = absmax2;
  a.out = out_u32;
  a.off0 = off0;
  a.off1 = off1;
  a.off2 = off2;
  // A split equal to n_bytes means "segment absent"; it is never reached.
  a.split1 = static_cast<uint32_t>(split_byte_1);
  a.split2 = static_cast<uint32_t>(split_byte_2);
  a.hb_shift = hb;
  a.sb_shift = sb;
  a.blk0_1 = static_cast<uint32_t>(split_byte_1 >> hb);
  a.blk0_2 = static_cast<uint32_t>(split_byte_2 >> hb);
  a.sbase1 = static_cast<uint32_t>(absmax2_base_1);
  a.sbase2 = static_cast<uint32_t>(absmax2_base_2);
  a.n_bytes = static_cast<uint32_t>(n_bytes);
  a.n_units = static_cast<uint32_t>(n_bytes / 4);
  a.wide = half_block >= 16 ? 1 : 0;
  return RUS_OK;
}

uint32_t blocks_for(const Nf4Args& a) {
  const uint32_t per_block = kThreads * kUnrollMain;  // kUnrollTab == kUnrollMain
  const uint32_t g = (a.n_units + per_block - 1) / per_block;
  return g == 0 ? 1 : g;  // tail-only input
}

}  // namespace
}  // namespace rus

extern "C" int rus_nf4_dequant(const uint8_t* packed, const uint8_t* absmax, const float* code2,
                               const float* absmax2, float off0, float off1, float off2,
                               int64_t split_byte_1, int64_t split_byte_2, int64_t absmax2_base_1,
                               int64_t absmax2_base_2, int64_t n_bytes, int64_t n_absmax,
                               int64_t n_absmax2, int32_t blocksize, int32_t super_blocksize,
                               uint32_t* out_u32, void* stream) {
  using namespace rus;
  if (n_bytes == 0) return RUS_OK;
  Nf4Args a;
  if (int e = make_job("rus_nf4_dequant", packed, absmax, code2, absmax2, off0, off1, off2,
                       split_byte_1, split_byte_2, absmax2_base_1, absmax2_base_2, n_bytes,
                       n_absmax, n_absmax2, blocksize, super_blocksize, out_u32, a))
    return e;
  hipLaunchKernelGGL(nf4_dequant_kernel<kUnrollMain>, dim3(blocks_for(a)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return check_launch("rus_nf4_dequant");
}

extern "C" int rus_nf4_dequant_multi(const rus_nf4_job* jobs, int32_t n_jobs, const float* code2,
                                     int32_t blocksize, int32_t super_blocksize, void* stream) {
  using namespace rus;
  const char* fn = "rus_nf4_dequant_multi";
  if (n_jobs <= 0 || n_jobs > kMaxJobs || !jobs)
    return fail(RUS_ERR_INVALID, "%s: n_jobs=%d outside [1, %d]", fn, n_jobs, kMaxJobs);
  Nf4Multi m{};
  m.n_jobs = n_jobs;
  uint32_t total = 0;
  for (int j = 0; j < n_jobs; ++j) {
    const rus_nf4_job& q = jobs[j];
    if (int e = make_job(fn, q.packed, q.absmax, code2, q.absmax2, q.off0, q.off1, q.off2,
                         q.split_byte_1, q.split_byte_2, q.absmax2_base_1, q.absmax2_base_2,
                         q.n_bytes, q.n_absmax, q.n_absmax2, blocksize, super_blocksize,
                         q.out_u32, m.job[j]))
      return e;
    m.start[j] = total;
    total += blocks_for(m.job[j]);
  }
  for (int j = n_jobs; j <= kMaxJobs; ++j) m.start[j] = total;
  hipLaunchKernelGGL(nf4_dequant_multi_kernel<kUnrollMain>, dim3(total), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), m);
  return check_launch(fn);
}

extern "C" int rus_nf4_dequant_multi_norm(const rus_nf4_job* jobs, int32_t n_jobs,
                                          const float* code2, int32_t blocksize,
                                          int32_t super_blocksize, const rus_norm_side* side,
                                          const rus_lora_rows* down, void* stream) {
  using namespace rus;
  const char* fn = "rus_nf4_dequant_multi_norm";
  if (n_jobs <= 0 || n_jobs > kMaxJobs || !jobs || !side)
    return fail(RUS_ERR_INVALID, "%s: n_jobs=%d outside [1, %d] or no norm", fn, n_jobs,
                kMaxJobs);
  const rus_norm_side& q = *side;
  const bool bwd = q.kind == RUS_NORM_BWD;
  if (q.kind != RUS_NORM_FWD && !bwd) return fail(RUS_ERR_INVALID, "%s: kind %d", fn, q.kind);
  if (q.w_dtype != RUS_DTYPE_F16 && q.w_dtype != RUS_DTYPE_F32)
    return fail(RUS_ERR_INVALID, "%s: w_dtype %d", fn, q.w_dtype);
  if (q.n_rows <= 0 || q.n_rows >= (int64_t(1) << 31) || q.n_cols <= 0 || q.stride_row < q.n_cols)
    return fail(RUS_ERR_INVALID, "%s: bad norm shape", fn);
  if (!q.x || !q.weight || !q.rstd || !q.out || (bwd && !q.h) || (!bwd && q.residual && !q.sum_out))
    return fail(RUS_ERR_INVALID, "%s: null norm operand", fn);
  const int nit = q.n_cols <= 512 ? 1 : q.n_cols <= 1024 ? 2 : q.n_cols <= 1536 ? 3
                  : q.n_cols <= 2048 ? 4 : 0;
  if (nit == 0 || q.n_cols % 8 || q.stride_row % 8 || !aligned(q.x, 16) || !aligned(q.out, 16) ||
      !aligned(q.weight, 16) || (q.residual && !aligned(q.residual, 16)) ||
      (q.h && !aligned(q.h, 16)) || (q.sum_out && !aligned(q.sum_out, 16)))
    return fail(RUS_ERR_UNSUPPORTED,
                "%s: the norm needs n_cols <= 2048, n_cols and stride multiples of 8 and "
                "16-byte aligned rows", fn);
  DownRows dn{};
  if (down) {
    if (bwd || down->x != q.out || down->n_tokens != q.n_rows || down->d != q.n_cols ||
        down->stride_x != q.stride_row)
      return fail(RUS_ERR_INVALID,
                  "%s: the carried LoRA-down must read the forward norm's output rows", fn);
    if (int e = lora_rows_args(fn, *down, dn)) return e;
  }
  Nf4Multi m{};
  m.n_jobs = n_jobs;
  uint32_t total = 0;
  for (int j = 0; j < n_jobs; ++j) {
    const rus_nf4_job& jb = jobs[j];
    if (int e = make_job(fn, jb.packed, jb.absmax, code2, jb.absmax2, jb.off0, jb.off1, jb.off2,
                         jb.split_byte_1, jb.split_byte_2, jb.absmax2_base_1, jb.absmax2_base_2,
                         jb.n_bytes, jb.n_absmax, jb.n_absmax2, blocksize, super_blocksize,
                         jb.out_u32, m.job[j]))
      return e;
    m.start[j] = total;
    total += blocks_for(m.job[j]);
  }
  for (int j = n_jobs; j <= kMaxJobs; ++j) m.start[j] = total;
  NormSide ns{static_cast<const f16*>(q.x),
              static_cast<const f16*>(q.residual),
              static_cast<const f16*>(q.h),
              q.weight,
              q.rstd,
              static_cast<f16*>(q.sum_out),
              static_cast<f16*>(q.out),
              static_cast<int>(q.n_rows),
              static_cast<int>(q.n_cols),
              q.stride_row,
              q.eps,
              static_cast<uint32_t>((q.n_rows + kThreads / kWave - 1) / (kThreads / kWave)),
              down ? 1 : 0,
              dn};
  const dim3 grid(total + ns.blocks);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto launch = [&](auto bwd_c, auto wtag, auto nit_c) {
    constexpr bool B = decltype(bwd_c)::value;
    constexpr int N = decltype(nit_c)::value;
    using WT = decltype(wtag);
    if constexpr (!B) {
      if (ns.has_down) {
        hipLaunchKernelGGL((nf4_dequant_norm_down_kernel<kUnrollMain, WT, N>), grid,
                           dim3(kThreads), 0, st, m, ns);
        return;
      }
    }
    hipLaunchKernelGGL((nf4_dequant_norm_kernel<kUnrollMain, B, WT, N>), grid, dim3(kThreads), 0,
                       st, m, ns);
  };
  auto by_nit = [&](auto bwd_c, auto wtag) {
    switch (nit) {
      case 1: launch(bwd_c, wtag, std::integral_constant<int, 1>{}); break;
      case 2: launch(bwd_c, wtag, std::integral_constant<int, 2>{}); break;
      case 3: launch(bwd_c, wtag, std::integral_constant<int, 3>{}); break;
      default: launch(bwd_c, wtag, std::integral_constant<int, 4>{}); break;
    }
  };
  auto by_w = [&](auto bwd_c) {
    if (q.w_dtype == RUS_DTYPE_F16)
      by_nit(bwd_c, f16{});
    else
      by_nit(bwd_c, float{});
  };
  if (bwd)
    by_w(std::true_type{});
  else
    by_w(std::false_type{});
  return check_launch(fn);
}
