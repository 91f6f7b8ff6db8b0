// The fp16 MFMA GEMM mainloop shared by the lm_head kernels (lmhead.hip) and the projections'
// split-K product (gemm.hip): C[M, N] (+)= A[M, K] . op(B) on v_mfma_f32_32x32x16_f16, 256 x 256
// block tiles, blocks numbered XCD-aware, A always K-contiguous ([M, lda]) and B either
// K-contiguous ([N, ldb], op(B) = B^T) or N-contiguous ([K, ldb], op(B) = B), the second read
// out of LDS with gfx950's transposing ds_read_b64_tr_b16.
#pragma once

#include <type_traits>

#include "common.h"

namespace rus {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 64;
constexpr int kThreads = 256;
constexpr int kWM = 128, kWN = 128;
constexpr int kMT = kWM / 32, kNT = kWN / 32;
constexpr int kTileBytes = kBM * kBK * 2;  // 32 KiB
constexpr int kSmemBytes = 4 * kTileBytes;  // 128 KiB: the mainloop's four stages, the epilogues' staging

struct GemmArgs {
  const f16* A;  // [M, lda], rows K-contiguous
  const f16* B;  // [N, ldb] K-contiguous, or [K, ldb] N-contiguous (the KN mainloop)
  int64_t lda, ldb;
  int M, N;
  int K;            // multiple of kBK
  int k_per_split;  // multiple of kBK
  int splits;
  int tiles_m, tiles_n;
};

struct Tile {
  int m0, n0, split;
};

__device__ __forceinline__ bool tile_of(const GemmArgs& g, Tile& t) {
  const int total = g.tiles_m * g.tiles_n * g.splits;
  const int per_xcd = (total + 7) >> 3;
  const int local = blockIdx.x >> 3;
  const int work = (blockIdx.x & 7) * per_xcd + local;
  if (local >= per_xcd || work >= total) return false;
  const int tn = work % g.tiles_n;
  const int rest = work / g.tiles_n;
  t.m0 = (rest % g.tiles_m) * kBM;
  t.split = rest / g.tiles_m;
  t.n0 = tn * kBN;
  return true;
}

// acc[mt][nt] += A[m0 + wm*128 + mt*32 .. +32, k] . B[n0 + wn*128 + nt*32 .. +32, k]^T over the
// split's K range. Accumulator layout (v_mfma_f32_32x32x16_f16): register r of lane l holds
// row 8*(r/4) + 4*(l/32) + r%4, column l%32 of the 32x32 tile.
//
// Two pipelines. mainloop_t (the four-wave kernels: statistics and logit gradient) stages K 32 at
// a time through NS LDS buffers of 32 KiB (A then B, 256 rows x 64 bytes each; NS = 4);
// mainloop_k64 (the eight-wave kernels) stages K 64 at a time, below. Global memory is copied
// straight into LDS (global_load_lds_dwordx4: each lane's 16 bytes land at buffer + lane * 16),
// NS - 1 stages ahead of the MFMAs, so no register holds a tile in flight. The 16-byte chunk c of row r is stored
// at chunk c ^ ((r >> 2) & 3) of its 64-byte row, which a lane realises by loading the chunk
// that belongs at its position; the MFMAs' 16-byte fragment reads (16 consecutive rows per quarter
// wave, one chunk) then hit all 64 banks once. The fragment reads are explicit ds_read_b128 with
// explicit lgkmcnt waits (the compiler would otherwise wait for every LDS-bound global load before
// any LDS read); vmcnt waits and the one barrier per stage sit inside the stage's second K step,
// so the MFMA pipe keeps busy across stages.
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

constexpr int kDK = 32;                  // K per LDS stage
constexpr int kStageBytes = 2 * kBM * kDK * 2;  // A + B: 32 KiB
constexpr int kNStages = 4;
static_assert(kNStages * kStageBytes == kSmemBytes, "stages fill the kernel's LDS");

template <int OFF>
__device__ __forceinline__ u32x4v lds_read16(uint32_t addr) {
  u32x4v v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

// The fragments of one K step of 16 from LDS addresses a (4 A row groups) / b (NT B row groups).
template <int NT>
__device__ __forceinline__ void read_frags(uint32_t a, uint32_t b, u32x4v (&fa)[kMT],
                                           u32x4v (&fb)[NT]) {
  fa[0] = lds_read16<0>(a);
  fa[1] = lds_read16<2048>(a);
  fa[2] = lds_read16<4096>(a);
  fa[3] = lds_read16<6144>(a);
  fb[0] = lds_read16<0>(b);
  fb[1] = lds_read16<2048>(b);
  if constexpr (NT == 4) {
    fb[2] = lds_read16<4096>(b);
    fb[3] = lds_read16<6144>(b);
  }
}

// Every LDS read issued so far has returned; ties the fragments so that no MFMA using them is
// scheduled before the wait.
template <int NT>
__device__ __forceinline__ void wait_frags(u32x4v (&fa)[kMT], u32x4v (&fb)[NT]) {
  if constexpr (NT == 4)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1]),
                   "+v"(fb[2]), "+v"(fb[3]));
  else
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(fb[0]), "+v"(fb[1]));
}

template <int NT>
__device__ __forceinline__ void mma16(const u32x4v (&fa)[kMT], const u32x4v (&fb)[NT],
                                      f32x16 (&acc)[kMT][NT]) {
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          __builtin_bit_cast(f16x8, fa[mt]), __builtin_bit_cast(f16x8, fb[nt]), acc[mt][nt], 0,
          0, 0);
}

// B stored [K][N] (N-contiguous) in LDS: 32 rows of 256 columns (512 bytes) per stage, the
// 16-byte chunk c of row r at chunk c ^ ((r & 3) << 2). ds_read_b64_tr_b16 lets each group of 16
// lanes read a 4 x 16 block and transposes it: lane i of the group receives the 16-bit element
// i % 4 of the 8 bytes read by lanes i / 4 + 4 e (e = 0..3) of the group. With lane j of the group
// pointing at row k0 + j / 4, columns n0 + 4 (j % 4) .. +4, lane i therefore holds
// B[k0 + e][n0 + i], e = 0..3: the low or high half of its MFMA B operand (8 consecutive K of
// column n0 + i). The four rows a group reads sit in four different 64-byte quarters of the
// 256-byte bank window, so a half wave's 32 lanes hit all 64 banks once.
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

template <int OFF>
__device__ __forceinline__ u32x2v lds_read8_tr(uint32_t addr) {
  u32x2v v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}

constexpr int kKNRowBytes = kBN * 2;  // one K row of the B stage: 512 bytes

// The fragments of K step KK (0 or 1) of a stage: A as read_frags, B from the per-tile addresses
// b[nt] (+ sb, the stage's offset).
template <int NT, int KK>
__device__ __forceinline__ void read_frags_kn(uint32_t a, const uint32_t (&b)[NT], uint32_t sb,
                                              u32x4v (&fa)[kMT], u32x2v (&lo)[NT],
                                              u32x2v (&hi)[NT]) {
  fa[0] = lds_read16<0>(a);
  fa[1] = lds_read16<2048>(a);
  fa[2] = lds_read16<4096>(a);
  fa[3] = lds_read16<6144>(a);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    lo[nt] = lds_read8_tr<KK * 16 * kKNRowBytes>(b[nt] + sb);
    hi[nt] = lds_read8_tr<KK * 16 * kKNRowBytes + 4 * kKNRowBytes>(b[nt] + sb);
  }
}

template <int NT>
__device__ __forceinline__ void wait_frags_kn(u32x4v (&fa)[kMT], u32x2v (&lo)[NT],
                                              u32x2v (&hi)[NT]) {
  if constexpr (NT == 4)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(lo[0]), "+v"(lo[1]),
                   "+v"(lo[2]), "+v"(lo[3]), "+v"(hi[0]), "+v"(hi[1]), "+v"(hi[2]), "+v"(hi[3]));
  else
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(fa[0]), "+v"(fa[1]), "+v"(fa[2]), "+v"(fa[3]), "+v"(lo[0]), "+v"(lo[1]),
                   "+v"(hi[0]), "+v"(hi[1]));
}

template <int NT>
__device__ __forceinline__ void mma16_kn(const u32x4v (&fa)[kMT], const u32x2v (&lo)[NT],
                                         const u32x2v (&hi)[NT], f32x16 (&acc)[kMT][NT]) {
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const u32x4v b = {lo[nt].x, lo[nt].y, hi[nt].x, hi[nt].y};
      acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          __builtin_bit_cast(f16x8, fa[mt]), __builtin_bit_cast(f16x8, b), acc[mt][nt], 0, 0, 0);
    }
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt not waited on).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Waits until at most `stages` (0..4) stages of PER copies each are still in flight.
template <int PER>
__device__ __forceinline__ void wait_stages(int stages) {
  if (stages >= 4)
    wait_vmcnt<4 * PER>();
  else if (stages == 3)
    wait_vmcnt<3 * PER>();
  else if (stages == 2)
    wait_vmcnt<2 * PER>();
  else if (stages == 1)
    wait_vmcnt<PER>();
  else
    wait_vmcnt<0>();
}

// NW = 4: waves 2 (M halves) x 2 (N halves) of 128 x 128 (acc[4][4], one wave per SIMD), the
// layout of the kernels whose epilogues need 4 x 4 accumulator tiles per wave; NW = 8: 2 x 4 waves
// of 128 x 64 (acc[4][2]). Same LDS stages and A swizzle either way. KN: B is [K, ldb]
// N-contiguous (NW = 8 only), staged as 32 K rows of 512 bytes per stage. The eight-wave kernels
// run mainloop_k64 instead: its whole-line copies made them ~10% faster (isolated, same bits).
template <int NW, bool KN = false, int NS = kNStages>
__device__ __forceinline__ void mainloop_t(const GemmArgs& g, const Tile& tl, char* smem,
                                           f32x16 (&acc)[kMT][16 / NW]) {
  static_assert(!KN || NW == 8, "the N-contiguous B layout runs on eight waves");
  constexpr int NT = 16 / NW;        // 32-column MFMA tiles per wave
  constexpr int RW = kBN / (NW / 2);  // B rows (N) per wave: 128 or 64
  constexpr int CP = 16 / NW;        // copies per thread per operand and stage: 4 or 2
  constexpr int PER = 2 * CP;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);
  const int kb = tl.split * g.k_per_split;
  const int ke = min(kb + g.k_per_split, g.K);
  const int KT = ke > kb ? (ke - kb) / kDK : 0;
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x16{};
  if (KT == 0) {
    __syncthreads();
    return;
  }
  // Copies: instruction i of wave w fills bytes 1024 (NW i + w) .. +1024 of the stage's A and B
  // tiles. A (and K-contiguous B): rows 16 NW i + 16 w .. +16 of 64 bytes; lane l covers row
  // 16 NW i + 16 w + l/4 at position l%4, i.e. the chunk (l%4) ^ ((l/16) & 3). N-contiguous B:
  // K rows 2 (NW i + w) + l/32 of 512 bytes; lane l covers position l%32 of its row r, i.e. the
  // chunk (l%32) ^ ((r & 3) << 2), columns n0 + 8 chunk .. +8.
  const int lrow = 16 * wave + (lane >> 2);
  const int lchunk = (lane & 3) ^ ((lane >> 4) & 3);
  const char* gA = reinterpret_cast<const char*>(g.A);
  const char* gB = reinterpret_cast<const char*>(g.B);
  uint32_t oa[CP], ob[CP];
#pragma unroll
  for (int i = 0; i < CP; ++i) {
    // Rows (columns) past the matrix edge re-read the last one: finite values the epilogues
    // discard.
    const int ra_ = min(tl.m0 + lrow + 16 * NW * i, g.M - 1);
    oa[i] = static_cast<uint32_t>((ra_ * g.lda + kb + lchunk * 8) * 2);
    if constexpr (KN) {
      const int krow = 2 * (NW * i + wave) + (lane >> 5);
      const int col = min(tl.n0 + 8 * ((lane & 31) ^ ((krow & 3) << 2)), g.N - 8);
      ob[i] = static_cast<uint32_t>(((kb + krow) * g.ldb + col) * 2);
    } else {
      const int rb_ = min(tl.n0 + lrow + 16 * NW * i, g.N - 1);
      ob[i] = static_cast<uint32_t>((rb_ * g.ldb + kb + lchunk * 8) * 2);
    }
  }
  const uint32_t bstep = KN ? static_cast<uint32_t>(kDK * g.ldb * 2) : kDK * 2;
  auto issue = [&](int k) {  // stage k's copies into buffer k % NS
    char* st = smem + (k % NS) * kStageBytes;
    const uint32_t abytes = k * (kDK * 2), bbytes = k * bstep;
#pragma unroll
    for (int i = 0; i < CP; ++i) {
      __builtin_amdgcn_global_load_lds(gA + oa[i] + abytes,
                                       (lds_void_ptr)(st + (NW * i + wave) * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(gB + ob[i] + bbytes,
                                       (lds_void_ptr)(st + kBM * 64 + (NW * i + wave) * 1024), 16,
                                       0, 0);
    }
  };
  const int pre = min(NS, KT);
  for (int k = 0; k < pre; ++k) issue(k);
  wait_stages<PER>(pre - 1);  // stage 0 landed (this wave's copies)
  __builtin_amdgcn_s_barrier();  // ... and every wave's
  // Fragment addresses: A row wm*128 + (l & 31), B row wn*RW + (l & 31) (+ 32 per MFMA tile,
  // immediate), chunk 2 kk + l/32 stored at chunk ^ ((l >> 2) & 3). N-contiguous B: lane l of
  // group g = l/16 (j = l%16) reads K row 16 kk + 8 (g/2) + j/4 (+ 4 for the high half), columns
  // wn*64 + 32 nt + 16 (g%2) + 4 (j%4).
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_ptr)smem));
  const int sw = (lane >> 2) & 3, half = lane >> 5;
  const uint32_t c0 = ((0 + half) ^ sw) << 4, c1 = ((2 + half) ^ sw) << 4;
  const uint32_t arow = lds0 + (wm * kWM + (lane & 31)) * 64;
  const uint32_t a0 = arow + c0, a1 = arow + c1;
  if constexpr (KN) {
    const int j = lane & 15, nh = (lane >> 4) & 1;
    uint32_t bk[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int col = wn * RW + nt * 32 + 16 * nh + 4 * (j & 3);
      bk[nt] = lds0 + kBM * 64 + (8 * half + (j >> 2)) * kKNRowBytes +
               (((col >> 3) ^ ((j >> 2) << 2)) << 4) + (col & 7) * 2;
    }
    u32x4v fa0[kMT], fa1[kMT];
    u32x2v lo0[NT], hi0[NT], lo1[NT], hi1[NT];
    read_frags_kn<NT, 0>(a0, bk, 0, fa0, lo0, hi0);
    wait_frags_kn<NT>(fa0, lo0, hi0);
    for (int k = 0; k < KT; ++k) {
      const uint32_t sb = (k % NS) * kStageBytes;
      read_frags_kn<NT, 1>(a1 + sb, bk, sb, fa1, lo1, hi1);  // step 1 of stage k
      __builtin_amdgcn_sched_barrier(0);
      mma16_kn<NT>(fa0, lo0, hi0, acc);  // step 0 of stage k
      __builtin_amdgcn_sched_barrier(0);
      wait_frags_kn<NT>(fa1, lo1, hi1);
      if (k + 1 < KT) {
        wait_stages<PER>(min(NS - 2, KT - 2 - k));
        __builtin_amdgcn_s_barrier();
        if (k + NS < KT) issue(k + NS);
        const uint32_t nb = ((k + 1) % NS) * kStageBytes;
        read_frags_kn<NT, 0>(a0 + nb, bk, nb, fa0, lo0, hi0);  // step 0 of stage k + 1
      }
      __builtin_amdgcn_sched_barrier(0);
      mma16_kn<NT>(fa1, lo1, hi1, acc);  // step 1 of stage k
      __builtin_amdgcn_sched_barrier(0);
      if (k + 1 < KT) wait_frags_kn<NT>(fa0, lo0, hi0);
    }
  } else {
    const uint32_t brow = lds0 + kBM * 64 + (wn * RW + (lane & 31)) * 64;
    const uint32_t b0 = brow + c0, b1 = brow + c1;
    u32x4v fa0[kMT], fb0[NT], fa1[kMT], fb1[NT];
    read_frags<NT>(a0, b0, fa0, fb0);
    wait_frags<NT>(fa0, fb0);
    for (int k = 0; k < KT; ++k) {
      const uint32_t sb = (k % NS) * kStageBytes;
      read_frags<NT>(a1 + sb, b1 + sb, fa1, fb1);  // step 1 of stage k
      __builtin_amdgcn_sched_barrier(0);
      mma16<NT>(fa0, fb0, acc);  // step 0 of stage k
      __builtin_amdgcn_sched_barrier(0);
      wait_frags<NT>(fa1, fb1);
      if (k + 1 < KT) {
        // Stage k + 1 has landed for every wave, and every wave has read stage k: its buffer
        // takes stage k + 4.
        wait_stages<PER>(min(NS - 2, KT - 2 - k));
        __builtin_amdgcn_s_barrier();
        if (k + NS < KT) issue(k + NS);
        const uint32_t nb = ((k + 1) % NS) * kStageBytes;
        read_frags<NT>(a0 + nb, b0 + nb, fa0, fb0);  // step 0 of stage k + 1
      }
      __builtin_amdgcn_sched_barrier(0);
      mma16<NT>(fa1, fb1, acc);  // step 1 of stage k
      __builtin_amdgcn_sched_barrier(0);
      if (k + 1 < KT) wait_frags<NT>(fa0, fb0);
    }
  }
  __syncthreads();  // the epilogues reuse the LDS
}

// Eight waves (2 x 4 of 128 x 64) with K staged 64 at a time through two 64 KiB LDS buffers:
// every global -> LDS copy instruction then moves 8 whole 128-byte lines (8 rows x 64 K of a
// K-contiguous operand) instead of 16 half lines, which doubles what the copy path delivers per
// CU. Rows of 128 bytes, the 16-byte chunk c of row r stored at c ^ ((r >> 1) & 7): the 16 rows a
// quarter wave reads at one chunk then cover all 64 banks once. N-contiguous B: 64 K rows of 512
// bytes per stage (the chunk c of row r at c ^ ((r & 3) << 2), as in the 32-deep stages). The
// copies of stage k + 2 are issued after the barrier that ends the reads of stage k; one barrier
// per 64 K.
constexpr int kDK64 = 64;
constexpr int kStage64 = 2 * kBM * kDK64 * 2;  // 64 KiB
constexpr int kSmem64 = 2 * kStage64;          // 128 KiB

template <int NW, bool KN>
__device__ __forceinline__ void mainloop_k64(const GemmArgs& g, const Tile& tl, char* smem,
                                             f32x16 (&acc)[kMT][16 / NW]) {
  static_assert(NW == 4 || NW == 8, "four waves of 128 x 128 or eight of 128 x 64");
  static_assert(!KN || NW == 8, "the N-contiguous B layout runs on eight waves");
  constexpr int NT = 16 / NW;         // 32-column MFMA tiles per wave
  constexpr int RW = kBN / (NW / 2);  // B rows (N) per wave: 128 or 64
  constexpr int CP = 32 / NW;         // copies per wave per operand and stage: 8 or 4
  constexpr int PER = 2 * CP;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(t >> 6));
  const int wm = wave / (NW / 2), wn = wave % (NW / 2);
  const int kb = tl.split * g.k_per_split;
  const int ke = min(kb + g.k_per_split, g.K);
  const int KT = ke > kb ? (ke - kb) / kDK64 : 0;
#pragma unroll
  for (int mt = 0; mt < kMT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = f32x16{};
  if (KT == 0) {
    __syncthreads();
    return;
  }
  // Copies: instruction i of wave w fills bytes 1024 (NW i + w) .. +1024 of the stage's A tile
  // (rows 8 (NW i + w) .. +8; lane l covers row + l/8 at position l%8, i.e. the chunk
  // (l%8) ^ ((row >> 1) & 7)) and the same bytes of the B tile (K-contiguous as A; N-contiguous:
  // K rows 2 (NW i + w) + l/32 of 512 bytes, lane l at position l%32 of its row r, the chunk
  // (l%32) ^ ((r & 3) << 2), columns n0 + 8 chunk .. +8).
  const char* gA = reinterpret_cast<const char*>(g.A);
  const char* gB = reinterpret_cast<const char*>(g.B);
  uint32_t oa[CP], ob[CP];
#pragma unroll
  for (int i = 0; i < CP; ++i) {
    const int row = 8 * (NW * i + wave) + (lane >> 3);
    const int ch = (lane & 7) ^ ((row >> 1) & 7);
    // Rows (columns) past the matrix edge re-read the last one: finite values the epilogues
    // discard.
    const int ra_ = min(tl.m0 + row, g.M - 1);
    oa[i] = static_cast<uint32_t>((ra_ * g.lda + kb + ch * 8) * 2);
    if constexpr (KN) {
      const int krow = 2 * (NW * i + wave) + (lane >> 5);
      const int col = min(tl.n0 + 8 * ((lane & 31) ^ ((krow & 3) << 2)), g.N - 8);
      ob[i] = static_cast<uint32_t>(((kb + krow) * g.ldb + col) * 2);
    } else {
      const int rb_ = min(tl.n0 + row, g.N - 1);
      ob[i] = static_cast<uint32_t>((rb_ * g.ldb + kb + ch * 8) * 2);
    }
  }
  const uint32_t bstep = KN ? static_cast<uint32_t>(kDK64 * g.ldb * 2) : kDK64 * 2;
  auto issue = [&](int k) {  // stage k's copies into buffer k % 2
    char* st = smem + (k & 1) * kStage64 + wave * 1024;
    const uint32_t abytes = k * (kDK64 * 2), bbytes = k * bstep;
#pragma unroll
    for (int i = 0; i < CP; ++i) {
      __builtin_amdgcn_global_load_lds(gA + oa[i] + abytes, (lds_void_ptr)(st + i * NW * 1024),
                                       16, 0, 0);
      __builtin_amdgcn_global_load_lds(gB + ob[i] + bbytes,
                                       (lds_void_ptr)(st + kBM * 128 + i * NW * 1024), 16, 0, 0);
    }
  };
  // Fragment addresses. A: row wm*128 + (l & 31) (+ 32 per MFMA tile: immediate 4096), chunk
  // 2 kk + l/32 at position chunk ^ ((l >> 1) & 7) (the low row bits are those of l). B
  // K-contiguous likewise (rows wn*RW + ...); N-contiguous: lane l of group g = l/16 (j = l%16)
  // reads K row 16 kk + 8 (g/2) + j/4 (+ 4 for the high half), columns wn*64 + 32 nt + 16 (g%2)
  // + 4 (j%4).
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_ptr)smem));
  const int sw = (lane >> 1) & 7, half = lane >> 5;
  uint32_t cpos[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) cpos[kk] = static_cast<uint32_t>(((2 * kk + half) ^ sw) << 4);
  const uint32_t arow = lds0 + (wm * kWM + (lane & 31)) * 128;
  const uint32_t brow = lds0 + kBM * 128 + (wn * RW + (lane & 31)) * 128;
  uint32_t bk[NT];
  if constexpr (KN) {
    const int j = lane & 15, nh = (lane >> 4) & 1;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int col = wn * RW + nt * 32 + 16 * nh + 4 * (j & 3);
      bk[nt] = lds0 + kBM * 128 + (8 * half + (j >> 2)) * kKNRowBytes +
               (((col >> 3) ^ ((j >> 2) << 2)) << 4) + (col & 7) * 2;
    }
  }
  u32x4v fa[2][kMT], fb[2][NT];
  u32x2v lo[2][NT], hi[2][NT];
  // Fragments of K step kk (0..3) of the stage at byte offset sb into register set S.
  auto read = [&](auto S, uint32_t sb, int kk) {
    constexpr int s = decltype(S)::value;
    const uint32_t a = arow + sb + cpos[kk];
    fa[s][0] = lds_read16<0>(a);
    fa[s][1] = lds_read16<4096>(a);
    fa[s][2] = lds_read16<8192>(a);
    fa[s][3] = lds_read16<12288>(a);
    if constexpr (KN) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        lo[s][nt] = lds_read8_tr<0>(bk[nt] + sb + kk * 16 * kKNRowBytes);
        hi[s][nt] = lds_read8_tr<4 * kKNRowBytes>(bk[nt] + sb + kk * 16 * kKNRowBytes);
      }
    } else {
      const uint32_t b = brow + sb + cpos[kk];
      fb[s][0] = lds_read16<0>(b);
      fb[s][1] = lds_read16<4096>(b);
      if constexpr (NT == 4) {
        fb[s][2] = lds_read16<8192>(b);
        fb[s][3] = lds_read16<12288>(b);
      }
    }
  };
  auto wait = [&](auto S) {
    constexpr int s = decltype(S)::value;
    if constexpr (KN)
      wait_frags_kn<NT>(fa[s], lo[s], hi[s]);
    else
      wait_frags<NT>(fa[s], fb[s]);
  };
  auto mma = [&](auto S) {
    constexpr int s = decltype(S)::value;
    if constexpr (KN)
      mma16_kn<NT>(fa[s], lo[s], hi[s], acc);
    else
      mma16<NT>(fa[s], fb[s], acc);
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  issue(0);
  if (KT > 1) issue(1);
  if (KT > 1)
    wait_vmcnt<PER>();  // stage 0 landed (this wave's copies)
  else
    wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();  // ... and every wave's
  read(S0{}, 0, 0);
  wait(S0{});
  for (int k = 0; k < KT; ++k) {
    const uint32_t sb = (k & 1) * kStage64;
    read(S1{}, sb, 1);
    __builtin_amdgcn_sched_barrier(0);
    mma(S0{});
    __builtin_amdgcn_sched_barrier(0);
    wait(S1{});
    read(S0{}, sb, 2);
    __builtin_amdgcn_sched_barrier(0);
    mma(S1{});
    __builtin_amdgcn_sched_barrier(0);
    wait(S0{});
    read(S1{}, sb, 3);
    __builtin_amdgcn_sched_barrier(0);
    mma(S0{});
    __builtin_amdgcn_sched_barrier(0);
    wait(S1{});
    if (k + 1 < KT) {
      // Stage k + 1 has landed for every wave, and every wave has read stage k: its buffer
      // takes stage k + 2.
      wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      if (k + 2 < KT) issue(k + 2);
      read(S0{}, sb ^ kStage64, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma(S1{});
    __builtin_amdgcn_sched_barrier(0);
    if (k + 1 < KT) wait(S0{});
  }
  __syncthreads();  // the epilogues reuse the LDS
}

__device__ __forceinline__ void mainloop(const GemmArgs& g, const Tile& tl, char* smem,
                                         f32x16 (&acc)[kMT][4]) {
  mainloop_t<4>(g, tl, smem, acc);
}

__device__ __forceinline__ void mainloop(const GemmArgs& g, const Tile& tl, char* smem,
                                         f32x16 (&acc)[kMT][2]) {
  mainloop_k64<8, false>(g, tl, smem, acc);
}

// The eight-wave mainloop with B stored [K, ldb] N-contiguous.
__device__ __forceinline__ void mainloop_kn(const GemmArgs& g, const Tile& tl, char* smem,
                                            f32x16 (&acc)[kMT][2]) {
  mainloop_k64<8, true>(g, tl, smem, acc);
}

// Eight waves (two per SIMD): the accumulators of a 128 x 64 wave tile leave room for a second
// wave per SIMD, whose MFMAs run while the first waits on its fragment reads and copies.
constexpr int kThreads8 = 512;

int launch_grid(const GemmArgs& g) {
  const int total = g.tiles_m * g.tiles_n * g.splits;
  return 8 * ((total + 7) / 8);
}

int check_operand(const char* fn, const void* p, int64_t ld, const char* name) {
  if (!p) return fail(RUS_ERR_INVALID, "%s: %s is null", fn, name);
  if (!aligned(p, 16) || ld % 8)
    return fail(RUS_ERR_INVALID, "%s: %s must be 16-byte aligned with a row stride multiple of 8",
                fn, name);
  return RUS_OK;
}

}  // namespace
}  // namespace rus
