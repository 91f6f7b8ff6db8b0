// LoRA-delta add + NeoX rotary embedding (forward) and its adjoint with [dQ | dK | dV] packing
// (backward) for gfx950.
//
// Behaviour follows solution/kernels.py:206-348 (qkv_lora_rope_fwd_kernel,
// qkv_lora_rope_bwd_kernel) and the LoRA-gradient scaling of solution/ops.py:144-147: NeoX pairs
// element j with j + head_dim/2 of the same head, cos/sin rows are indexed by each token's
// position, and outputs are token-major [n_tokens, heads, head_dim]. Design (CDNA4, wave64):
//   * one thread owns 8 consecutive elements of the low half of one head and the matching 8 of
//     the high half (two 16-byte fp16 accesses each way); threads are numbered token-major, then
//     head, then column, so each wave access covers whole 128-byte lines of consecutive heads;
//   * Q, K and V heads of a token are all handled in the same launch (one pass over qkv, q_lora,
//     v_lora), and the backward also emits the scaled LoRA gradients from the rounded packed
//     values, which the reference computes with two extra elementwise launches;
//   * positions are clamped into the cos/sin table, so a bad position can never read out of
//     bounds; an optional device flag records that it happened;
//   * built with -ffp-contract=off: products and sums round exactly as an eager fp32 restatement.
#include "common.h"

namespace rus {
namespace {

constexpr int kThreads = 256;
constexpr int kSpan = 8;  // elements per thread in each half of a head
constexpr int kMaxMidHead = 256;  // largest head_dim of the in-kernel LoRA delta (B rows in LDS)

__device__ __forceinline__ int64_t clamp_pos(const int64_t* __restrict__ pos, int64_t t,
                                             int64_t n_pos, int32_t* err_flag) {
  int64_t p = pos[t];
  if (p < 0 || p >= n_pos) {
    if (err_flag) *err_flag = 1;
    p = p < 0 ? 0 : n_pos - 1;
  }
  return p;
}

template <typename T>
struct RopeFwdArgs {
  const T* qkv;
  const T* q_lora;
  const T* v_lora;
  const T* cos;
  const T* sin;
  const int64_t* pos;
  T* q_out;
  T* k_out;
  T* v_out;
  int64_t n_tokens, stride_qkv, stride_ql, stride_vl, stride_cos, n_pos;
  float scale_q, scale_v;
  int h_q, h_kv, head_dim;
  int32_t* err_flag;
  // LoRA from the rank-r factors instead (fp16 only): delta = fp16(mid[t] . B[col]), mid [N, r],
  // B [cols, r] row-major.
  const T* mid_q;
  const T* mid_v;
  const T* b_q;
  const T* b_v;
};

// Row slot of B row c in the LDS copy: rows permuted within each group of 8 (low three bits
// XORed with the group's index mod 8). The eight lanes of a wave that read at one step take rows
// 8 apart (columns col0 + i, col0 = 8 j), which the plain layout puts in the same banks; the
// permutation spreads them over eight bank groups. A bijection on each group: same values.
__device__ __forceinline__ int b_slot(int c) { return (c & ~7) | ((c & 7) ^ ((c >> 3) & 7)); }

// The LoRA delta of columns col0 .. col0+7 and col0+half .. +7 from mid row m and B [cols, R]
// (rows in b_slot order): fp16(sum_k m[k] * B[col, k]), the reference's fp16 mid B^T product
// (ops.py:776-778).
template <typename T, int R>
__device__ __forceinline__ void lora_up(const float (&m)[R], const T* __restrict__ b, int col0,
                                        int half, float (&dl)[kSpan], float (&dh)[kSpan]) {
#pragma unroll
  for (int i = 0; i < kSpan; ++i) {
    float bl[R], bh[R];
    load_f32<T, R>(b + b_slot(col0 + i) * R, bl);
    load_f32<T, R>(b + b_slot(col0 + half + i) * R, bh);
    float sl = 0.0f, sh = 0.0f;
#pragma unroll
    for (int k = 0; k < R; ++k) {
      sl = __builtin_fmaf(m[k], bl[k], sl);
      sh = __builtin_fmaf(m[k], bh[k], sh);
    }
    dl[i] = round_to<T>(sl);
    dh[i] = round_to<T>(sh);
  }
}

// LORA: 0 none, 1 precomputed q_lora / v_lora rows, 2 rank-R factors (mid, B).
template <typename T, int LORA, int R>
__global__ __launch_bounds__(kThreads) void rope_fwd_kernel(RopeFwdArgs<T> a) {
  constexpr bool HAS_LORA = LORA == 1;
  const int half = a.head_dim / 2;
  const int per_head = half / kSpan;
  // Head-major blocks: one head x kThreads / per_head tokens, so a block touches one head's
  // rows of the LoRA factor B (L1-resident) instead of all of them.
  const int tpb = kThreads / per_head;
  const int64_t n_tiles = (a.n_tokens + tpb - 1) / tpb;
  const int hd = static_cast<int>(blockIdx.x / n_tiles);
  const int64_t t = (blockIdx.x - hd * n_tiles) * tpb + threadIdx.x / per_head;
  const int j = (threadIdx.x % per_head) * kSpan;
  // LORA == 2: this head's rows of B (head_dim x R fp16) staged in LDS once per block.
  __shared__ __attribute__((aligned(16))) T s_b[LORA == 2 ? kMaxMidHead * R : 1];
  if constexpr (LORA == 2) {
    const T* bsrc = nullptr;
    if (hd < a.h_q)
      bsrc = a.b_q + static_cast<int64_t>(hd) * a.head_dim * R;
    else if (hd >= a.h_q + a.h_kv)
      bsrc = a.b_v + static_cast<int64_t>(hd - a.h_q - a.h_kv) * a.head_dim * R;
    if (bsrc) {
      const int n4 = a.head_dim * R / 4;  // 8-byte chunks (B is 8-byte aligned), R / 4 per row
      for (int c = threadIdx.x; c < n4; c += kThreads) {
        const int row = c / (R / 4), part = c - row * (R / 4);
        reinterpret_cast<uint2*>(s_b)[b_slot(row) * (R / 4) + part] =
            reinterpret_cast<const uint2*>(bsrc)[c];
      }
    }
    __syncthreads();
  }
  if (t >= a.n_tokens || static_cast<int>(threadIdx.x) >= tpb * per_head) return;

  float lo[kSpan], hi[kSpan];
  const T* row = a.qkv + t * a.stride_qkv + static_cast<int64_t>(hd) * a.head_dim;
  load_f32<T, kSpan>(row + j, lo);
  load_f32<T, kSpan>(row + j + half, hi);

  // Every head kind ends at the one pair of stores below: with a store site per branch the
  // compiler merged the branches' stores and split them into 2-, 4- and 8-byte pieces.
  const bool is_v = hd >= a.h_q + a.h_kv, is_q = hd < a.h_q;
  float ol[kSpan], oh[kSpan];
  T* o;
  if (is_v) {  // V head: LoRA delta only
    const int kv = hd - a.h_q - a.h_kv;
    if constexpr (LORA == 2) {
      float m[R], dl[kSpan], dh[kSpan];
      load_f32<T, R>(a.mid_v + t * R, m);
      lora_up<T, R>(m, s_b, j, half, dl, dh);
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
        lo[i] = lo[i] + dl[i] * a.scale_v;
        hi[i] = hi[i] + dh[i] * a.scale_v;
      }
    }
    if (HAS_LORA) {
      float dl[kSpan], dh[kSpan];
      const T* vl = a.v_lora + t * a.stride_vl + static_cast<int64_t>(kv) * a.head_dim;
      load_f32<T, kSpan>(vl + j, dl);
      load_f32<T, kSpan>(vl + j + half, dh);
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
        lo[i] = lo[i] + dl[i] * a.scale_v;
        hi[i] = hi[i] + dh[i] * a.scale_v;
      }
    }
#pragma unroll
    for (int i = 0; i < kSpan; ++i) {
      ol[i] = lo[i];
      oh[i] = hi[i];
    }
    o = a.v_out + (t * a.h_kv + kv) * a.head_dim;
  } else {
    if constexpr (LORA == 2) {
      if (is_q) {
        float m[R], dl[kSpan], dh[kSpan];
        load_f32<T, R>(a.mid_q + t * R, m);
        lora_up<T, R>(m, s_b, j, half, dl, dh);
#pragma unroll
        for (int i = 0; i < kSpan; ++i) {
          lo[i] = lo[i] + dl[i] * a.scale_q;
          hi[i] = hi[i] + dh[i] * a.scale_q;
        }
      }
    }
    if (HAS_LORA && is_q) {
      float dl[kSpan], dh[kSpan];
      const T* ql = a.q_lora + t * a.stride_ql + static_cast<int64_t>(hd) * a.head_dim;
      load_f32<T, kSpan>(ql + j, dl);
      load_f32<T, kSpan>(ql + j + half, dh);
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
        lo[i] = lo[i] + dl[i] * a.scale_q;
        hi[i] = hi[i] + dh[i] * a.scale_q;
      }
    }
    const int64_t p = clamp_pos(a.pos, t, a.n_pos, a.err_flag);
    float cl[kSpan], ch[kSpan], sl[kSpan], sh[kSpan];
    const T* cr = a.cos + p * a.stride_cos;
    const T* sr = a.sin + p * a.stride_cos;
    load_f32<T, kSpan>(cr + j, cl);
    load_f32<T, kSpan>(cr + j + half, ch);
    load_f32<T, kSpan>(sr + j, sl);
    load_f32<T, kSpan>(sr + j + half, sh);
#pragma unroll
    for (int i = 0; i < kSpan; ++i) {
      ol[i] = lo[i] * cl[i] - hi[i] * sl[i];
      oh[i] = hi[i] * ch[i] + lo[i] * sh[i];
    }
    o = is_q ? a.q_out + (t * a.h_q + hd) * a.head_dim
             : a.k_out + (t * a.h_kv + (hd - a.h_q)) * a.head_dim;
  }
  store_from_f32<T, kSpan>(o + j, ol);
  store_from_f32<T, kSpan>(o + j + half, oh);
}

template <typename T>
struct RopeBwdArgs {
  const T* dq;
  const T* dk;
  const T* dv;
  const T* cos;
  const T* sin;
  const int64_t* pos;
  T* dqkv;
  T* dq_lora;
  T* dv_lora;
  int64_t n_tokens, stride_dqkv, stride_cos, n_pos;
  float scale_q, scale_v;
  int h_q, h_kv, head_dim;
  int32_t* err_flag;
};

template <typename T, bool LORA_OUT>
__global__ __launch_bounds__(kThreads) void rope_bwd_kernel(RopeBwdArgs<T> a) {
  const int half = a.head_dim / 2;
  const int per_head = half / kSpan;
  const int heads = a.h_q + 2 * a.h_kv;
  const int slots = heads * per_head;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t t = gid / slots;
  if (t >= a.n_tokens) return;
  const int slot = static_cast<int>(gid - t * slots);
  const int hd = slot / per_head;
  const int j = (slot - hd * per_head) * kSpan;
  T* out = a.dqkv + t * a.stride_dqkv + static_cast<int64_t>(hd) * a.head_dim;

  // One store site per output for every head kind (see rope_fwd_kernel).
  const bool is_v = hd >= a.h_q + a.h_kv, is_q = hd < a.h_q;
  const T* src = is_v ? a.dv + (t * a.h_kv + (hd - a.h_q - a.h_kv)) * a.head_dim
                 : is_q ? a.dq + (t * a.h_q + hd) * a.head_dim
                        : a.dk + (t * a.h_kv + (hd - a.h_q)) * a.head_dim;
  float lo[kSpan], hi[kSpan], ol[kSpan], oh[kSpan];
  load_f32<T, kSpan>(src + j, lo);
  load_f32<T, kSpan>(src + j + half, hi);
  if (is_v) {  // dV: copied (and scaled into dv_lora)
#pragma unroll
    for (int i = 0; i < kSpan; ++i) {
      ol[i] = lo[i];
      oh[i] = hi[i];
    }
  } else {
    const int64_t p = clamp_pos(a.pos, t, a.n_pos, a.err_flag);
    float cl[kSpan], ch[kSpan], sl[kSpan], sh[kSpan];
    const T* cr = a.cos + p * a.stride_cos;
    const T* sr = a.sin + p * a.stride_cos;
    load_f32<T, kSpan>(cr + j, cl);
    load_f32<T, kSpan>(cr + j + half, ch);
    load_f32<T, kSpan>(sr + j, sl);
    load_f32<T, kSpan>(sr + j + half, sh);
#pragma unroll
    for (int i = 0; i < kSpan; ++i) {
      ol[i] = round_to<T>(lo[i] * cl[i] + hi[i] * sh[i]);
      oh[i] = round_to<T>(hi[i] * ch[i] - lo[i] * sl[i]);
    }
  }
  store_from_f32<T, kSpan>(out + j, ol);
  store_from_f32<T, kSpan>(out + j + half, oh);
  if (LORA_OUT && (is_v || is_q)) {
    const float sc = is_v ? a.scale_v : a.scale_q;
#pragma unroll
    for (int i = 0; i < kSpan; ++i) {
      ol[i] = ol[i] * sc;
      oh[i] = oh[i] * sc;
    }
    T* l = is_v ? a.dv_lora + (t * a.h_kv + (hd - a.h_q - a.h_kv)) * a.head_dim
                : a.dq_lora + (t * a.h_q + hd) * a.head_dim;
    store_from_f32<T, kSpan>(l + j, ol);
    store_from_f32<T, kSpan>(l + j + half, oh);
  }
}

// rope_bwd_kernel<f16, true> that also forms the rank-R LoRA products of its outputs:
// d_mid_q = fp16(dq_lora B_q) [N, R] and d_mid_v = fp16(dv_lora B_v) (solution/ops.py:975-992,
// d_mid = dq @ B), with B given rank-major (bt = B^T [R, d]). A block holds whole tokens (every
// slot of a token), so the reductions over a token's columns stay in the block: each thread
// forms R partial sums over its 16 elements, a 16-lane transpose reduction leaves one rank per
// lane, and the per-token merge of the 16-lane groups (all of one kind: the slot ranges of the
// q, k and v heads are multiples of 16) runs in group order through LDS.
struct RopeBwdMidArgs {
  RopeBwdArgs<f16> b;
  const f16* bt_q;  // [R, h_q * head_dim]
  const f16* bt_v;  // [R, h_kv * head_dim]
  f16* dmid_q;      // [N, R]
  f16* dmid_v;
  // Non-null: dK and dV come as the attention backward's fp32 per-query-head partials
  // [h_q, N, head_dim] (b.dk / b.dv unused), each KV group's heads summed here.
  const float* dk_part;
  const float* dv_part;
};

constexpr int kMaxGroupSum = 8;  // query heads per KV head the partial sums support

// dK or dV values c .. c + kSpan of KV head kv, token t, from the per-query-head partials: the
// group's h_q / h_kv heads added in head order in fp32, rounded to fp16 once (the values the
// attention backward's own group sum writes).
__device__ __forceinline__ void load_group_sum(const float* __restrict__ part, int kv, int grp,
                                               int64_t n_tok, int64_t t, int c, int head_dim,
                                               float (&out)[kSpan]) {
  const float* p = part + (static_cast<int64_t>(kv) * grp * n_tok + t) * head_dim + c;
  const int64_t hs = n_tok * head_dim;
  float v[kMaxGroupSum][kSpan];
#pragma unroll
  for (int j = 0; j < kMaxGroupSum; ++j)
    if (j < grp) load_f32<float, kSpan>(p + j * hs, v[j]);
#pragma unroll
  for (int i = 0; i < kSpan; ++i) {
    float acc = v[0][i];
#pragma unroll
    for (int j = 1; j < kMaxGroupSum; ++j)
      if (j < grp) acc += v[j][i];
    out[i] = round_to<f16>(acc);
  }
}

constexpr int kMidR = 16;  // rank of the fused d_mid products

// p (16 values per lane) -> lane l holds the sum of p[l % 16] over its 16-lane group.
__device__ __forceinline__ float group16_transpose_sum(const float (&p)[16], int lane) {
  float v8[8], v4[4], v2[2];
  const bool b3 = lane & 8, b2 = lane & 4, b1 = lane & 2, b0 = lane & 1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float send = b3 ? p[i] : p[i + 8];
    v8[i] = (b3 ? p[i + 8] : p[i]) + __shfl_xor(send, 8);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float send = b2 ? v8[i] : v8[i + 4];
    v4[i] = (b2 ? v8[i + 4] : v8[i]) + __shfl_xor(send, 4);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float send = b1 ? v4[i] : v4[i + 2];
    v2[i] = (b1 ? v4[i + 2] : v4[i]) + __shfl_xor(send, 2);
  }
  const float send = b0 ? v2[0] : v2[1];
  return (b0 ? v2[1] : v2[0]) + __shfl_xor(send, 1);
}

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

// p[r] += sum_i lo[i] bt[r][c + i] + hi[i] bt[r][c + half + i], the B^T fragments loaded rank by
// rank (holding all sixteen ranks' fragments at once took 213 VGPRs, two waves per SIMD).
__device__ __forceinline__ void mid_partial(float (&p)[kMidR], const float (&lo)[kSpan],
                                                     const float (&hi)[kSpan],
                                                     const f16* __restrict__ bt, int64_t d,
                                                     int64_t c, int half) {
#pragma unroll
  for (int r = 0; r < kMidR; ++r) {
    const f16x8_t bl = *reinterpret_cast<const f16x8_t*>(bt + r * d + c);
    const f16x8_t bh = *reinterpret_cast<const f16x8_t*>(bt + r * d + c + half);
#pragma unroll
    for (int i = 0; i < kSpan; ++i)
      p[r] += lo[i] * static_cast<float>(bl[i]) + hi[i] * static_cast<float>(bh[i]);
  }
}

__global__ __launch_bounds__(kThreads) void rope_bwd_mid_kernel(RopeBwdMidArgs m) {
  const RopeBwdArgs<f16>& a = m.b;
  const int half = a.head_dim / 2;
  const int per_head = half / kSpan;
  const int heads = a.h_q + 2 * a.h_kv;
  const int slots = heads * per_head;  // divides kThreads, multiple of 16 (host-checked)
  const int tpb = kThreads / slots;
  const int tb = threadIdx.x / slots;
  const int slot = threadIdx.x - tb * slots;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * tpb;
  const int64_t t = t0 + tb;
  const int hd = slot / per_head;
  const int j = (slot - hd * per_head) * kSpan;
  const int lane = threadIdx.x & 63;
  const int64_t d_q = static_cast<int64_t>(a.h_q) * a.head_dim;
  const int64_t d_v = static_cast<int64_t>(a.h_kv) * a.head_dim;

  float p[kMidR];
#pragma unroll
  for (int r = 0; r < kMidR; ++r) p[r] = 0.0f;
  const bool is_q = hd < a.h_q, is_v = hd >= a.h_q + a.h_kv;
  const f16* bt = is_q ? m.bt_q : m.bt_v;
  const int64_t bd = is_q ? d_q : d_v;
  const int64_t bc = static_cast<int64_t>(is_q ? hd : hd - a.h_q - a.h_kv) * a.head_dim + j;
  if (t < a.n_tokens) {
    // One store site per output for every head kind (see rope_fwd_kernel).
    f16* out = a.dqkv + t * a.stride_dqkv + static_cast<int64_t>(hd) * a.head_dim;
    const int kv = is_v ? hd - a.h_q - a.h_kv : hd - a.h_q;  // KV head of a k / v slot
    float lo[kSpan], hi[kSpan], ol[kSpan], oh[kSpan];
    const float* part = is_v ? m.dv_part : is_q ? nullptr : m.dk_part;
    if (part) {  // dK / dV from the attention backward's per-query-head partials
      const int grp = a.h_q / a.h_kv;
      load_group_sum(part, kv, grp, a.n_tokens, t, j, a.head_dim, lo);
      load_group_sum(part, kv, grp, a.n_tokens, t, j + half, a.head_dim, hi);
    } else {
      const f16* src = is_v ? a.dv + (t * a.h_kv + kv) * a.head_dim
                       : is_q ? a.dq + (t * a.h_q + hd) * a.head_dim
                              : a.dk + (t * a.h_kv + kv) * a.head_dim;
      load_f32<f16, kSpan>(src + j, lo);
      load_f32<f16, kSpan>(src + j + half, hi);
    }
    if (is_v) {  // dV: copied
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
        ol[i] = lo[i];
        oh[i] = hi[i];
      }
    } else {
      const int64_t ps = clamp_pos(a.pos, t, a.n_pos, a.err_flag);
      float cl[kSpan], ch[kSpan], sl[kSpan], sh[kSpan];
      const f16* cr = a.cos + ps * a.stride_cos;
      const f16* sr = a.sin + ps * a.stride_cos;
      load_f32<f16, kSpan>(cr + j, cl);
      load_f32<f16, kSpan>(cr + j + half, ch);
      load_f32<f16, kSpan>(sr + j, sl);
      load_f32<f16, kSpan>(sr + j + half, sh);
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
        ol[i] = round_to<f16>(lo[i] * cl[i] + hi[i] * sh[i]);
        oh[i] = round_to<f16>(hi[i] * ch[i] - lo[i] * sl[i]);
      }
    }
    store_from_f32<f16, kSpan>(out + j, ol);
    store_from_f32<f16, kSpan>(out + j + half, oh);
    if (is_v || is_q) {  // the scaled LoRA gradient rows and their d_mid partials
      const float sc = is_v ? a.scale_v : a.scale_q;
#pragma unroll
      for (int i = 0; i < kSpan; ++i) {
        ol[i] = round_to<f16>(ol[i] * sc);  // the stored dq_lora / dv_lora values
        oh[i] = round_to<f16>(oh[i] * sc);
      }
      f16* l = is_v ? a.dv_lora + (t * a.h_kv + kv) * a.head_dim
                    : a.dq_lora + (t * a.h_q + hd) * a.head_dim;
      store_from_f32<f16, kSpan>(l + j, ol);
      store_from_f32<f16, kSpan>(l + j + half, oh);
      mid_partial(p, ol, oh, bt, bd, bc, half);
    }
  }
  __shared__ float red[kThreads / 16][kMidR];
  red[threadIdx.x >> 4][threadIdx.x & 15] = group16_transpose_sum(p, lane);
  __syncthreads();
  const int groups = slots / 16;
  const int gq = a.h_q * per_head / 16, gv0 = (a.h_q + a.h_kv) * per_head / 16;
  if (threadIdx.x < tpb * 2 * kMidR) {
    const int tk = threadIdx.x / (2 * kMidR), rr = threadIdx.x % (2 * kMidR);
    const int64_t tt = t0 + tk;
    if (tt < a.n_tokens) {
      const bool out_q = rr < kMidR;
      const int r = out_q ? rr : rr - kMidR;
      float acc = 0.0f;
      for (int g = out_q ? 0 : gv0; g < (out_q ? gq : groups); ++g) acc += red[tk * groups + g][r];
      (out_q ? m.dmid_q : m.dmid_v)[tt * kMidR + r] = from_f32<f16>(acc);
    }
  }
}

int check_heads(const char* fn, int64_t n_tokens, int32_t h_q, int32_t h_kv, int32_t head_dim,
                int64_t n_pos, int64_t stride_cos, int32_t dtype) {
  if (dtype != RUS_DTYPE_F16 && dtype != RUS_DTYPE_F32)
    return fail(RUS_ERR_INVALID, "%s: dtype %d not fp16(0)/fp32(1)", fn, dtype);
  if (n_tokens < 0 || n_tokens >= (int64_t(1) << 31))
    return fail(RUS_ERR_INVALID, "%s: n_tokens=%lld", fn, (long long)n_tokens);
  if (h_q <= 0 || h_kv <= 0 || head_dim <= 0 || head_dim % (2 * kSpan) ||
      head_dim > 2 * kSpan * kThreads)
    return fail(RUS_ERR_INVALID, "%s: h_q=%d h_kv=%d head_dim=%d (multiple of 16 required)", fn,
                h_q, h_kv, head_dim);
  if (n_pos <= 0 || stride_cos < head_dim)
    return fail(RUS_ERR_INVALID, "%s: cos/sin table [%lld, stride %lld] too small", fn,
                (long long)n_pos, (long long)stride_cos);
  return RUS_OK;
}

// Every pointer and row stride must allow 16-byte (fp16: 8 elements) accesses at element offsets
// that are multiples of 8.
template <typename T>
bool aligned8(const void* p, int64_t stride) {
  return p == nullptr || (aligned(p, 16) && (stride * static_cast<int64_t>(sizeof(T))) % 16 == 0);
}

template <typename T>
int fwd_typed(const RopeFwdArgs<T>& a, hipStream_t st) {
  if (!aligned8<T>(a.qkv, a.stride_qkv) || !aligned8<T>(a.q_lora, a.stride_ql) ||
      !aligned8<T>(a.v_lora, a.stride_vl) || !aligned8<T>(a.cos, a.stride_cos) ||
      !aligned8<T>(a.sin, a.stride_cos) || !aligned(a.q_out, 16) || !aligned(a.k_out, 16) ||
      !aligned(a.v_out, 16))
    return fail(RUS_ERR_INVALID, "rus_qkv_lora_rope_fwd: pointers/strides must be 16-byte aligned");
  const int64_t tpb = kThreads / (a.head_dim / 2 / kSpan);  // tokens per head-major block
  const dim3 grid(static_cast<unsigned>((a.h_q + 2 * a.h_kv) * ((a.n_tokens + tpb - 1) / tpb)));
  if (a.q_lora)
    hipLaunchKernelGGL((rope_fwd_kernel<T, 1, 0>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((rope_fwd_kernel<T, 0, 0>), grid, dim3(kThreads), 0, st, a);
  return check_launch("rus_qkv_lora_rope_fwd");
}

int fwd_mid(const RopeFwdArgs<f16>& a, int r, hipStream_t st) {
  const char* fn = "rus_qkv_lora_rope_fwd_mid";
  if (!aligned8<f16>(a.qkv, a.stride_qkv) || !aligned8<f16>(a.cos, a.stride_cos) ||
      !aligned8<f16>(a.sin, a.stride_cos) || !aligned(a.q_out, 16) || !aligned(a.k_out, 16) ||
      !aligned(a.v_out, 16) || !aligned(a.mid_q, 8) || !aligned(a.mid_v, 8) ||
      !aligned(a.b_q, 8) || !aligned(a.b_v, 8))
    return fail(RUS_ERR_INVALID, "%s: pointers/strides must be aligned (16 B rows, 8 B factors)",
                fn);
  if (a.head_dim > kMaxMidHead)
    return fail(RUS_ERR_UNSUPPORTED, "%s: head_dim %d above %d", fn, a.head_dim, kMaxMidHead);
  const int64_t tpb = kThreads / (a.head_dim / 2 / kSpan);  // tokens per head-major block
  const dim3 grid(static_cast<unsigned>((a.h_q + 2 * a.h_kv) * ((a.n_tokens + tpb - 1) / tpb)));
  switch (r) {
    case 4: hipLaunchKernelGGL((rope_fwd_kernel<f16, 2, 4>), grid, dim3(kThreads), 0, st, a); break;
    case 8: hipLaunchKernelGGL((rope_fwd_kernel<f16, 2, 8>), grid, dim3(kThreads), 0, st, a); break;
    case 16: hipLaunchKernelGGL((rope_fwd_kernel<f16, 2, 16>), grid, dim3(kThreads), 0, st, a); break;
    case 32: hipLaunchKernelGGL((rope_fwd_kernel<f16, 2, 32>), grid, dim3(kThreads), 0, st, a); break;
    default: return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d not in {4,8,16,32}", fn, r);
  }
  return check_launch(fn);
}

template <typename T>
int bwd_typed(const RopeBwdArgs<T>& a, hipStream_t st) {
  if (!aligned(a.dq, 16) || !aligned(a.dk, 16) || !aligned(a.dv, 16) ||
      !aligned8<T>(a.cos, a.stride_cos) || !aligned8<T>(a.sin, a.stride_cos) ||
      !aligned8<T>(a.dqkv, a.stride_dqkv) || (a.dq_lora && !aligned(a.dq_lora, 16)) ||
      (a.dv_lora && !aligned(a.dv_lora, 16)))
    return fail(RUS_ERR_INVALID, "rus_qkv_rope_bwd: pointers/strides must be 16-byte aligned");
  const int64_t slots = static_cast<int64_t>(a.h_q + 2 * a.h_kv) * (a.head_dim / 2 / kSpan);
  const int64_t threads = a.n_tokens * slots;
  const dim3 grid(static_cast<unsigned>((threads + kThreads - 1) / kThreads));
  if (a.dq_lora)
    hipLaunchKernelGGL((rope_bwd_kernel<T, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((rope_bwd_kernel<T, false>), grid, dim3(kThreads), 0, st, a);
  return check_launch("rus_qkv_rope_bwd");
}

int bwd_mid(const char* fn, const RopeBwdMidArgs& m, hipStream_t st) {
  const RopeBwdArgs<f16>& a = m.b;
  const int per_head = a.head_dim / 2 / kSpan;
  const int slots = (a.h_q + 2 * a.h_kv) * per_head;
  if (kThreads % slots || slots % 16 || (a.h_q * per_head) % 16 || (a.h_kv * per_head) % 16)
    return fail(RUS_ERR_UNSUPPORTED,
                "%s: h_q=%d h_kv=%d head_dim=%d: a token's slots must divide %d and each head "
                "kind's slots be a multiple of 16", fn, a.h_q, a.h_kv, a.head_dim, kThreads);
  const bool parts = m.dk_part != nullptr;
  if (!aligned(a.dq, 16) || (parts ? !aligned(m.dk_part, 16) : !aligned(a.dk, 16)) ||
      (parts ? !aligned(m.dv_part, 16) : !aligned(a.dv, 16)) ||
      !aligned8<f16>(a.cos, a.stride_cos) || !aligned8<f16>(a.sin, a.stride_cos) ||
      !aligned8<f16>(a.dqkv, a.stride_dqkv) || !aligned(a.dq_lora, 16) ||
      !aligned(a.dv_lora, 16) || !aligned(m.bt_q, 16) || !aligned(m.bt_v, 16))
    return fail(RUS_ERR_INVALID, "%s: pointers/strides must be 16-byte aligned", fn);
  if (parts && a.h_q / a.h_kv > kMaxGroupSum)
    return fail(RUS_ERR_UNSUPPORTED, "%s: %d query heads per KV head (at most %d)", fn,
                a.h_q / a.h_kv, kMaxGroupSum);
  const int64_t tpb = kThreads / slots;
  const dim3 grid(static_cast<unsigned>((a.n_tokens + tpb - 1) / tpb));
  hipLaunchKernelGGL(rope_bwd_mid_kernel, grid, dim3(kThreads), 0, st, m);
  return check_launch(fn);
}

}  // namespace
}  // namespace rus

extern "C" int rus_qkv_lora_rope_fwd(const void* qkv, const void* q_lora, const void* v_lora,
                                     const void* cos, const void* sin, const int64_t* pos_ids,
                                     void* q_out, void* k_out, void* v_out, int64_t n_tokens,
                                     int64_t stride_qkv, int64_t stride_ql, int64_t stride_vl,
                                     int64_t stride_cos, int64_t n_pos, float scale_q,
                                     float scale_v, int32_t h_q, int32_t h_kv, int32_t head_dim,
                                     int32_t* err_flag, int32_t dtype, void* stream) {
  using namespace rus;
  if (int e = check_heads("rus_qkv_lora_rope_fwd", n_tokens, h_q, h_kv, head_dim, n_pos,
                          stride_cos, dtype))
    return e;
  if (n_tokens == 0) return RUS_OK;
  if (!qkv || !cos || !sin || !pos_ids || !q_out || !k_out || !v_out)
    return fail(RUS_ERR_INVALID, "rus_qkv_lora_rope_fwd: null pointer argument");
  if ((q_lora == nullptr) != (v_lora == nullptr))
    return fail(RUS_ERR_INVALID, "rus_qkv_lora_rope_fwd: q_lora and v_lora must both be given");
  const int64_t width = static_cast<int64_t>(h_q + 2 * h_kv) * head_dim;
  if (stride_qkv < width || (q_lora && (stride_ql < int64_t(h_q) * head_dim ||
                                        stride_vl < int64_t(h_kv) * head_dim)))
    return fail(RUS_ERR_INVALID, "rus_qkv_lora_rope_fwd: row strides smaller than rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_ROPE_FWD(T)                                                                          \
  {                                                                                              \
    RopeFwdArgs<T> a{static_cast<const T*>(qkv), static_cast<const T*>(q_lora),                 \
                     static_cast<const T*>(v_lora), static_cast<const T*>(cos),                 \
                     static_cast<const T*>(sin), pos_ids, static_cast<T*>(q_out),               \
                     static_cast<T*>(k_out), static_cast<T*>(v_out), n_tokens, stride_qkv,      \
                     stride_ql, stride_vl, stride_cos, n_pos, scale_q, scale_v, h_q, h_kv,      \
                     head_dim, err_flag};                                                        \
    return fwd_typed<T>(a, st);                                                                  \
  }
  if (dtype == RUS_DTYPE_F16) RUS_ROPE_FWD(f16)
  RUS_ROPE_FWD(float)
#undef RUS_ROPE_FWD
}

extern "C" int rus_qkv_rope_bwd(const void* dq_rot, const void* dk_rot, const void* dv,
                                const void* cos, const void* sin, const int64_t* pos_ids,
                                void* dqkv, void* dq_lora, void* dv_lora, int64_t n_tokens,
                                int64_t stride_dqkv, int64_t stride_cos, int64_t n_pos,
                                float scale_q, float scale_v, int32_t h_q, int32_t h_kv,
                                int32_t head_dim, int32_t* err_flag, int32_t dtype,
                                void* stream) {
  using namespace rus;
  if (int e = check_heads("rus_qkv_rope_bwd", n_tokens, h_q, h_kv, head_dim, n_pos, stride_cos,
                          dtype))
    return e;
  if (n_tokens == 0) return RUS_OK;
  if (!dq_rot || !dk_rot || !dv || !cos || !sin || !pos_ids || !dqkv)
    return fail(RUS_ERR_INVALID, "rus_qkv_rope_bwd: null pointer argument");
  if ((dq_lora == nullptr) != (dv_lora == nullptr))
    return fail(RUS_ERR_INVALID, "rus_qkv_rope_bwd: dq_lora and dv_lora must both be given");
  if (stride_dqkv < static_cast<int64_t>(h_q + 2 * h_kv) * head_dim)
    return fail(RUS_ERR_INVALID, "rus_qkv_rope_bwd: stride_dqkv smaller than a row");
  hipStream_t st = static_cast<hipStream_t>(stream);
#define RUS_ROPE_BWD(T)                                                                         \
  {                                                                                             \
    RopeBwdArgs<T> a{static_cast<const T*>(dq_rot), static_cast<const T*>(dk_rot),             \
                     static_cast<const T*>(dv),     static_cast<const T*>(cos),                \
                     static_cast<const T*>(sin),    pos_ids,                                   \
                     static_cast<T*>(dqkv),         static_cast<T*>(dq_lora),                  \
                     static_cast<T*>(dv_lora),      n_tokens,                                  \
                     stride_dqkv,                   stride_cos,                                \
                     n_pos,                         scale_q,                                   \
                     scale_v,                       h_q,                                       \
                     h_kv,                          head_dim,                                  \
                     err_flag};                                                                 \
    return bwd_typed<T>(a, st);                                                                 \
  }
  if (dtype == RUS_DTYPE_F16) RUS_ROPE_BWD(f16)
  RUS_ROPE_BWD(float)
#undef RUS_ROPE_BWD
}

extern "C" int rus_qkv_lora_rope_fwd_mid(const void* qkv, const void* mid_q, const void* mid_v,
                                         const void* b_q, const void* b_v, int32_t r,
                                         const void* cos, const void* sin,
                                         const int64_t* pos_ids, void* q_out, void* k_out,
                                         void* v_out, int64_t n_tokens, int64_t stride_qkv,
                                         int64_t stride_cos, int64_t n_pos, float scale_q,
                                         float scale_v, int32_t h_q, int32_t h_kv,
                                         int32_t head_dim, int32_t* err_flag, void* stream) {
  using namespace rus;
  const char* fn = "rus_qkv_lora_rope_fwd_mid";
  if (int e = check_heads(fn, n_tokens, h_q, h_kv, head_dim, n_pos, stride_cos, RUS_DTYPE_F16))
    return e;
  if (n_tokens == 0) return RUS_OK;
  if (!qkv || !mid_q || !mid_v || !b_q || !b_v || !cos || !sin || !pos_ids || !q_out || !k_out ||
      !v_out)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (stride_qkv < static_cast<int64_t>(h_q + 2 * h_kv) * head_dim)
    return fail(RUS_ERR_INVALID, "%s: stride_qkv smaller than a row", fn);
  RopeFwdArgs<f16> a{};
  a.qkv = static_cast<const f16*>(qkv);
  a.cos = static_cast<const f16*>(cos);
  a.sin = static_cast<const f16*>(sin);
  a.pos = pos_ids;
  a.q_out = static_cast<f16*>(q_out);
  a.k_out = static_cast<f16*>(k_out);
  a.v_out = static_cast<f16*>(v_out);
  a.n_tokens = n_tokens;
  a.stride_qkv = stride_qkv;
  a.stride_cos = stride_cos;
  a.n_pos = n_pos;
  a.scale_q = scale_q;
  a.scale_v = scale_v;
  a.h_q = h_q;
  a.h_kv = h_kv;
  a.head_dim = head_dim;
  a.err_flag = err_flag;
  a.mid_q = static_cast<const f16*>(mid_q);
  a.mid_v = static_cast<const f16*>(mid_v);
  a.b_q = static_cast<const f16*>(b_q);
  a.b_v = static_cast<const f16*>(b_v);
  return fwd_mid(a, r, static_cast<hipStream_t>(stream));
}

static int rope_bwd_mid_entry(const char* fn, const void* dq_rot, const void* dk_rot,
                              const void* dv, const float* dk_part, const float* dv_part,
                              const void* cos, const void* sin, const int64_t* pos_ids,
                              void* dqkv, void* dq_lora, void* dv_lora, const void* bt_q,
                              const void* bt_v, int32_t r, void* d_mid_q, void* d_mid_v,
                              int64_t n_tokens, int64_t stride_dqkv, int64_t stride_cos,
                              int64_t n_pos, float scale_q, float scale_v, int32_t h_q,
                              int32_t h_kv, int32_t head_dim, int32_t* err_flag, void* stream) {
  using namespace rus;
  if (int e = check_heads(fn, n_tokens, h_q, h_kv, head_dim, n_pos, stride_cos, RUS_DTYPE_F16))
    return e;
  if (r != kMidR) return fail(RUS_ERR_UNSUPPORTED, "%s: rank %d (only %d)", fn, r, kMidR);
  if (n_tokens == 0) return RUS_OK;
  if (!dq_rot || !(dk_rot || dk_part) || !(dv || dv_part) || !cos || !sin || !pos_ids || !dqkv ||
      !dq_lora || !dv_lora || !bt_q || !bt_v || !d_mid_q || !d_mid_v)
    return fail(RUS_ERR_INVALID, "%s: null pointer argument", fn);
  if (stride_dqkv < static_cast<int64_t>(h_q + 2 * h_kv) * head_dim)
    return fail(RUS_ERR_INVALID, "%s: stride_dqkv smaller than a row", fn);
  RopeBwdMidArgs m{};
  m.b = RopeBwdArgs<f16>{static_cast<const f16*>(dq_rot), static_cast<const f16*>(dk_rot),
                         static_cast<const f16*>(dv),     static_cast<const f16*>(cos),
                         static_cast<const f16*>(sin),    pos_ids,
                         static_cast<f16*>(dqkv),         static_cast<f16*>(dq_lora),
                         static_cast<f16*>(dv_lora),      n_tokens,
                         stride_dqkv,                     stride_cos,
                         n_pos,                           scale_q,
                         scale_v,                         h_q,
                         h_kv,                            head_dim,
                         err_flag};
  m.bt_q = static_cast<const f16*>(bt_q);
  m.bt_v = static_cast<const f16*>(bt_v);
  m.dmid_q = static_cast<f16*>(d_mid_q);
  m.dmid_v = static_cast<f16*>(d_mid_v);
  m.dk_part = dk_part;
  m.dv_part = dv_part;
  return bwd_mid(fn, m, static_cast<hipStream_t>(stream));
}

extern "C" int rus_qkv_rope_bwd_mid(const void* dq_rot, const void* dk_rot, const void* dv,
                                    const void* cos, const void* sin, const int64_t* pos_ids,
                                    void* dqkv, void* dq_lora, void* dv_lora, const void* bt_q,
                                    const void* bt_v, int32_t r, void* d_mid_q, void* d_mid_v,
                                    int64_t n_tokens, int64_t stride_dqkv, int64_t stride_cos,
                                    int64_t n_pos, float scale_q, float scale_v, int32_t h_q,
                                    int32_t h_kv, int32_t head_dim, int32_t* err_flag,
                                    void* stream) {
  if (!dk_rot || !dv) return rus::fail(RUS_ERR_INVALID, "rus_qkv_rope_bwd_mid: null pointer argument");
  return rope_bwd_mid_entry("rus_qkv_rope_bwd_mid", dq_rot, dk_rot, dv, nullptr, nullptr, cos,
                            sin, pos_ids, dqkv, dq_lora, dv_lora, bt_q, bt_v, r, d_mid_q,
                            d_mid_v, n_tokens, stride_dqkv, stride_cos, n_pos, scale_q, scale_v,
                            h_q, h_kv, head_dim, err_flag, stream);
}

extern "C" int rus_qkv_rope_bwd_mid_parts(const void* dq_rot, const float* dk_part,
                                          const float* dv_part, const void* cos, const void* sin,
                                          const int64_t* pos_ids, void* dqkv, void* dq_lora,
                                          void* dv_lora, const void* bt_q, const void* bt_v,
                                          int32_t r, void* d_mid_q, void* d_mid_v,
                                          int64_t n_tokens, int64_t stride_dqkv,
                                          int64_t stride_cos, int64_t n_pos, float scale_q,
                                          float scale_v, int32_t h_q, int32_t h_kv,
                                          int32_t head_dim, int32_t* err_flag, void* stream) {
  if (!dk_part || !dv_part)
    return rus::fail(RUS_ERR_INVALID, "rus_qkv_rope_bwd_mid_parts: null pointer argument");
  return rope_bwd_mid_entry("rus_qkv_rope_bwd_mid_parts", dq_rot, nullptr, nullptr, dk_part,
                            dv_part, cos, sin, pos_ids, dqkv, dq_lora, dv_lora, bt_q, bt_v, r,
                            d_mid_q, d_mid_v, n_tokens, stride_dqkv, stride_cos, n_pos, scale_q,
                            scale_v, h_q, h_kv, head_dim, err_flag, stream);
}
