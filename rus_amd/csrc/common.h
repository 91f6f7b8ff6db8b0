// Shared helpers for the gfx950 kernels: vector types, typed vector loads/stores, wave64
// reductions, argument checking and error reporting for the C ABI (include/rus_amd.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rus_amd.h"

namespace rus {

typedef _Float16 f16;
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------------------------
// Error reporting (thread-local message, see rus_last_error()).
// ---------------------------------------------------------------------------------------------
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Checks hipGetLastError() after a launch; returns RUS_OK or RUS_ERR_LAUNCH.
int check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---------------------------------------------------------------------------------------------
// Typed vector access: N elements of T moved as one aligned access (16 bytes for f16x8 / f32x4).
// ---------------------------------------------------------------------------------------------
// Alignment is capped at 16 bytes: callers guarantee 16-byte (or pack-size) aligned addresses, and
// wider packs are moved as several 16-byte accesses.
template <typename T, int N>
struct alignas(sizeof(T) * N > 16 ? 16 : sizeof(T) * N) Pack {
  T v[N];
};

// Packs of 16 / 8 / 4 bytes move as one vector access of that width (the pack bit-cast to a
// 32-bit-lane vector): a struct copy is a memcpy to the compiler, which it may split into 2-, 4-
// and 8-byte pieces where control flow merges two stores of the same pack.
typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2s __attribute__((ext_vector_type(2)));

template <int BYTES>
struct VecOf {
  typedef Pack<uint16_t, BYTES / 2> type;  // 2-byte packs (single fp16 elements)
};
template <>
struct VecOf<16> {
  typedef u32x4s type;
};
template <>
struct VecOf<8> {
  typedef u32x2s type;
};
template <>
struct VecOf<4> {
  typedef uint32_t type;
};

template <typename T, int N>
__device__ __forceinline__ Pack<T, N> load_pack(const T* __restrict__ p) {
  constexpr int B = sizeof(Pack<T, N>);
  constexpr int C = B > 16 ? 16 : B;  // bytes per access: packs above 16 bytes go in 16-byte parts
  typedef typename VecOf<C>::type V;
  static_assert(sizeof(V) == C && B % C == 0, "whole accesses per pack");
  const V* src = static_cast<const V*>(__builtin_assume_aligned(p, alignof(Pack<T, N>)));
  V v[B / C];
#pragma unroll
  for (int k = 0; k < B / C; ++k) v[k] = src[k];
  return __builtin_bit_cast(Pack<T, N>, v);
}

template <typename T, int N>
__device__ __forceinline__ void store_pack(T* __restrict__ p, const Pack<T, N>& t) {
  constexpr int B = sizeof(Pack<T, N>);
  constexpr int C = B > 16 ? 16 : B;
  typedef typename VecOf<C>::type V;
  static_assert(sizeof(V) == C && B % C == 0, "whole accesses per pack");
  struct Parts {
    V v[B / C];
  };
  const Parts parts = __builtin_bit_cast(Parts, t);
  V* dst = static_cast<V*>(__builtin_assume_aligned(p, alignof(Pack<T, N>)));
#pragma unroll
  for (int k = 0; k < B / C; ++k) dst[k] = parts.v[k];
}

template <typename T, int N>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float (&out)[N]) {
  const Pack<T, N> t = load_pack<T, N>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = static_cast<float>(t.v[i]);
}

// fp32 -> T (round to nearest even) of the fp32 value x as it stands. The empty asm makes x
// opaque: without it the compiler may fold a preceding fp32 product into the conversion as a
// mixed-precision FMA (v_fma_mixlo_f16), which rounds the exact product once to fp16 instead of
// first to fp32 and then to fp16 — a different result in rare halfway cases.
template <typename T>
__device__ __forceinline__ T from_f32(float x) {
  if constexpr (sizeof(T) < sizeof(float)) asm("" : "+v"(x));
  return static_cast<T>(x);
}

template <typename T, int N>
__device__ __forceinline__ void store_from_f32(T* __restrict__ p, const float (&in)[N]) {
  Pack<T, N> t;
#pragma unroll
  for (int i = 0; i < N; ++i) t.v[i] = from_f32<T>(in[i]);
  store_pack<T, N>(p, t);
}

// 16-byte load with the non-temporal hint (global_load_dwordx4 ... nt), for inputs a launch reads
// exactly once: their lines are not kept, so they do not displace the lines of the launch's
// write stream. A SwiGLU forward over [8192, 17920] fp16 streams 0.68 of 8 TB/s with plain loads
// and 0.79 with the hint on MI355X. Stores stay plain: the next launch reads a launch's outputs,
// and non-temporal stores, which keep the lines out of the last-level cache, made the training
// step slower (0.6-1.5%) although they raised isolated streaming rates.
template <typename T, int N>
__device__ __forceinline__ void load_f32_stream(const T* __restrict__ p, float (&out)[N]) {
  static_assert((sizeof(T) * N) % 16 == 0, "whole 16-byte packs");
  constexpr int E = 16 / sizeof(T);  // elements per 16-byte pack
#pragma unroll
  for (int c = 0; c < N / E; ++c) {
    const u32x4s w = __builtin_nontemporal_load(reinterpret_cast<const u32x4s*>(p) + c);
    const Pack<T, E> t = __builtin_bit_cast(Pack<T, E>, w);
#pragma unroll
    for (int i = 0; i < E; ++i) out[c * E + i] = static_cast<float>(t.v[i]);
  }
}

// load_f32_stream for whole 16-byte packs, load_f32 otherwise (narrower packs of odd widths).
template <typename T, int N>
__device__ __forceinline__ void load_f32_once(const T* __restrict__ p, float (&out)[N]) {
  if constexpr ((sizeof(T) * N) % 16 == 0)
    load_f32_stream<T, N>(p, out);
  else
    load_f32<T, N>(p, out);
}

// Round through the storage type (fp32 -> T -> fp32), i.e. what a T-typed intermediate holds.
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return static_cast<float>(from_f32<T>(x));
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// ---------------------------------------------------------------------------------------------
// Cross-block sums in one launch ("last block reduces"). Blocks store fp32 partials with
// device-coherent 4-byte accesses (agent-scope relaxed atomics: performed where every XCD's L2
// agrees, so no cache-wide write-back or invalidate is needed, which is what a device-scope
// fence would cost), count their arrival on an int32 counter, and the last of n blocks to arrive
// reads all n partials and sums them in a fixed order: deterministic, no atomics on data.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ void store_partial(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float load_partial(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Called by every thread of a block once its partial stores are issued: true, in every thread,
// in the last of the n blocks sharing `counter` to arrive. Each thread waits for its own memory
// accesses to complete before the block arrives; the last block puts the counter back to 0
// (counters are zero when a launch starts and are left zero). No block waits for another.
// The block's verdict travels through `flag`, an int of LDS that no thread touches from the call
// until it returns (callers whose LDS is full pass a word of memory they are done with).
__device__ __forceinline__ bool arrive_last_at(int* counter, int n, int* flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);  // every memory access of this thread has completed
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == n - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last ? 1 : 0;
  }
  __syncthreads();
  return *flag != 0;
}

__device__ __forceinline__ bool arrive_last(int* counter, int n) {
  __shared__ int s_last;
  return arrive_last_at(counter, n, &s_last);
}

}  // namespace rus
