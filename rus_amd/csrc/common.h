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

template <typename T, int N>
__device__ __forceinline__ void load_f32(const T* __restrict__ p, float (&out)[N]) {
  const Pack<T, N> t = *reinterpret_cast<const Pack<T, N>*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = static_cast<float>(t.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void store_from_f32(T* __restrict__ p, const float (&in)[N]) {
  Pack<T, N> t;
#pragma unroll
  for (int i = 0; i < N; ++i) t.v[i] = static_cast<T>(in[i]);
  *reinterpret_cast<Pack<T, N>*>(p) = t;
}

// Round through the storage type (fp32 -> T -> fp32), i.e. what a T-typed intermediate holds.
template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return static_cast<float>(static_cast<T>(x));
}

// Sum over the 64 lanes of a wavefront; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

}  // namespace rus
