// Error reporting shared by every C-ABI entry point (include/rus_amd.h).
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace rus {

static thread_local char g_error[1024] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(RUS_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  }
  return RUS_OK;
}

}  // namespace rus

extern "C" const char* rus_last_error(void) { return rus::g_error; }

extern "C" int rus_abi_version(void) { return RUS_ABI_VERSION; }

// Node census of a captured graph (diagnostic): counts[t] = number of nodes of hipGraphNodeType t,
// for t < n_counts; types beyond n_counts are added to the last entry.
extern "C" int rus_graph_node_counts(void* graph, int64_t* counts, int32_t n_counts) {
  using namespace rus;
  if (!graph || !counts || n_counts <= 0)
    return fail(RUS_ERR_INVALID, "rus_graph_node_counts: null graph/counts or n_counts <= 0");
  hipGraph_t g = static_cast<hipGraph_t>(graph);
  size_t n = 0;
  hipError_t e = hipGraphGetNodes(g, nullptr, &n);
  if (e != hipSuccess)
    return fail(RUS_ERR_LAUNCH, "rus_graph_node_counts: hipGraphGetNodes: %s", hipGetErrorString(e));
  for (int i = 0; i < n_counts; ++i) counts[i] = 0;
  if (n == 0) return RUS_OK;
  hipGraphNode_t* nodes = new hipGraphNode_t[n];
  e = hipGraphGetNodes(g, nodes, &n);
  int rc = RUS_OK;
  if (e != hipSuccess) {
    rc = fail(RUS_ERR_LAUNCH, "rus_graph_node_counts: hipGraphGetNodes: %s", hipGetErrorString(e));
  } else {
    for (size_t i = 0; i < n; ++i) {
      hipGraphNodeType t;
      e = hipGraphNodeGetType(nodes[i], &t);
      if (e != hipSuccess) {
        rc = fail(RUS_ERR_LAUNCH, "rus_graph_node_counts: hipGraphNodeGetType: %s",
                  hipGetErrorString(e));
        break;
      }
      const int k = static_cast<int>(t) < n_counts ? static_cast<int>(t) : n_counts - 1;
      counts[k] += 1;
    }
  }
  delete[] nodes;
  return rc;
}

namespace rus {
namespace {

// dst[i] = src[i] over 16-byte words, grid-stride; src may be pinned host memory (read over the
// bus by the kernel).
__global__ __launch_bounds__(256) void copy16_kernel(const uint4* __restrict__ src,
                                                     uint4* __restrict__ dst, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * 256)
    dst[i] = src[i];
}

// dst[i, :] = src[ids[i], :] for rows of `words` 16-byte words; src may be pinned host memory
// (each row read over the bus by the kernel). An id outside [0, n_src) yields a zero row and sets
// *err_flag (when given). Block = 4 waves; each wave copies one row at a time.
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint4* __restrict__ src,
                                                          int64_t n_src, int64_t words,
                                                          const int64_t* __restrict__ ids,
                                                          int64_t n_ids, uint4* __restrict__ dst,
                                                          int32_t* err_flag) {
  const int lane = threadIdx.x & 63;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); r < n_ids;
       r += static_cast<int64_t>(gridDim.x) * 4) {
    const int64_t id = ids[r];
    const bool ok = id >= 0 && id < n_src;
    if (!ok && err_flag && lane == 0) *err_flag = 1;
    uint4* d = dst + r * words;
    if (ok) {
      const uint4* s = src + id * words;
      for (int64_t w = lane; w < words; w += 64) d[w] = s[w];
    } else {
      for (int64_t w = lane; w < words; w += 64) d[w] = uint4{0, 0, 0, 0};
    }
  }
}

}  // namespace
}  // namespace rus

extern "C" int rus_copy_from_host(void* dst, const void* host_src, int64_t n_bytes,
                                  void* stream) {
  using namespace rus;
  const char* fn = "rus_copy_from_host";
  if (n_bytes < 0 || n_bytes % 16) return fail(RUS_ERR_INVALID, "%s: n_bytes %% 16 != 0", fn);
  if (n_bytes == 0) return RUS_OK;
  if (!dst || !host_src || !aligned(dst, 16) || !aligned(host_src, 16))
    return fail(RUS_ERR_INVALID, "%s: null or misaligned pointer", fn);
  // Only page-locked host memory mapped for the device may be read by the kernel.
  void* dev_src = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&dev_src, const_cast<void*>(host_src), 0);
  if (e != hipSuccess || !dev_src)
    return fail(RUS_ERR_INVALID, "%s: source is not page-locked, device-mapped host memory (%s)",
                fn, hipGetErrorString(e));
  const int64_t n = n_bytes / 16;
  const unsigned blocks = static_cast<unsigned>(n < 256 * 64 ? (n + 255) / 256 : 64);
  hipLaunchKernelGGL(copy16_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(dev_src), static_cast<uint4*>(dst), n);
  return check_launch(fn);
}

extern "C" int rus_gather_rows_from_host(const void* host_src, int64_t n_src_rows,
                                         int64_t row_bytes, const int64_t* ids, int64_t n_ids,
                                         void* dst, int32_t* err_flag, void* stream) {
  using namespace rus;
  const char* fn = "rus_gather_rows_from_host";
  if (n_src_rows < 0 || n_ids < 0 || row_bytes <= 0 || row_bytes % 16)
    return fail(RUS_ERR_INVALID, "%s: bad sizes (row_bytes must be a positive multiple of 16)", fn);
  if (n_ids == 0) return RUS_OK;
  if (!dst || !host_src || !ids || !aligned(dst, 16) || !aligned(host_src, 16) || !aligned(ids, 8))
    return fail(RUS_ERR_INVALID, "%s: null or misaligned pointer", fn);
  void* dev_src = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&dev_src, const_cast<void*>(host_src), 0);
  if (e != hipSuccess || !dev_src)
    return fail(RUS_ERR_INVALID, "%s: source is not page-locked, device-mapped host memory (%s)",
                fn, hipGetErrorString(e));
  const int64_t blocks = (n_ids + 3) / 4;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>(blocks < 1024 ? blocks : 1024)),
                     dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint4*>(dev_src), n_src_rows, row_bytes / 16, ids, n_ids,
                     static_cast<uint4*>(dst), err_flag);
  return check_launch(fn);
}
