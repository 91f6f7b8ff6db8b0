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
