// C-ABI plumbing: per-thread error message, ABI queries, HIP graph capture.
#include <cstdio>
#include <cstdlib>
#include <string>

#include "common.h"

namespace dtree {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// Test hook: DTREE_TEST_OFF_XCD=1 makes the kernels treat every workgroup as
// placed off its expected XCD, so the cross-XCD (sc1) exchange paths run even
// though the dispatcher always places workgroups round-robin. Read per launch.
bool off_xcd_test() {
  const char* e = std::getenv("DTREE_TEST_OFF_XCD");
  return e && e[0] == '1';
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return DTREE_OK;
  g_last_error = std::string(what) + ": " + hipGetErrorString(e);
  return DTREE_E_HIP;
}

}  // namespace dtree

using namespace dtree;

extern "C" const char* dtree_last_error(void) { return g_last_error.c_str(); }

extern "C" int dtree_abi_version(void) { return DTREE_ABI_VERSION; }

extern "C" size_t dtree_step_desc_bytes(void) { return sizeof(DtreeStepDesc); }

extern "C" size_t dtree_gemm_args_bytes(void) { return sizeof(DtreeGemmArgs); }

extern "C" size_t dtree_attn_args_bytes(void) { return sizeof(DtreeAttnArgs); }

extern "C" int dtree_graph_begin(hipStream_t stream) {
  return hip_check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

extern "C" int dtree_graph_end(hipStream_t stream, void** graph_exec) {
  DTREE_REQUIRE(graph_exec, "graph_end: null out pointer");
  hipGraph_t graph = nullptr;
  int rc = hip_check(hipStreamEndCapture(stream, &graph), "hipStreamEndCapture");
  if (rc) return rc;
  hipGraphExec_t exec = nullptr;
  rc = hip_check(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
  hipGraphDestroy(graph);
  if (rc) return rc;
  *graph_exec = exec;
  return DTREE_OK;
}

extern "C" int dtree_graph_launch(void* graph_exec, hipStream_t stream) {
  DTREE_REQUIRE(graph_exec, "graph_launch: null graph");
  return hip_check(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), stream), "hipGraphLaunch");
}

extern "C" int dtree_graph_destroy(void* graph_exec) {
  if (!graph_exec) return DTREE_OK;
  return hip_check(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
}
