// C-ABI plumbing: per-thread error message, ABI queries, HIP graph capture.
#include <algorithm>
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

// Polls before a bounded cross-workgroup wait gives up (~1 us each, ~2 s in
// all). DTREE_TEST_SPIN_LIMIT=n lowers the bound (read at every launch), so
// tests can make a wait give up from the host while every workgroup still
// runs to its end; -1 makes every wait give up before its first poll.
int attn_spin_limit() {
  const char* e = std::getenv("DTREE_TEST_SPIN_LIMIT");
  return e && e[0] ? std::max(-1, std::atoi(e)) : (1 << 21);
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

// ---- host-side validation of tree inputs ------------------------------------
// The kernels read trees from device memory and cannot report a malformed one
// synchronously (they only keep their accesses in bounds, see valid_parent),
// so a binder validates on the host before the upload.

extern "C" int dtree_validate_parents(const int32_t* parents, int32_t num_nodes) {
  if (!parents) return fail(DTREE_E_ARG, "validate_parents: null pointer");
  if (num_nodes < 1 || num_nodes > DTREE_MAX_NODES)
    return fail(DTREE_E_TREE, "tree must have 1.." + std::to_string(DTREE_MAX_NODES) + " nodes, got " +
                                  std::to_string(num_nodes));
  if (parents[0] != -1) return fail(DTREE_E_TREE, "tree root parent must be -1, got " + std::to_string(parents[0]));
  for (int i = 1; i < num_nodes; ++i)
    if (parents[i] < 0 || parents[i] >= i)
      return fail(DTREE_E_TREE, "tree parent index must precede child, got parents[" + std::to_string(i) +
                                    "]=" + std::to_string(parents[i]));
  return DTREE_OK;
}

extern "C" int dtree_step_desc_validate(const DtreeStepDesc* d, int32_t max_nodes, int32_t max_past_length,
                                        int32_t vocab_size) {
  if (!d) return fail(DTREE_E_ARG, "step_desc_validate: null pointer");
  if (max_nodes < 1 || max_nodes > DTREE_MAX_NODES || vocab_size < 1 || max_past_length < 0)
    return fail(DTREE_E_ARG, "step_desc_validate: max_nodes in [1, 128], vocab_size >= 1, max_past_length >= 0");
  const int L = d->num_nodes;
  if (L < 1 || L > max_nodes)
    return fail(DTREE_E_TREE, "tree must have 1.." + std::to_string(max_nodes) + " nodes, got " + std::to_string(L));
  if (d->past_length < 0 || d->past_length > max_past_length)
    return fail(DTREE_E_ARG, "past_length " + std::to_string(d->past_length) + " outside [0, " +
                                 std::to_string(max_past_length) + "]");
  int rc = dtree_validate_parents(d->parents, L);
  if (rc) return rc;
  for (int i = 0; i < L; ++i) {
    if (d->tokens[i] < 0 || d->tokens[i] >= vocab_size)
      return fail(DTREE_E_ARG, "token id " + std::to_string(d->tokens[i]) + " outside the vocabulary");
    if (d->positions[i] < 0) return fail(DTREE_E_ARG, "negative RoPE position at node " + std::to_string(i));
    // ancestor-or-self bitset = the parent's plus bit i (the root: bit 0 only)
    for (int w = 0; w < DTREE_MASK_WORDS; ++w) {
      uint32_t want = i == 0 ? 0u : d->ancestors[d->parents[i]][w];
      if (w == i / 32) want |= 1u << (i % 32);
      if (d->ancestors[i][w] != want)
        return fail(DTREE_E_TREE, "ancestors[" + std::to_string(i) + "] is not the parent's set plus the node itself");
    }
  }
  if (d->n_accepted < 0 || d->n_accepted > L)
    return fail(DTREE_E_ARG, "n_accepted outside [0, num_nodes]");
  for (int j = 0; j < d->n_accepted; ++j)
    if (d->accepted[j] < 0 || d->accepted[j] >= L)
      return fail(DTREE_E_ARG, "accepted[" + std::to_string(j) + "] outside [0, num_nodes)");
  return DTREE_OK;
}
