// hipGraph capture / replay of execution plans.
//
// Handle 0 is the process-wide graph of the reference's CudaGraphState
// singleton and graph_* entry points (src/python_bindings/bindings.cpp:
// 137-187,475-547): begin ends any dangling capture and starts a global-mode
// capture on the handle's dedicated non-blocking stream; end instantiates;
// launch replays; reset drops all.  Further handles (aicf_graph_create) are
// independent graphs with their own streams, captured in thread-local mode,
// so several plans can stay instantiated side by side.
//
// Re-capturing on a handle that already holds an executable graph updates
// that executable in place (hipGraphExecUpdate) when the new graph has the
// same topology - the usual case when a plan is captured again with other
// buffers bound - and instantiates afresh only when the update is refused.
//
// Launch replays the executable on the caller's stream (NULL: the null
// stream, torch's default), so the replay runs after the work already queued
// there (input copies, host-side updates of device scalars) and before the
// work queued there afterwards (reads of its results), in stream order and
// with no cross-stream events.  The dedicated stream is the capture stream.
// The reference replays on its dedicated stream with no ordering against
// the caller's work.
#include <hip/hip_runtime_api.h>

#include <map>
#include <memory>
#include <mutex>

#include "../common/host_util.hpp"

namespace {

struct GraphState {
  bool capturing = false;
  bool captured = false;
  bool global_mode = true;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipStream_t stream = nullptr;
  uint64_t updates = 0;  // re-captures applied through hipGraphExecUpdate

  hipError_t ensure_stream() {
    hipError_t e = hipSuccess;
    if (!stream) e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    return e;
  }

  void destroy_graph() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    exec = nullptr;
    graph = nullptr;
    captured = false;
  }

  void end_dangling_capture() {
    if (!stream) return;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone) {
      hipGraph_t tmp = nullptr;
      if (hipStreamEndCapture(stream, &tmp) == hipSuccess && tmp) (void)hipGraphDestroy(tmp);
    }
    (void)hipGetLastError();
  }

  void reset_full() {
    end_dangling_capture();
    destroy_graph();
    capturing = false;
  }

  void release() {
    reset_full();
    if (stream) (void)hipStreamDestroy(stream);
    stream = nullptr;
  }
};

std::mutex g_mu;
std::map<uint64_t, std::unique_ptr<GraphState>> g_graphs;
uint64_t g_next_handle = 1;

GraphState* lookup(uint64_t h) {
  auto it = g_graphs.find(h);
  if (it != g_graphs.end()) return it->second.get();
  if (h != 0) return nullptr;
  auto& slot = g_graphs[0];
  slot = std::make_unique<GraphState>();
  return slot.get();
}

int32_t fail(hipError_t e, const char* what) {
  aicf::hip::set_last_error(what, hipGetErrorString(e));
  return AICF_STATUS_INTERNAL;
}

int32_t bad_handle(uint64_t h) {
  (void)h;
  aicf::hip::set_last_error("graph", "unknown graph handle");
  return AICF_STATUS_INVALID_ARGUMENT;
}

int32_t begin_on(GraphState& g, uint64_t* out_stream) {
  // a dangling capture is abandoned; an instantiated executable is kept
  // (but not launchable) until end() decides between update and rebuild
  g.end_dangling_capture();
  g.capturing = false;
  g.captured = false;
  hipError_t e = g.ensure_stream();
  if (e != hipSuccess) return fail(e, "hipStreamCreateWithFlags");
  e = hipStreamBeginCapture(g.stream, g.global_mode ? hipStreamCaptureModeGlobal
                                                    : hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return fail(e, "hipStreamBeginCapture");
  g.capturing = true;
  if (out_stream) *out_stream = reinterpret_cast<uint64_t>(g.stream);
  return AICF_STATUS_OK;
}

int32_t end_on(GraphState& g) {
  if (!g.capturing) {
    aicf::hip::set_last_error("graph_end", "graph_end called but not capturing");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  g.capturing = false;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(g.stream, &graph);
  if (e != hipSuccess) return fail(e, "hipStreamEndCapture");
  if (g.exec) {
    hipGraphNode_t err_node = nullptr;
    hipGraphExecUpdateResult res = hipGraphExecUpdateError;
    e = hipGraphExecUpdate(g.exec, graph, &err_node, &res);
    if (e == hipSuccess && res == hipGraphExecUpdateSuccess) {
      if (g.graph) (void)hipGraphDestroy(g.graph);
      g.graph = graph;
      g.captured = true;
      ++g.updates;
      return AICF_STATUS_OK;
    }
    (void)hipGetLastError();
    g.destroy_graph();
  } else if (g.graph) {
    (void)hipGraphDestroy(g.graph);
    g.graph = nullptr;
  }
  g.graph = graph;
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) return fail(e, "hipGraphInstantiate");
  g.exec = exec;
  g.captured = true;
  return AICF_STATUS_OK;
}

int32_t launch_on(GraphState& g, void* caller_stream) {
  if (!g.captured || !g.exec) {
    aicf::hip::set_last_error("graph_launch", "graph_launch called but no captured graph exists");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  // NULL is the null stream (torch's default stream)
  const hipError_t e = hipGraphLaunch(g.exec, reinterpret_cast<hipStream_t>(caller_stream));
  if (e != hipSuccess) return fail(e, "hipGraphLaunch");
  return AICF_STATUS_OK;
}

int32_t state_of(const GraphState& g) {
  if (g.capturing) return 1;
  if (g.captured) return 2;
  return 0;
}

}  // namespace

extern "C" {

// ---- handle 0: the reference's singleton graph --------------------------------
int32_t aicf_graph_begin(uint64_t* out_stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(0);
  // the singleton drops its previous graph at begin (bindings.cpp:475-490)
  g->reset_full();
  return begin_on(*g, out_stream);
}

int32_t aicf_graph_end(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return end_on(*lookup(0));
}

int32_t aicf_graph_launch(void* caller_stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  return launch_on(*lookup(0), caller_stream);
}

int32_t aicf_graph_reset(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  lookup(0)->reset_full();
  return AICF_STATUS_OK;
}

uint64_t aicf_graph_stream(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return reinterpret_cast<uint64_t>(lookup(0)->stream);
}

int32_t aicf_graph_state(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return state_of(*lookup(0));
}

// ---- further handles ----------------------------------------------------------
int32_t aicf_graph_create(uint64_t* out_handle) {
  if (!out_handle) return AICF_STATUS_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lock(g_mu);
  const uint64_t h = g_next_handle++;
  auto g = std::make_unique<GraphState>();
  g->global_mode = false;
  g_graphs[h] = std::move(g);
  *out_handle = h;
  return AICF_STATUS_OK;
}

int32_t aicf_graph_destroy(uint64_t handle) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (handle == 0) {
    aicf::hip::set_last_error("graph_destroy", "handle 0 is the process-wide graph; use aicf_graph_reset");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  auto it = g_graphs.find(handle);
  if (it == g_graphs.end()) return bad_handle(handle);
  it->second->release();
  g_graphs.erase(it);
  return AICF_STATUS_OK;
}

int32_t aicf_graph_begin_h(uint64_t handle, uint64_t* out_stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(handle);
  if (!g) return bad_handle(handle);
  return begin_on(*g, out_stream);
}

int32_t aicf_graph_end_h(uint64_t handle) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(handle);
  if (!g) return bad_handle(handle);
  return end_on(*g);
}

int32_t aicf_graph_launch_h(uint64_t handle, void* caller_stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(handle);
  if (!g) return bad_handle(handle);
  return launch_on(*g, caller_stream);
}

int32_t aicf_graph_reset_h(uint64_t handle) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(handle);
  if (!g) return bad_handle(handle);
  g->reset_full();
  return AICF_STATUS_OK;
}

uint64_t aicf_graph_stream_h(uint64_t handle) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(handle);
  return g ? reinterpret_cast<uint64_t>(g->stream) : 0;
}

int32_t aicf_graph_state_h(uint64_t handle) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(handle);
  return g ? state_of(*g) : -1;
}

uint64_t aicf_graph_updates_h(uint64_t handle) {
  std::lock_guard<std::mutex> lock(g_mu);
  GraphState* g = lookup(handle);
  return g ? g->updates : 0;
}

}  // extern "C"
