// hipGraph capture / replay of an execution plan: one process-wide graph on
// a dedicated non-blocking stream.
//
// Behaviour follows the CudaGraphState singleton and graph_* entry points of
// src/python_bindings/bindings.cpp:137-187,475-547 in the reference:
// begin ends any dangling capture, drops the old graph and starts a
// global-mode capture; end instantiates; launch replays; reset drops all.
// One addition: launch can first wait on an event recorded on the caller's
// stream, so device-scalar updates queued there are ordered before the
// replay (the reference replays with no such edge).
#include <hip/hip_runtime_api.h>

#include <mutex>

#include "../common/host_util.hpp"

namespace {

struct GraphState {
  bool capturing = false;
  bool captured = false;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipStream_t stream = nullptr;
  hipEvent_t edge = nullptr;

  hipError_t ensure_stream() {
    hipError_t e = hipSuccess;
    if (!stream) e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    if (e == hipSuccess && !edge) e = hipEventCreateWithFlags(&edge, hipEventDisableTiming);
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
};

GraphState g_state;
std::mutex g_mu;

int32_t fail(hipError_t e, const char* what) {
  aicf::hip::set_last_error(what, hipGetErrorString(e));
  return AICF_STATUS_INTERNAL;
}

}  // namespace

extern "C" {

int32_t aicf_graph_begin(uint64_t* out_stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  g_state.reset_full();
  hipError_t e = g_state.ensure_stream();
  if (e != hipSuccess) return fail(e, "hipStreamCreateWithFlags");
  e = hipStreamBeginCapture(g_state.stream, hipStreamCaptureModeGlobal);
  if (e != hipSuccess) return fail(e, "hipStreamBeginCapture");
  g_state.capturing = true;
  if (out_stream) *out_stream = reinterpret_cast<uint64_t>(g_state.stream);
  return AICF_STATUS_OK;
}

int32_t aicf_graph_end(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_state.capturing) {
    aicf::hip::set_last_error("graph_end", "graph_end called but not capturing");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  g_state.capturing = false;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(g_state.stream, &graph);
  if (e != hipSuccess) return fail(e, "hipStreamEndCapture");
  g_state.graph = graph;
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) return fail(e, "hipGraphInstantiate");
  g_state.exec = exec;
  g_state.captured = true;
  return AICF_STATUS_OK;
}

int32_t aicf_graph_launch(void* caller_stream) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_state.captured || !g_state.exec) {
    aicf::hip::set_last_error("graph_launch", "graph_launch called but no captured graph exists");
    return AICF_STATUS_INVALID_ARGUMENT;
  }
  hipError_t e = g_state.ensure_stream();
  if (e != hipSuccess) return fail(e, "hipStreamCreateWithFlags");
  hipStream_t caller = reinterpret_cast<hipStream_t>(caller_stream);
  if (caller && caller != g_state.stream) {
    e = hipEventRecord(g_state.edge, caller);
    if (e != hipSuccess) return fail(e, "hipEventRecord");
    e = hipStreamWaitEvent(g_state.stream, g_state.edge, 0);
    if (e != hipSuccess) return fail(e, "hipStreamWaitEvent");
  }
  e = hipGraphLaunch(g_state.exec, g_state.stream);
  if (e != hipSuccess) return fail(e, "hipGraphLaunch");
  return AICF_STATUS_OK;
}

int32_t aicf_graph_reset(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  g_state.reset_full();
  return AICF_STATUS_OK;
}

uint64_t aicf_graph_stream(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  return reinterpret_cast<uint64_t>(g_state.stream);
}

int32_t aicf_graph_state(void) {
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_state.capturing) return 1;
  if (g_state.captured) return 2;
  return 0;
}

}  // extern "C"
