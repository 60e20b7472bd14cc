// Capture and replay of a launch sequence through the C ABI, for hosts without torch: the
// reference's WebGPUPlatform.beginCapture / endCapture / replay (`webtorch/platform.py:45-56`)
// as HIP stream capture. Everything a caller launches on the stream between miq_graph_begin and
// miq_graph_end is recorded (the library's kernels read their shapes and pointers at launch, so
// the buffers must stay alive while the graph exists); miq_graph_launch replays the recording on
// any stream. The decode kernels keep their state (position, token ids) in device memory, so a
// replayed one-token step advances the sequence by itself.
#include "miq_common.h"

using namespace miq;

// A failed runtime call, reported through the return code (fail() also clears the runtime's
// last-error state, so it does not surface later as the failure of an unrelated launch).
static int hip_fail(const char* what, hipError_t e) { return fail(MIQ_ERR_HIP, "%s: %s", what, hipGetErrorString(e)); }

extern "C" int miq_graph_begin(void* stream) {
  MIQ_REQUIRE(stream, MIQ_ERR_INVALID, "graph_begin: capture needs a stream other than the null stream");
  const hipError_t e = hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail("graph_begin: hipStreamBeginCapture", e);
  return MIQ_OK;
}

extern "C" int miq_graph_end(void* stream, void** graph) {
  MIQ_REQUIRE(stream && graph, MIQ_ERR_INVALID, "graph_end: null stream or output");
  *graph = nullptr;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g);
  if (e != hipSuccess || !g) return hip_fail("graph_end: hipStreamEndCapture", e != hipSuccess ? e : hipErrorUnknown);
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  const hipError_t d = hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail("graph_end: hipGraphInstantiate", e);
  if (d != hipSuccess) {
    (void)hipGraphExecDestroy(x);
    return hip_fail("graph_end: hipGraphDestroy", d);
  }
  *graph = x;
  return MIQ_OK;
}

extern "C" int miq_graph_launch(void* graph, void* stream) {
  MIQ_REQUIRE(graph, MIQ_ERR_INVALID, "graph_launch: null graph");
  const hipError_t e = hipGraphLaunch(static_cast<hipGraphExec_t>(graph), static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail("graph_launch: hipGraphLaunch", e);
  return MIQ_OK;
}

extern "C" int miq_graph_destroy(void* graph) {
  if (!graph) return MIQ_OK;
  const hipError_t e = hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph));
  if (e != hipSuccess) return hip_fail("graph_destroy: hipGraphExecDestroy", e);
  return MIQ_OK;
}
