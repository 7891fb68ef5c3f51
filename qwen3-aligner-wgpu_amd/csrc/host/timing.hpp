// timing.hpp -- shared step timer of the host mirror: warm-up, optional
// capture of one step into a hipGraph, then HIP events on the context's stream
// and the host clock around exactly `steps` steps.
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>

#include "qa.h"

namespace qa_host {

inline int timing_status(hipError_t e) { return e == hipSuccess ? QA_OK : QA_EDEVICE; }

// Runs `warmup` untimed steps, then `steps` timed ones.  With use_graph one
// step is captured into a hipGraph and the warm-up steps are replays of it,
// as the timed ones are; one eager step precedes the capture (the first call
// of a step sizes the context's workspace, which cannot grow under capture).
// Warm-up steps taken eagerly instead, with the graph launched once before
// the timed replays, left the first timed run of a process ~3.5% slower than
// a second one.
template <class Step>
int time_steps(qa_ctx* ctx, int warmup, int steps, int use_graph, Step&& step, double* ms,
               double* wall_ms = nullptr) {
  hipStream_t s = (hipStream_t)qa_ctx_stream(ctx);
  if (use_graph && warmup < 1) warmup = 1;
  for (int i = 0; i < (use_graph ? 1 : warmup); ++i)
    if (int rc = step()) return rc;
  if (int rc = qa_sync(ctx)) return rc;
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph = nullptr;
  if (use_graph) {
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return QA_EDEVICE;
    const int rc = step();
    const hipError_t ec = hipStreamEndCapture(s, &graph);
    if (rc) return rc;
    if (ec != hipSuccess) return QA_EDEVICE;
    if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) return QA_EDEVICE;
    for (int i = 0; i < warmup; ++i)  // the first replay also uploads the graph
      if (hipGraphLaunch(exec, s) != hipSuccess) return QA_EDEVICE;
    if (int rc2 = qa_sync(ctx)) return rc2;
  }
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  const auto w0 = std::chrono::steady_clock::now();
  (void)hipEventRecord(e0, s);
  int rc = QA_OK;
  for (int i = 0; i < steps && rc == QA_OK; ++i) {
    if (exec)
      rc = timing_status(hipGraphLaunch(exec, s));
    else
      rc = step();
  }
  (void)hipEventRecord(e1, s);
  const int rs = qa_sync(ctx);
  const auto w1 = std::chrono::steady_clock::now();
  if (wall_ms && steps > 0)
    *wall_ms = std::chrono::duration<double, std::milli>(w1 - w0).count() / steps;
  float t = 0.f;
  (void)hipEventElapsedTime(&t, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  if (rc) return rc;
  if (rs) return rs;
  *ms = steps > 0 ? (double)t / steps : 0.0;
  return QA_OK;
}

}  // namespace qa_host
