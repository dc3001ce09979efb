// kanjoos_amd/csrc/knj_spans.h -- per-launch device spans for the profiler.
//
// Every kernel launch of the step paths goes through KNJ_LAUNCH.  Normally that
// is a plain hipLaunchKernelGGL.  While a SpanSink is installed on the calling
// thread (a profiling run, which launches the step directly rather than
// replaying its graph), the launch is issued with hipExtLaunchKernelGGL and a
// start/stop event pair that the command processor records around that
// dispatch alone, so a span is the kernel's own execution interval, not the
// host's view of it.  The enqueue code names the op a launch belongs to with
// span_scope(class, layer) / span_class(class); the sink tags each event pair
// with that name and the kernel's symbol.  A full ring counts drops instead of
// growing: events are created before the run, never inside it.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace knj {

struct SpanTag {
  const char* cls;
  const char* kernel;
  int layer;
};

struct SpanSink {
  hipEvent_t* ev = nullptr;  // 2 * cap events, created by the owner
  int cap = 0;
  int used = 0;
  uint64_t dropped = 0;
  const char* cls = "";
  int layer = -1;
  std::vector<SpanTag> tags;
};

// The sink of the calling thread, or null (defined in knj_model.hip).
extern thread_local SpanSink* tl_span_sink;

inline void span_scope(const char* cls, int layer) {
  if (SpanSink* s = tl_span_sink) {
    s->cls = cls;
    s->layer = layer;
  }
}
inline void span_class(const char* cls) {
  if (SpanSink* s = tl_span_sink) s->cls = cls;
}

// Event pair for the next launch, or false when no sink is installed or its
// ring is full (counted as dropped).
inline bool span_take(const char* kernel, hipEvent_t* a, hipEvent_t* b) {
  SpanSink* s = tl_span_sink;
  if (!s) return false;
  if (s->used >= s->cap) {
    ++s->dropped;
    return false;
  }
  while (*kernel == '(' || *kernel == ' ') ++kernel;
  *a = s->ev[2 * s->used];
  *b = s->ev[2 * s->used + 1];
  s->tags.push_back(SpanTag{s->cls, kernel, s->layer});
  ++s->used;
  return true;
}

}  // namespace knj

#define KNJ_LAUNCH(kernel, grid, block, lds, stream, ...)                                      \
  do {                                                                                         \
    hipEvent_t knj_ev0_ = nullptr, knj_ev1_ = nullptr;                                         \
    if (::knj::span_take(#kernel, &knj_ev0_, &knj_ev1_))                                       \
      hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)(lds), stream, knj_ev0_, knj_ev1_, \
                            0u, __VA_ARGS__);                                                  \
    else                                                                                       \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                      \
  } while (0)
