// Optional per-kernel timing with HIP events recorded on the launch stream.
// Off by default (one branch per launch); bench.py switches it on for a
// profiled pass and reads back the average duration of every kernel name.
#pragma once

#include <hip/hip_runtime.h>

namespace sa {

// Takes two events and records the first on s (both null when timing is off
// or no event could be had).
void prof_begin(hipStream_t s, hipEvent_t* a, hipEvent_t* b);
// Records b on s and publishes the closed record (name, a, b); no-op for null
// events.  Only closed records are ever visible to sa_profile_collect.
void prof_end(const char* name, hipEvent_t a, hipEvent_t b, hipStream_t s);

// RAII helper: records a start event on construction, the stop event on
// destruction (after the launch statement of its scope).  The scope owns its
// events until it publishes them.
struct ProfScope {
  const char* name;
  hipStream_t s;
  hipEvent_t a = nullptr, b = nullptr;
  ProfScope(const char* n, hipStream_t stream) : name(n), s(stream) { prof_begin(s, &a, &b); }
  ~ProfScope() { prof_end(name, a, b, s); }
  ProfScope(const ProfScope&) = delete;
  ProfScope& operator=(const ProfScope&) = delete;
};

}  // namespace sa
