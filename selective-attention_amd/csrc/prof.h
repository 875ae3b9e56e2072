// Optional per-kernel timing with HIP events recorded on the launch stream.
// Off by default (one branch per launch); bench.py switches it on for a
// profiled pass and reads back the average duration of every kernel name.
#pragma once

#include <hip/hip_runtime.h>

namespace sa {

int prof_begin(const char* name, hipStream_t s);  // returns a record slot or -1
void prof_end(int slot, hipStream_t s);

// RAII helper: records a start event on construction, the stop event on
// destruction (after the launch statement of its scope).
struct ProfScope {
  int slot;
  hipStream_t s;
  ProfScope(const char* name, hipStream_t stream) : slot(prof_begin(name, stream)), s(stream) {}
  ~ProfScope() { prof_end(slot, s); }
};

}  // namespace sa
