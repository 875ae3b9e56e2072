// C-ABI plumbing: per-thread last-error string and library version.
// No C++ exception crosses the ABI; every entry point returns 0 on success,
// 1 for an argument error (message in sa_last_error) and 2 for a HIP error.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "prof.h"

extern "C" {

static thread_local char g_err[1024] = {0};

void sa_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

const char* sa_last_error(void) { return g_err; }

int sa_version(void) { return 2; }

}  // extern "C"

// ---------------------------------------------------------------------------
// per-kernel event timing (see prof.h).  Entry points may be called from
// several host threads: the switch is atomic, and the record list and the
// free events are guarded by one mutex, which a launch takes only while
// profiling is on.  A launch holds its two events in its own ProfScope and
// appends the record only once both are recorded, so a collect on another
// thread never sees (or recycles the events of) a launch in progress.
// ---------------------------------------------------------------------------
namespace {
struct ProfRec {
  const char* name;
  hipEvent_t a, b;
};
std::atomic<bool> g_prof_on{false};
std::mutex g_prof_mu;
std::vector<ProfRec> g_recs;
std::vector<hipEvent_t> g_free;

hipEvent_t take_event() {   // caller holds g_prof_mu
  if (!g_free.empty()) {
    hipEvent_t e = g_free.back();
    g_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

namespace sa {
void prof_begin(hipStream_t s, hipEvent_t* a, hipEvent_t* b) {
  *a = *b = nullptr;
  if (!g_prof_on.load(std::memory_order_relaxed)) return;
  {
    std::lock_guard<std::mutex> lock(g_prof_mu);
    hipEvent_t ea = take_event(), eb = take_event();
    if (!ea || !eb) {
      if (ea) g_free.push_back(ea);
      if (eb) g_free.push_back(eb);
      return;
    }
    *a = ea;
    *b = eb;
  }
  (void)hipEventRecord(*a, s);
}
void prof_end(const char* name, hipEvent_t a, hipEvent_t b, hipStream_t s) {
  if (!a || !b) return;
  (void)hipEventRecord(b, s);
  std::lock_guard<std::mutex> lock(g_prof_mu);
  g_recs.push_back(ProfRec{name, a, b});
}
}  // namespace sa

extern "C" {

void sa_profile_enable(int on) { g_prof_on.store(on != 0, std::memory_order_relaxed); }

// Synchronises the recorded events, aggregates by kernel name and clears the
// records.  Writes up to max_kernels entries: names (NUL-separated into
// names_buf), total milliseconds and launch counts.  Returns the number of
// distinct kernels (or -1 on a HIP error).
int sa_profile_collect(char* names_buf, int names_len, float* total_ms, int* counts,
                       int max_kernels) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  std::vector<std::string> names;
  std::vector<float> tot;
  std::vector<int> cnt;
  int rc = 0;
  for (auto& r : g_recs) {
    float ms = 0.f;
    if (hipEventSynchronize(r.b) != hipSuccess || hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess)
      rc = -1;
    size_t k = 0;
    while (k < names.size() && names[k] != r.name) ++k;
    if (k == names.size()) {
      names.emplace_back(r.name);
      tot.push_back(0.f);
      cnt.push_back(0);
    }
    tot[k] += ms;
    cnt[k] += 1;
    g_free.push_back(r.a);
    g_free.push_back(r.b);
  }
  g_recs.clear();
  if (rc) return -1;
  int off = 0;
  const int n = static_cast<int>(names.size());
  for (int k = 0; k < n && k < max_kernels; ++k) {
    const int len = static_cast<int>(names[k].size()) + 1;
    if (off + len <= names_len) {
      memcpy(names_buf + off, names[k].c_str(), len);
      off += len;
    }
    total_ms[k] = tot[k];
    counts[k] = cnt[k];
  }
  return n;
}

}  // extern "C"
