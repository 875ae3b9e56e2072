// C-ABI plumbing: per-thread last-error string and library version.
// No C++ exception crosses the ABI; every entry point returns 0 on success,
// 1 for an argument error (message in sa_last_error) and 2 for a HIP error.
#include <stdarg.h>
#include <stdio.h>

extern "C" {

static thread_local char g_err[1024] = {0};

void sa_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

const char* sa_last_error(void) { return g_err; }

int sa_version(void) { return 1; }

}  // extern "C"
