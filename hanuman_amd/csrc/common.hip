// Library-level entry points: error reporting, ABI version and size helpers.
#include <string>

#include "hmoe_common.h"

namespace hmoe {

namespace {
thread_local std::string g_last_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return HMOE_ERR_HIP;
  }
  return HMOE_OK;
}

}  // namespace hmoe

extern "C" {

const char* hmoe_last_error(void) { return hmoe::g_last_error.c_str(); }

int hmoe_abi_version(void) { return 1; }

int64_t hmoe_capacity(int64_t tokens, int top_k, int n_experts, double capacity_factor) {
  if (tokens <= 0 || top_k <= 0 || n_experts <= 0) return 0;
  const int64_t rows = tokens * top_k;
  if (capacity_factor <= 0.0) return rows;
  // ceil(CF*T*K/N) evaluated as the oracle does (double arithmetic).
  double c = capacity_factor * static_cast<double>(tokens) * static_cast<double>(top_k) /
             static_cast<double>(n_experts);
  int64_t ci = static_cast<int64_t>(c);
  if (static_cast<double>(ci) < c) ci += 1;
  return ci;
}

int64_t hmoe_rows_cap(int64_t tokens, int top_k, int n_experts, int64_t capacity) {
  const int64_t rows = tokens * top_k;
  const int64_t cap_rows = static_cast<int64_t>(n_experts) * capacity;
  return rows < cap_rows ? rows : cap_rows;
}

}  // extern "C"
