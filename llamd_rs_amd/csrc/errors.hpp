// errors.hpp -- the library's per-thread error text (llamd_hip_last_error),
// for host files other than capi.cpp.
#pragma once

namespace llamd {

// printf-style; always returns -1 so callers can `return set_error(...)`.
int set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));

}  // namespace llamd
