// Error reporting shared by the sources behind the C ABI: every entry point returns a status and
// leaves its message for qe_last_error() (include/qe.h).
#pragma once

namespace qe {
// Stores the printf-formatted message as the calling thread's last error and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
}  // namespace qe
