// The library's per-thread error message (read by pa_last_error_message),
// shared by the C-ABI layer and the host-side planner.
#pragma once

namespace pa {

// Formats the calling thread's last error message and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
const char* last_error_message();

}  // namespace pa
