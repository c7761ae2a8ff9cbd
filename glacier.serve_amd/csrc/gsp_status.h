// Thread-local error reporting of the C ABI: every entry point clears the
// message on entry and sets it together with a non-zero status on failure.
#pragma once

namespace gsp {

void clear_error();
// Formats the message, stores it for gsp_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace gsp
