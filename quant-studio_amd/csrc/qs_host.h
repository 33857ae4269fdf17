// Host-side helpers shared by the library's translation units.
#pragma once

namespace qs_host {

// Store a formatted message for qs_last_error() on the calling thread and
// return code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clear the calling thread's message.
void clear_error();

}  // namespace qs_host
