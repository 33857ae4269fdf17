// Host-side helpers shared by the library's translation units.
#pragma once

namespace qs_host {

// Store a formatted message for qs_last_error() on the calling thread and
// return code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clear the calling thread's message.
void clear_error();

// True for the types whose quantizer cannot run without an imatrix
// (IQ2_XXS / IQ2_XS / IQ2_S); every other type runs with imatrix == NULL.
bool quantizer_requires_imatrix(int ggml_type);

}  // namespace qs_host
