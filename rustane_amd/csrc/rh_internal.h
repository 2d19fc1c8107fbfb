// rh_internal.h -- host-side helpers shared by the runtime's translation units.
#pragma once
#include <string>

#include "../../include/rustane_hip.h"

// Records msg as the context's last error (when ctx is set) and returns code.
int rh_internal_fail(rh_ctx* ctx, int code, const std::string& msg);
// The calling thread's last error from a context-free entry point.
const char* rh_internal_tls_error();
