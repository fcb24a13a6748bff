// Helpers shared by the C-ABI translation units (defined in capi.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

struct chimera_ctx;

namespace chimera {

// Records msg as the calling thread's last error and returns code.
int api_fail(int code, const std::string& msg);

// Null-checks the context, makes its device current and returns its stream.
int api_enter(chimera_ctx* c, hipStream_t* stream);

}  // namespace chimera
