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

// While the context's profiling is on (and it is not capturing a graph),
// HIP events on its stream bracket the work issued between the two calls and
// its duration is added to stage `stage` of chimera_stage_times.
void stage_begin(chimera_ctx* c, int stage);
void stage_end(chimera_ctx* c);

}  // namespace chimera
