// moe_lib.h - library-internal helpers shared by the C ABI translation units.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/moehip.h"

namespace moe {
// Records a message for moe_last_error() and returns `st`.
moe_status set_error(moe_status st, const char* fmt, ...);
// MOE_OK, or MOE_ERR_HIP with "<what>: <hip error string>" recorded.
moe_status check_hip(hipError_t e, const char* what);
// Initialises device 0 if moe_init has not been called.
moe_status ensure_init();
// The library's stream.
hipStream_t stream();
// Layers and models alive (moe_shutdown refuses while any is).
void live_objects(int delta);
// Free the library-owned device buffers of one translation unit (the
// stream has drained; called by moe_shutdown only).
void release_gemv_workspace();
void release_layer_scratch();
}  // namespace moe
