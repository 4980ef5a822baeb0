// Host functions of oc_api.hip that the C ABI's other source files use.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

#include "orthocache_hip.h"

namespace oc {

// Sets the thread's oc_last_error() message; returns code.
int api_fail(int code, const char* fmt, ...);
// OC_OK, or OC_ERR_HIP with the runtime's message.
int api_hip_check(hipError_t e, const char* what);
// The body of oc_decode_layer on the given workspace (validation included).
int decode_layer_run(const oc_layer_args* a, void* workspace, size_t workspace_bytes, void* stream,
                     const char* name);

}  // namespace oc
