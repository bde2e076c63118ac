// runtime_internal.h -- status plumbing shared by the C-ABI translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "kimkv_hip.h"

namespace kimkv {

// Records the native error for kimkv_last_native_error() and maps it.
kimkv_status record_error(hipError_t error, kimkv_status failure);

// Status of the launch just issued (hipGetLastError) mapped to the C-ABI.
inline kimkv_status launch_status()
{
    return record_error(hipGetLastError(), KIMKV_SUBMISSION_FAILED);
}

inline hipStream_t native(kimkv_stream_t stream) { return static_cast<hipStream_t>(stream); }

// Decode-kernel event timing used by the benchmark (kimkv_decode_timing).
void decode_timing_begin(hipStream_t stream, void** start);
void decode_timing_end(hipStream_t stream, void* start);

}  // namespace kimkv
