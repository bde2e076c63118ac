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

// Kernel event timing used by the benchmark (kimkv_decode_timing,
// kimkv_prefill_timing): events recorded on the launch stream around each
// launch while enabled.
enum class TimedKernel : int { Decode = 0, Prefill = 1, Append = 2 };
void kernel_timing_begin(TimedKernel kind, hipStream_t stream, void** start);
void kernel_timing_end(TimedKernel kind, hipStream_t stream, void* start);

}  // namespace kimkv
