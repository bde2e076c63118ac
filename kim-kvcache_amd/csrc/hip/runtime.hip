// runtime.hip -- C-ABI runtime wrappers and device pool storage.
//
// Storage keeps the interface of CudaKvStorage (src/cuda/kv/storage.cpp:99-190)
// with a layout of its own: one device allocation for both pools,
// zero-filled, layer-major (page_base in device_common.h).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <limits>
#include <mutex>
#include <new>
#include <vector>

#include "device_common.h"
#include "runtime_internal.h"

namespace kimkv {

namespace {
thread_local int g_last_native_error = 0;

struct DecodeTiming {
    std::mutex mutex;
    bool enabled{false};
    uint32_t every{1};        // time every n-th launch
    uint64_t seen{0};
    std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
    std::vector<hipEvent_t> spare;   // read events, reused
    double total_ms{0.0};
    uint64_t launches{0};
    // The union of the drained launches' intervals (launches on several
    // streams overlap), measured from the window's first start event.
    std::vector<std::pair<double, double>> intervals;
    double busy_ms{0.0};   // of the last closed window
};

// A timing event: reused when one is spare.  No system-scope fence when it
// is reached (nothing is published to the host; the fence's cache
// writeback would only add to the timed span).
hipEvent_t timing_event_locked(DecodeTiming& t)
{
    if (!t.spare.empty()) {
        hipEvent_t const e = t.spare.back();
        t.spare.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    return hipEventCreateWithFlags(&e, hipEventDisableSystemFence) == hipSuccess ? e : nullptr;
}

void spare_event_locked(DecodeTiming& t, hipEvent_t e)
{
    try {
        t.spare.push_back(e);
    } catch (...) {
        static_cast<void>(hipEventDestroy(e));
    }
}

DecodeTiming& timing(TimedKernel kind = TimedKernel::Decode)
{
    static DecodeTiming instances[3];
    return instances[static_cast<int>(kind)];
}

void drain_locked(DecodeTiming& t)
{
    if (t.pending.empty()) return;
    hipEvent_t const ref = t.pending.front().first;
    for (auto& pair : t.pending) {
        if (hipEventSynchronize(pair.second) == hipSuccess) {
            float ms = 0.0f;
            float from = 0.0f;
            float to = 0.0f;
            if (hipEventElapsedTime(&ms, pair.first, pair.second) == hipSuccess) {
                t.total_ms += ms;
                t.launches += 1;
                if (hipEventElapsedTime(&from, ref, pair.first) == hipSuccess
                    && hipEventElapsedTime(&to, ref, pair.second) == hipSuccess) {
                    try {
                        t.intervals.emplace_back(from, to);
                    } catch (...) {
                    }
                }
            }
        }
    }
    for (auto& pair : t.pending) {
        spare_event_locked(t, pair.first);
        spare_event_locked(t, pair.second);
    }
    t.pending.clear();
}

// Length of the union of the window's intervals.
double busy_locked(DecodeTiming& t)
{
    std::sort(t.intervals.begin(), t.intervals.end());
    double busy = 0.0;
    double lo = 0.0;
    double hi = 0.0;
    bool open = false;
    for (auto const& iv : t.intervals) {
        if (!open || iv.first > hi) {
            if (open) busy += hi - lo;
            lo = iv.first;
            hi = iv.second;
            open = true;
        } else if (iv.second > hi) {
            hi = iv.second;
        }
    }
    if (open) busy += hi - lo;
    return busy;
}
}  // namespace

// Moves the fault word to the mapped host word and clears it in one atomic
// exchange, so bits set by concurrent work are never lost.
__global__ __launch_bounds__(64) void take_faults_kernel(uint32_t* faults, uint32_t* host_word)
{
    if (threadIdx.x == 0) *host_word = atomicExch(faults, 0u);
}

kimkv_status record_error(hipError_t error, kimkv_status failure)
{
    if (error == hipSuccess) {
        return KIMKV_OK;
    }
    g_last_native_error = static_cast<int>(error);
    return failure;
}

void kernel_timing_begin(TimedKernel kind, hipStream_t stream, void** start)
{
    *start = nullptr;
    DecodeTiming& t = timing(kind);
    std::lock_guard<std::mutex> lock(t.mutex);
    if (!t.enabled || t.seen++ % t.every != 0) {
        return;
    }
    hipEvent_t const event = timing_event_locked(t);
    if (event != nullptr && hipEventRecord(event, stream) == hipSuccess) {
        *start = event;
    } else if (event != nullptr) {
        spare_event_locked(t, event);
    }
}

void kernel_timing_end(TimedKernel kind, hipStream_t stream, void* start)
{
    if (start == nullptr) {
        return;
    }
    DecodeTiming& t = timing(kind);
    std::lock_guard<std::mutex> lock(t.mutex);
    hipEvent_t const stop = timing_event_locked(t);
    bool recorded = false;
    if (stop != nullptr && hipEventRecord(stop, stream) == hipSuccess) {
        try {
            t.pending.emplace_back(static_cast<hipEvent_t>(start), stop);
            recorded = true;
        } catch (...) {
        }
    }
    if (!recorded) {
        // The start event may still be pending on the stream: destroying a
        // recorded event is allowed (HIP releases it once it completes).
        static_cast<void>(hipEventDestroy(static_cast<hipEvent_t>(start)));
        if (stop != nullptr) static_cast<void>(hipEventDestroy(stop));
    }
}

}  // namespace kimkv

using kimkv::record_error;

extern "C" {

int kimkv_device_count(void)
{
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) {
        return 0;
    }
    return count;
}

int kimkv_last_native_error(void) { return kimkv::g_last_native_error; }

kimkv_status kimkv_device_malloc(void** ptr, size_t bytes)
{
    if (ptr == nullptr) return KIMKV_INVALID_ARGUMENT;
    *ptr = nullptr;
    if (bytes == 0) return KIMKV_OK;
    return record_error(hipMalloc(ptr, bytes), KIMKV_ALLOCATION_FAILED);
}

kimkv_status kimkv_device_free(void* ptr)
{
    if (ptr == nullptr) return KIMKV_OK;
    return record_error(hipFree(ptr), KIMKV_INTERNAL_ERROR);
}

kimkv_status kimkv_host_malloc_pinned(void** ptr, size_t bytes)
{
    if (ptr == nullptr) return KIMKV_INVALID_ARGUMENT;
    *ptr = nullptr;
    if (bytes == 0) return KIMKV_OK;
    return record_error(hipHostMalloc(ptr, bytes, hipHostMallocDefault), KIMKV_ALLOCATION_FAILED);
}

kimkv_status kimkv_host_malloc_mapped(void** host_ptr, void** device_ptr, size_t bytes)
{
    if (host_ptr == nullptr || device_ptr == nullptr) return KIMKV_INVALID_ARGUMENT;
    *host_ptr = nullptr;
    *device_ptr = nullptr;
    if (bytes == 0) return KIMKV_OK;
    kimkv_status const s =
        record_error(hipHostMalloc(host_ptr, bytes, hipHostMallocMapped | hipHostMallocCoherent), KIMKV_ALLOCATION_FAILED);
    if (s != KIMKV_OK) return s;
    void* dev = nullptr;
    kimkv_status const d = record_error(hipHostGetDevicePointer(&dev, *host_ptr, 0), KIMKV_ALLOCATION_FAILED);
    if (d != KIMKV_OK) {
        static_cast<void>(hipHostFree(*host_ptr));
        *host_ptr = nullptr;
        return d;
    }
    *device_ptr = dev;
    return KIMKV_OK;
}

kimkv_status kimkv_host_free_pinned(void* ptr)
{
    if (ptr == nullptr) return KIMKV_OK;
    return record_error(hipHostFree(ptr), KIMKV_INTERNAL_ERROR);
}

kimkv_status kimkv_memcpy_h2d_async(void* dst, const void* src, size_t bytes, kimkv_stream_t stream)
{
    if (bytes == 0) return KIMKV_OK;
    if (dst == nullptr || src == nullptr) return KIMKV_INVALID_ARGUMENT;
    return record_error(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, kimkv::native(stream)),
                        KIMKV_SUBMISSION_FAILED);
}

kimkv_status kimkv_memcpy_d2h_async(void* dst, const void* src, size_t bytes, kimkv_stream_t stream)
{
    if (bytes == 0) return KIMKV_OK;
    if (dst == nullptr || src == nullptr) return KIMKV_INVALID_ARGUMENT;
    return record_error(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, kimkv::native(stream)),
                        KIMKV_SUBMISSION_FAILED);
}

kimkv_status kimkv_memcpy_d2d_async(void* dst, const void* src, size_t bytes, kimkv_stream_t stream)
{
    if (bytes == 0) return KIMKV_OK;
    if (dst == nullptr || src == nullptr) return KIMKV_INVALID_ARGUMENT;
    return record_error(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, kimkv::native(stream)),
                        KIMKV_SUBMISSION_FAILED);
}

kimkv_status kimkv_stream_create(kimkv_stream_t* stream)
{
    if (stream == nullptr) return KIMKV_INVALID_ARGUMENT;
    hipStream_t s = nullptr;
    kimkv_status const status = record_error(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
                                             KIMKV_RUNTIME_UNAVAILABLE);
    *stream = s;
    return status;
}

kimkv_status kimkv_stream_destroy(kimkv_stream_t stream)
{
    if (stream == nullptr) return KIMKV_OK;
    return record_error(hipStreamDestroy(kimkv::native(stream)), KIMKV_INTERNAL_ERROR);
}

kimkv_status kimkv_stream_synchronize(kimkv_stream_t stream)
{
    return record_error(hipStreamSynchronize(kimkv::native(stream)), KIMKV_EXECUTION_FAILED);
}

kimkv_status kimkv_device_synchronize(void)
{
    return record_error(hipDeviceSynchronize(), KIMKV_EXECUTION_FAILED);
}

kimkv_status kimkv_event_create(void** event, int kind)
{
    if (event == nullptr || kind < 0 || kind > KIMKV_EVENT_ORDER_ONLY) return KIMKV_INVALID_ARGUMENT;
    unsigned const flags = kind == 1 ? hipEventDefault
        : kind == KIMKV_EVENT_ORDER_ONLY ? (hipEventDisableTiming | hipEventDisableSystemFence)
                                         : hipEventDisableTiming;
    hipEvent_t e = nullptr;
    kimkv_status const status = record_error(hipEventCreateWithFlags(&e, flags), KIMKV_RUNTIME_UNAVAILABLE);
    *event = e;
    return status;
}

kimkv_status kimkv_event_destroy(void* event)
{
    if (event == nullptr) return KIMKV_OK;
    return record_error(hipEventDestroy(static_cast<hipEvent_t>(event)), KIMKV_INTERNAL_ERROR);
}

kimkv_status kimkv_event_record(void* event, kimkv_stream_t stream)
{
    if (event == nullptr) return KIMKV_INVALID_ARGUMENT;
    return record_error(hipEventRecord(static_cast<hipEvent_t>(event), kimkv::native(stream)),
                        KIMKV_SUBMISSION_FAILED);
}

kimkv_status kimkv_stream_wait_event(kimkv_stream_t stream, void* event)
{
    if (event == nullptr) return KIMKV_INVALID_ARGUMENT;
    return record_error(hipStreamWaitEvent(kimkv::native(stream), static_cast<hipEvent_t>(event), 0),
                        KIMKV_SUBMISSION_FAILED);
}

kimkv_status kimkv_event_query(void* event)
{
    if (event == nullptr) return KIMKV_INVALID_ARGUMENT;
    hipError_t const e = hipEventQuery(static_cast<hipEvent_t>(event));
    if (e == hipErrorNotReady) return KIMKV_NOT_READY;
    return record_error(e, KIMKV_EXECUTION_FAILED);
}

kimkv_status kimkv_event_synchronize(void* event)
{
    if (event == nullptr) return KIMKV_INVALID_ARGUMENT;
    return record_error(hipEventSynchronize(static_cast<hipEvent_t>(event)), KIMKV_EXECUTION_FAILED);
}

kimkv_status kimkv_event_elapsed_ms(float* ms, void* start, void* stop)
{
    if (ms == nullptr || start == nullptr || stop == nullptr) return KIMKV_INVALID_ARGUMENT;
    return record_error(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                        KIMKV_EXECUTION_FAILED);
}

kimkv_status kimkv_storage_create(kimkv_storage** out, kimkv_layout layout, uint32_t micro_capacity,
                                  uint32_t extent_capacity, uint16_t micro_page_tokens,
                                  uint16_t extent_page_tokens)
{
    if (out == nullptr) return KIMKV_INVALID_ARGUMENT;
    *out = nullptr;
    if (layout.layers == 0 || layout.kv_heads == 0 || layout.head_dim == 0
        || micro_page_tokens == 0 || extent_page_tokens == 0 || layout.layers > 0x7FFFu) {
        return KIMKV_INVALID_ARGUMENT;
    }
    uint64_t const per_token = 2ull * layout.layers * layout.kv_heads * layout.head_dim;
    uint64_t const micro_elems = per_token * micro_page_tokens;
    uint64_t const extent_elems = per_token * extent_page_tokens;
    uint64_t const limit = std::numeric_limits<uint64_t>::max() / 4;
    if ((micro_capacity != 0 && micro_elems > limit / micro_capacity)
        || (extent_capacity != 0 && extent_elems > limit / extent_capacity)) {
        return KIMKV_INVALID_ARGUMENT;
    }
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        return KIMKV_RUNTIME_UNAVAILABLE;
    }
    auto* s = new (std::nothrow) kimkv_storage{};
    if (s == nullptr) return KIMKV_ALLOCATION_FAILED;
    s->layout = layout;
    s->micro_capacity = micro_capacity;
    s->extent_capacity = extent_capacity;
    s->micro_tokens = micro_page_tokens;
    s->extent_tokens = extent_page_tokens;
    s->micro_page_elements = micro_elems;
    s->extent_page_elements = extent_elems;
    hipError_t e = hipGetDevice(&s->device);
    if (e == hipSuccess) {
        e = hipDeviceGetAttribute(&s->compute_units, hipDeviceAttributeMultiprocessorCount, s->device);
    }
    // One allocation, layer-major (page_base in device_common.h): layer 0's
    // micro blocks, its extent blocks, then layer 1's, ...
    uint64_t const micro_bytes = micro_elems * micro_capacity * 2ull;
    uint64_t const extent_bytes = extent_elems * extent_capacity * 2ull;
    if (e == hipSuccess && micro_bytes + extent_bytes != 0) {
        e = hipMalloc(reinterpret_cast<void**>(&s->pool), micro_bytes + extent_bytes);
        if (e == hipSuccess) e = hipMemset(s->pool, 0, micro_bytes + extent_bytes);
        if (e == hipSuccess) {
            s->micro = s->pool;
            s->extent = s->pool + kimkv::slot_elements(layout, micro_page_tokens) * micro_capacity;
        }
    }
    if (e == hipSuccess) {
        e = hipMalloc(reinterpret_cast<void**>(&s->faults), 256);
        if (e == hipSuccess) e = hipMemset(s->faults, 0, 256);
    }
    size_t const counter_bytes = sizeof(uint32_t) * kWorkCounterSlots * kWorkCounterStride;
    if (e == hipSuccess) {
        e = hipMalloc(reinterpret_cast<void**>(&s->work_counters), counter_bytes);
        if (e == hipSuccess) e = hipMemset(s->work_counters, 0, counter_bytes);
    }
    if (e == hipSuccess) {
        e = hipHostMalloc(reinterpret_cast<void**>(&s->fault_host), 256, hipHostMallocMapped | hipHostMallocCoherent);
        if (e == hipSuccess) e = hipHostGetDevicePointer(reinterpret_cast<void**>(&s->fault_view), s->fault_host, 0);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        record_error(e, KIMKV_ALLOCATION_FAILED);
        if (s->pool) static_cast<void>(hipFree(s->pool));
        if (s->faults) static_cast<void>(hipFree(s->faults));
        if (s->work_counters) static_cast<void>(hipFree(s->work_counters));
        if (s->fault_host) static_cast<void>(hipHostFree(s->fault_host));
        delete s;
        return KIMKV_ALLOCATION_FAILED;
    }
    *out = s;
    return KIMKV_OK;
}

kimkv_status kimkv_storage_destroy(kimkv_storage* storage)
{
    if (storage == nullptr) return KIMKV_OK;
    // In-flight work may still read the pools (storage.cpp:22-32 waits too).
    static_cast<void>(hipDeviceSynchronize());
    if (storage->pool) static_cast<void>(hipFree(storage->pool));
    if (storage->faults) static_cast<void>(hipFree(storage->faults));
    if (storage->work_counters) static_cast<void>(hipFree(storage->work_counters));
    if (storage->fault_host) static_cast<void>(hipHostFree(storage->fault_host));
    delete storage;
    return KIMKV_OK;
}

kimkv_status kimkv_storage_faults(kimkv_storage* storage, kimkv_stream_t stream, uint32_t* faults)
{
    if (faults != nullptr) *faults = 0;
    if (storage == nullptr || storage->faults == nullptr || storage->fault_view == nullptr) {
        return KIMKV_INVALID_ARGUMENT;
    }
    // One reader of the mapped word at a time.
    static std::mutex mutex;
    std::lock_guard<std::mutex> lock(mutex);
    *reinterpret_cast<volatile uint32_t*>(storage->fault_host) = 0;
    kimkv::take_faults_kernel<<<1, 64, 0, kimkv::native(stream)>>>(storage->faults, storage->fault_view);
    kimkv_status const launched = kimkv::launch_status();
    if (launched != KIMKV_OK) return launched;
    kimkv_status const done = record_error(hipStreamSynchronize(kimkv::native(stream)), KIMKV_EXECUTION_FAILED);
    if (done != KIMKV_OK) return done;
    uint32_t const bits = *reinterpret_cast<volatile uint32_t*>(storage->fault_host);
    if (faults != nullptr) *faults = bits;
    return bits != 0 ? KIMKV_INVALID_ARGUMENT : KIMKV_OK;
}

kimkv_status kimkv_storage_query(const kimkv_storage* s, kimkv_storage_info* info)
{
    if (s == nullptr || info == nullptr) return KIMKV_INVALID_ARGUMENT;
    info->layout = s->layout;
    info->micro_capacity = s->micro_capacity;
    info->extent_capacity = s->extent_capacity;
    info->micro_page_tokens = s->micro_tokens;
    info->extent_page_tokens = s->extent_tokens;
    info->micro_page_elements = s->micro_page_elements;
    info->extent_page_elements = s->extent_page_elements;
    info->micro_reserved_bytes = s->micro_page_elements * s->micro_capacity * 2ull;
    info->extent_reserved_bytes = s->extent_page_elements * s->extent_capacity * 2ull;
    info->device = s->device;
    info->compute_units = s->compute_units;
    return KIMKV_OK;
}

uint16_t* kimkv_storage_page(const kimkv_storage* s, uint32_t kind, uint32_t slot)
{
    if (s == nullptr) return nullptr;
    if (kind == KIMKV_PAGE_MICRO && slot < s->micro_capacity && s->micro != nullptr) {
        return s->micro + static_cast<uint64_t>(slot) * kimkv::slot_elements(s->layout, s->micro_tokens);
    }
    if (kind == KIMKV_PAGE_EXTENT && slot < s->extent_capacity && s->extent != nullptr) {
        return s->extent + static_cast<uint64_t>(slot) * kimkv::slot_elements(s->layout, s->extent_tokens);
    }
    return nullptr;
}

uint16_t kimkv_synth_value(uint64_t seed, uint64_t row, uint32_t col)
{
    float const x = static_cast<float>(kimkv::synth_int(seed, row, col)) * (1.0f / 32768.0f);
    return __half_as_ushort(__float2half(x));
}

uint64_t kimkv_synth_kv_row(uint32_t stream, uint32_t layer, uint32_t component, uint32_t token)
{
    return kimkv::kv_row(stream, layer, component, token);
}

namespace {
kimkv_status kernel_timing(kimkv::TimedKernel kind, int enable, double* total_ms, uint64_t* launches)
{
    kimkv::DecodeTiming& t = kimkv::timing(kind);
    std::lock_guard<std::mutex> lock(t.mutex);
    kimkv::drain_locked(t);
    if (total_ms != nullptr) *total_ms = t.total_ms;
    if (launches != nullptr) *launches = t.launches;
    t.busy_ms = kimkv::busy_locked(t);
    t.intervals.clear();
    t.total_ms = 0.0;
    t.launches = 0;
    t.enabled = enable > 0;
    t.every = enable > 0 ? static_cast<uint32_t>(enable) : 1u;
    t.seen = 0;
    return KIMKV_OK;
}
}  // namespace

kimkv_status kimkv_decode_timing(int enable, double* total_ms, uint64_t* launches)
{
    return kernel_timing(kimkv::TimedKernel::Decode, enable, total_ms, launches);
}

kimkv_status kimkv_prefill_timing(int enable, double* total_ms, uint64_t* launches)
{
    return kernel_timing(kimkv::TimedKernel::Prefill, enable, total_ms, launches);
}

kimkv_status kimkv_append_timing(int enable, double* total_ms, uint64_t* launches)
{
    return kernel_timing(kimkv::TimedKernel::Append, enable, total_ms, launches);
}

kimkv_status kimkv_decode_timing_busy(double* busy_ms)
{
    if (busy_ms == nullptr) return KIMKV_INVALID_ARGUMENT;
    kimkv::DecodeTiming& t = kimkv::timing(kimkv::TimedKernel::Decode);
    std::lock_guard<std::mutex> lock(t.mutex);
    *busy_ms = t.busy_ms;
    return KIMKV_OK;
}

}  // extern "C"
