// runtime.hip — device memory, streams, events and error reporting of the
// extension interface (include/nerf_ext.h).  These let a host with no GPU
// framework (a C program, or Python through ctypes) stage inputs in HBM and
// time kernels on its own stream.
#include <stdio.h>
#include <string.h>

#include "common.hpp"

namespace nerf_hip {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

NerfStatus hip_fail(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
    return NERF_STATUS_CUDA_ERROR;
}

uint32_t device_cu_count() {
    static int cached_device = -1;
    static uint32_t cached   = 0;
    int dev                  = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256u;
    if (dev != cached_device) {
        hipDeviceProp_t prop{};
        if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 256u;
        cached        = (uint32_t)prop.multiProcessorCount;
        cached_device = dev;
    }
    return cached;
}

}  // namespace nerf_hip

using namespace nerf_hip;

extern "C" {

NERF_API const char* nerf_ext_last_error(void) { return g_last_error.c_str(); }

NERF_API NerfStatus nerf_ext_device_info(NerfExtDeviceInfo* out) {
    NERF_CHECK_ARG(out, "nerf_ext_device_info: null output");
    int dev = 0;
    NERF_HIP_TRY(hipGetDevice(&dev));
    hipDeviceProp_t prop{};
    NERF_HIP_TRY(hipGetDeviceProperties(&prop, dev));
    memset(out, 0, sizeof(*out));
    snprintf(out->name, sizeof(out->name), "%s", prop.name);
    snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    out->compute_units       = (uint32_t)prop.multiProcessorCount;
    out->lds_bytes_per_block = (uint32_t)prop.sharedMemPerBlock;
    out->global_mem_bytes    = (uint64_t)prop.totalGlobalMem;
    out->clock_khz           = (uint32_t)prop.clockRate;
    out->memory_clock_khz    = (uint32_t)prop.memoryClockRate;
    out->memory_bus_bits     = (uint32_t)prop.memoryBusWidth;
    out->l2_bytes            = (uint32_t)prop.l2CacheSize;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_malloc(void** out_ptr, uint64_t bytes) {
    NERF_CHECK_ARG(out_ptr, "nerf_ext_malloc: null output");
    *out_ptr = nullptr;
    if (bytes == 0) return NERF_STATUS_OK;
    NERF_HIP_TRY(hipMalloc(out_ptr, bytes));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_free(void* ptr) {
    if (!ptr) return NERF_STATUS_OK;
    NERF_HIP_TRY(hipFree(ptr));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_memcpy(void* dst, const void* src, uint64_t bytes, uint32_t kind) {
    if (bytes == 0) return NERF_STATUS_OK;
    NERF_CHECK_ARG(dst && src, "nerf_ext_memcpy: null pointer");
    hipMemcpyKind k;
    switch (kind) {
    case NERF_EXT_H2D: k = hipMemcpyHostToDevice; break;
    case NERF_EXT_D2H: k = hipMemcpyDeviceToHost; break;
    case NERF_EXT_D2D: k = hipMemcpyDeviceToDevice; break;
    default: set_error("nerf_ext_memcpy: bad kind"); return NERF_STATUS_INVALID_USAGE;
    }
    NERF_HIP_TRY(hipMemcpy(dst, src, bytes, k));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_memset(void* dst, int value, uint64_t bytes) {
    if (bytes == 0) return NERF_STATUS_OK;
    NERF_CHECK_ARG(dst, "nerf_ext_memset: null pointer");
    NERF_HIP_TRY(hipMemset(dst, value, bytes));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_synchronize(void) {
    NERF_HIP_TRY(hipDeviceSynchronize());
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_stream_create(void** out_stream) {
    NERF_CHECK_ARG(out_stream, "nerf_ext_stream_create: null output");
    hipStream_t s = nullptr;
    NERF_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *out_stream = (void*)s;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_stream_destroy(void* stream) {
    if (!stream) return NERF_STATUS_OK;
    NERF_HIP_TRY(hipStreamDestroy((hipStream_t)stream));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_stream_synchronize(void* stream) {
    NERF_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_event_create(void** out_event) {
    NERF_CHECK_ARG(out_event, "nerf_ext_event_create: null output");
    hipEvent_t e = nullptr;
    NERF_HIP_TRY(hipEventCreate(&e));
    *out_event = (void*)e;
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_event_destroy(void* event) {
    if (!event) return NERF_STATUS_OK;
    NERF_HIP_TRY(hipEventDestroy((hipEvent_t)event));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_event_record(void* event, void* stream) {
    NERF_CHECK_ARG(event, "nerf_ext_event_record: null event");
    NERF_HIP_TRY(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return NERF_STATUS_OK;
}

NERF_API NerfStatus nerf_ext_event_elapsed_ms(void* start, void* stop, float* out_ms) {
    NERF_CHECK_ARG(start && stop && out_ms, "nerf_ext_event_elapsed_ms: null argument");
    NERF_HIP_TRY(hipEventSynchronize((hipEvent_t)stop));
    NERF_HIP_TRY(hipEventElapsedTime(out_ms, (hipEvent_t)start, (hipEvent_t)stop));
    return NERF_STATUS_OK;
}

}  // extern "C"
