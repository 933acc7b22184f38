// arc_runtime.cpp -- device, memory, stream and event part of the C ABI
// (include/arcllm_hip.h), plus the thread-local error channel every entry
// point reports through.  Replaces the Vulkan device runtime of the
// reference (VkRuntime::{init,make_buffer,destroy_buffer},
// src/arcllm_v1_vulkan_runtime_support.h:498-664).
#include "../../include/arcllm_hip.h"
#include "arc_device.hpp"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>

namespace arc {

// Every device allocation of the library goes through device_alloc: the
// model arena, the session arena and arc_malloc.
static std::atomic<uint64_t> g_device_allocs{0};

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_hip(hipError_t e, const char* what)
{
    if (e == hipSuccess) return ARC_OK;
    const int code = (e == hipErrorOutOfMemory) ? ARC_ERR_OUT_OF_MEMORY
                     : (e == hipErrorNoDevice || e == hipErrorInvalidDevice) ? ARC_ERR_NO_DEVICE
                                                                               : ARC_ERR_DEVICE;
    return set_error(code, "%s: %s (%d)", what, hipGetErrorString(e), int(e));
}

int device_alloc(void** ptr, size_t bytes, const char* what)
{
    *ptr = nullptr;
    const int rc = check_hip(hipMalloc(ptr, bytes), what);
    if (!rc) g_device_allocs.fetch_add(1, std::memory_order_relaxed);
    return rc;
}

int residency_fits(uint64_t bytes, const char* what)
{
    size_t free_b = 0, total_b = 0;
    const int rc = check_hip(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
    if (rc) return rc;
    if (bytes > uint64_t(free_b) || uint64_t(free_b) - bytes < kResidencyHeadroom)
        return set_error(ARC_ERR_OUT_OF_MEMORY,
                         "%s: planned residency %llu bytes exceeds the free device memory %llu bytes less the "
                         "%llu-byte headroom",
                         what, static_cast<unsigned long long>(bytes), static_cast<unsigned long long>(free_b),
                         static_cast<unsigned long long>(kResidencyHeadroom));
    return ARC_OK;
}

}  // namespace arc

using arc::check_hip;
using arc::set_error;

extern "C" {

const char* arc_last_error(void) { return arc::g_err; }

const char* arc_version(void) { return "arcllm-mi355x 0.1 (gfx950)"; }

int arc_device_count(int* count)
{
    if (!count) return set_error(ARC_ERR_INVALID_ARGUMENT, "null count");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || e == hipErrorInsufficientDriver) {
        (void)hipGetLastError();
        *count = 0;
        return ARC_OK;
    }
    if (e != hipSuccess) return check_hip(e, "hipGetDeviceCount");
    *count = n;
    return ARC_OK;
}

int arc_set_device(int device) { return check_hip(hipSetDevice(device), "hipSetDevice"); }

int arc_device_info(char* name, size_t name_len, char* arch, size_t arch_len)
{
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    hipDeviceProp_t p;
    rc = check_hip(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
    if (rc) return rc;
    if (name && name_len) std::snprintf(name, name_len, "%s", p.name);
    if (arch && arch_len) std::snprintf(arch, arch_len, "%s", p.gcnArchName);
    return ARC_OK;
}

int arc_malloc(void** ptr, size_t bytes)
{
    if (!ptr || bytes == 0) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad malloc arguments");
    return arc::device_alloc(ptr, bytes, "hipMalloc");
}

int arc_device_allocations(uint64_t* count)
{
    if (!count) return set_error(ARC_ERR_INVALID_ARGUMENT, "null count");
    *count = arc::g_device_allocs.load(std::memory_order_relaxed);
    return ARC_OK;
}

int arc_free(void* ptr) { return ptr ? check_hip(hipFree(ptr), "hipFree") : ARC_OK; }

int arc_memcpy_htod(void* dst, const void* src, size_t bytes, arc_stream_t stream)
{
    if (!bytes) return ARC_OK;
    if (!dst || !src) return set_error(ARC_ERR_INVALID_ARGUMENT, "null memcpy pointer");
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)),
                     "hipMemcpy H2D");
}

int arc_memcpy_dtoh(void* dst, const void* src, size_t bytes, arc_stream_t stream)
{
    if (!bytes) return ARC_OK;
    if (!dst || !src) return set_error(ARC_ERR_INVALID_ARGUMENT, "null memcpy pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    int rc = check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "hipMemcpy D2H");
    if (rc) return rc;
    // pageable host destination: complete before returning
    return check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
}

int arc_memcpy_dtod(void* dst, const void* src, size_t bytes, arc_stream_t stream)
{
    if (!bytes) return ARC_OK;
    if (!dst || !src) return set_error(ARC_ERR_INVALID_ARGUMENT, "null memcpy pointer");
    return check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)),
                     "hipMemcpy D2D");
}

int arc_memset(void* dst, int value, size_t bytes, arc_stream_t stream)
{
    if (!bytes) return ARC_OK;
    if (!dst) return set_error(ARC_ERR_INVALID_ARGUMENT, "null memset pointer");
    return check_hip(hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream)), "hipMemset");
}

int arc_synchronize(void) { return check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

int arc_stream_create(arc_stream_t* stream)
{
    if (!stream) return set_error(ARC_ERR_INVALID_ARGUMENT, "null stream out");
    hipStream_t s = nullptr;
    // default priority; non-blocking with respect to the legacy null stream
    const int rc = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
    *stream = s;
    return rc;
}

int arc_stream_destroy(arc_stream_t stream)
{
    return stream ? check_hip(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy") : ARC_OK;
}

int arc_stream_synchronize(arc_stream_t stream)
{
    return check_hip(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
}

int arc_event_create(arc_event_t* event)
{
    if (!event) return set_error(ARC_ERR_INVALID_ARGUMENT, "null event out");
    hipEvent_t e = nullptr;
    const int rc = check_hip(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return rc;
}

int arc_event_destroy(arc_event_t event)
{
    return event ? check_hip(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy") : ARC_OK;
}

int arc_event_record(arc_event_t event, arc_stream_t stream)
{
    if (!event) return set_error(ARC_ERR_INVALID_ARGUMENT, "null event");
    return check_hip(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)),
                     "hipEventRecord");
}

int arc_event_elapsed_ms(arc_event_t start, arc_event_t stop, float* ms)
{
    if (!start || !stop || !ms) return set_error(ARC_ERR_INVALID_ARGUMENT, "bad event arguments");
    int rc = check_hip(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "hipEventSynchronize");
    if (rc) return rc;
    return check_hip(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                     "hipEventElapsedTime");
}

}  // extern "C"
