// knx_runtime.hip — device selection, memory, copies and streams of the KERNIX HIP layer, plus error plumbing.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "knx_common.hpp"
#include "knx_grid.hpp"

namespace knx {

static thread_local char g_err[512];

int fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

bool injected(const char* name)
{
    const char* v = getenv("KNX_HIP_FAIL");
    if (v == nullptr || *v == '\0') return false;
    if (strcmp(v, "all") == 0) return true;
    // comma separated list of entry-point names
    const size_t n = strlen(name);
    for (const char* p = v; *p;) {
        const char* e = strchr(p, ',');
        const size_t len = e ? (size_t)(e - p) : strlen(p);
        if (len == n && strncmp(p, name, n) == 0) return true;
        if (!e) break;
        p = e + 1;
    }
    return false;
}

int check_launch(const char* what)
{
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(KNX_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return KNX_OK;
}

constexpr int kMaxDevices = 64;
static int g_cus[kMaxDevices];  // compute units per device, 0 until queried

int num_cus()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    if (g_cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
        __atomic_store_n(&g_cus[dev], n, __ATOMIC_RELAXED);
    }
    return g_cus[dev];
}

unsigned grid_spin_limit()
{
    // KNX_GRID_SPIN: tests force a barrier to give up (0 = stop waiting at the first poll); every wave still ends
    const char* e = getenv("KNX_GRID_SPIN");
    if (e != nullptr && *e != '\0') {
        const long v = strtol(e, nullptr, 10);
        if (v >= 0 && v <= (long)KNX_GRID_SPIN_LIMIT) return (unsigned)v;
    }
    return KNX_GRID_SPIN_LIMIT;
}

}  // namespace knx

// The library runs on the device current on the calling thread (one process per GPU selects it with
// HIP_VISIBLE_DEVICES or hipSetDevice); each device is checked once for gfx950.
static std::mutex g_dev_mu;
static int g_dev_state[knx::kMaxDevices];  // 0 unchecked, 1 gfx950, -1 another architecture

extern "C" int knx_hip_init(void)
{
    KNX_ENTRY("knx_hip_init");
    int n = 0, cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur >= 0 && cur < knx::kMaxDevices &&
        __atomic_load_n(&g_dev_state[cur], __ATOMIC_ACQUIRE) > 0)
        return KNX_OK;  // checked before
    if (hipGetDeviceCount(&n) != hipSuccess || n < 1) return knx::fail(KNX_ENODEV, "knx_hip_init: no HIP device");
    if (hipGetDevice(&cur) != hipSuccess || cur < 0 || cur >= knx::kMaxDevices)
        return knx::fail(KNX_ENODEV, "knx_hip_init: no current device");
    std::lock_guard<std::mutex> lock(g_dev_mu);
    if (g_dev_state[cur] == 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, cur) != hipSuccess)
            return knx::fail(KNX_ENODEV, "knx_hip_init: cannot query device %d", cur);
        __atomic_store_n(&g_dev_state[cur], strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : -1, __ATOMIC_RELEASE);
        if (g_dev_state[cur] < 0)
            return knx::fail(KNX_ENODEV, "knx_hip_init: device %d is %s, this library is built for gfx950", cur,
                             prop.gcnArchName);
    }
    return g_dev_state[cur] > 0 ? KNX_OK : knx::fail(KNX_ENODEV, "knx_hip_init: device %d is not gfx950", cur);
}

extern "C" int knx_hip_get_device(int* device)
{
    KNX_REQUIRE(device != nullptr, "knx_hip_get_device");
    return hipGetDevice(device) == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_get_device failed");
}

extern "C" int knx_hip_set_device(int device)
{
    const hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) return KNX_OK;
    (void)hipGetLastError();  // a failed call leaves its error for the next launch check: clear it
    return knx::fail(KNX_EHIP, "knx_hip_set_device(%d): %s", device, hipGetErrorString(e));
}

extern "C" const char* knx_hip_last_error(void) { return knx::g_err; }

extern "C" int knx_hip_malloc(void** p, size_t bytes)
{
    KNX_ENTRY("knx_hip_malloc");
    KNX_REQUIRE(p != nullptr, "knx_hip_malloc");
    *p = nullptr;
    if (bytes == 0) bytes = 256;  // non-NULL handle for empty tensors
    const hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();  // not left for the next launch check
        return knx::fail(KNX_EHIP, "knx_hip_malloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    return KNX_OK;
}

extern "C" int knx_hip_free(void* p)
{
    if (p == nullptr) return KNX_OK;
    const hipError_t e = hipFree(p);
    return e == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_free: %s", hipGetErrorString(e));
}

extern "C" int knx_hip_host_malloc(void** p, size_t bytes)
{
    KNX_ENTRY("knx_hip_host_malloc");
    KNX_REQUIRE(p != nullptr, "knx_hip_host_malloc");
    *p = nullptr;
    if (bytes == 0) bytes = 256;
    const hipError_t e = hipHostMalloc(p, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
        return knx::fail(KNX_EHIP, "knx_hip_host_malloc(%zu): %s", bytes, hipGetErrorString(e));
    }
    return KNX_OK;
}

extern "C" int knx_hip_host_free(void* p)
{
    if (p == nullptr) return KNX_OK;
    const hipError_t e = hipHostFree(p);
    return e == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_host_free: %s", hipGetErrorString(e));
}

static int copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, void* stream, const char* name)
{
    if (knx::injected(name)) return knx::fail(KNX_EINJECT, "%s: injected failure", name);
    if (bytes == 0) return KNX_OK;
    KNX_REQUIRE(dst != nullptr && src != nullptr, name);
    const hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, knx::as_stream(stream));
    return e == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "%s(%zu): %s", name, bytes, hipGetErrorString(e));
}

extern "C" int knx_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream)
{
    return copy(dst, src, bytes, hipMemcpyHostToDevice, stream, "knx_hip_memcpy_h2d");
}

extern "C" int knx_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream)
{
    return copy(dst, src, bytes, hipMemcpyDeviceToHost, stream, "knx_hip_memcpy_d2h");
}

extern "C" int knx_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream)
{
    return copy(dst, src, bytes, hipMemcpyDeviceToDevice, stream, "knx_hip_memcpy_d2d");
}

extern "C" int knx_hip_memset(void* p, int value, size_t bytes, void* stream)
{
    KNX_ENTRY("knx_hip_memset");
    if (bytes == 0) return KNX_OK;
    KNX_REQUIRE(p != nullptr, "knx_hip_memset");
    const hipError_t e = hipMemsetAsync(p, value, bytes, knx::as_stream(stream));
    return e == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_memset(%zu): %s", bytes, hipGetErrorString(e));
}

extern "C" int knx_hip_stream_create(void** stream)
{
    KNX_ENTRY("knx_hip_stream_create");
    KNX_REQUIRE(stream != nullptr, "knx_hip_stream_create");
    hipStream_t s = nullptr;
    // Default priority only; a non-blocking stream so the model does not serialize with the null stream.
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return knx::fail(KNX_EHIP, "knx_hip_stream_create: %s", hipGetErrorString(e));
    *stream = s;
    return KNX_OK;
}

extern "C" int knx_hip_stream_destroy(void* stream)
{
    if (stream == nullptr) return KNX_OK;
    const hipError_t e = hipStreamDestroy(knx::as_stream(stream));
    return e == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_stream_destroy: %s", hipGetErrorString(e));
}

extern "C" int knx_hip_stream_sync(void* stream)
{
    KNX_ENTRY("knx_hip_stream_sync");
    const hipError_t e = hipStreamSynchronize(knx::as_stream(stream));
    return e == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_stream_sync: %s", hipGetErrorString(e));
}

extern "C" int knx_hip_event_create(void** event)
{
    KNX_ENTRY("knx_hip_event_create");
    KNX_REQUIRE(event != nullptr, "knx_hip_event_create");
    hipEvent_t e = nullptr;
    const hipError_t rc = hipEventCreateWithFlags(&e, hipEventDisableTiming);
    if (rc != hipSuccess) return knx::fail(KNX_EHIP, "knx_hip_event_create: %s", hipGetErrorString(rc));
    *event = e;
    return KNX_OK;
}

extern "C" int knx_hip_event_create_ordering(void** event)
{
    KNX_ENTRY("knx_hip_event_create_ordering");
    KNX_REQUIRE(event != nullptr, "knx_hip_event_create_ordering");
    // the system-scope release and acquire of an ordinary event record (cache write-back and invalidation) cost
    // about 1.8 µs of device time per record (a batch-1 forward on a caller's stream: 13.8 against 12.1 µs); kernels
    // see each other's results through the fences of their own dispatches, and a device-scope release alone
    // (hipEventReleaseToDevice) saves nothing
    hipEvent_t e = nullptr;
    const hipError_t rc = hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventDisableSystemFence);
    if (rc != hipSuccess) return knx::fail(KNX_EHIP, "knx_hip_event_create_ordering: %s", hipGetErrorString(rc));
    *event = e;
    return KNX_OK;
}

extern "C" int knx_hip_event_destroy(void* event)
{
    if (event == nullptr) return KNX_OK;
    const hipError_t rc = hipEventDestroy(static_cast<hipEvent_t>(event));
    return rc == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_event_destroy: %s", hipGetErrorString(rc));
}

extern "C" int knx_hip_event_record(void* event, void* stream)
{
    KNX_ENTRY("knx_hip_event_record");
    KNX_REQUIRE(event != nullptr, "knx_hip_event_record");
    const hipError_t rc = hipEventRecord(static_cast<hipEvent_t>(event), knx::as_stream(stream));
    return rc == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_event_record: %s", hipGetErrorString(rc));
}

extern "C" int knx_hip_stream_wait_event(void* stream, void* event)
{
    KNX_ENTRY("knx_hip_stream_wait_event");
    KNX_REQUIRE(event != nullptr, "knx_hip_stream_wait_event");
    const hipError_t rc = hipStreamWaitEvent(knx::as_stream(stream), static_cast<hipEvent_t>(event), 0);
    return rc == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_stream_wait_event: %s", hipGetErrorString(rc));
}

extern "C" int knx_hip_event_sync(void* event)
{
    if (event == nullptr) return KNX_OK;
    const hipError_t rc = hipEventSynchronize(static_cast<hipEvent_t>(event));
    return rc == hipSuccess ? KNX_OK : knx::fail(KNX_EHIP, "knx_hip_event_sync: %s", hipGetErrorString(rc));
}
