// runtime.hip -- lifecycle, error reporting, memory, streams, events and graphs
// of the doe_mi355x C ABI.
#include "common.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

namespace doe {

static thread_local char g_err[1024] = "";
static int g_device = -1;

int set_error(int status, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return status;
}

void clear_error() { g_err[0] = '\0'; }

int hip_fail(hipError_t e, const char *what) {
    return set_error(e == hipErrorOutOfMemory ? DOE_E_OOM : DOE_E_HIP, "%s failed: %s (%d)",
                     what, hipGetErrorString(e), (int)e);
}

int require_init() {
    if (g_device < 0) return set_error(DOE_E_NOT_INIT, "doe_init() was not called");
    return DOE_OK;
}

// Workspaces replaced by larger ones, freed by doe_shutdown.
static std::mutex g_retired_mu;
static std::vector<void *> g_retired;

void retire_workspace(void *ptr) {
    if (!ptr) return;
    std::lock_guard<std::mutex> lk(g_retired_mu);
    g_retired.push_back(ptr);
}

// byte fill: the unaligned head and tail byte by byte, the middle 16 bytes
// per store
__global__ __launch_bounds__(256) void fill_bytes_kernel(uint8_t *dst, size_t head, size_t n16, size_t total,
                                                         uint32_t v4) {
    const size_t tid = (size_t)blockIdx.x * 256 + threadIdx.x, stride = (size_t)gridDim.x * 256;
    const uint4 v = make_uint4(v4, v4, v4, v4);
    uint4 *mid = reinterpret_cast<uint4 *>(dst + head);
    for (size_t i = tid; i < n16; i += stride) mid[i] = v;
    const size_t tail0 = head + n16 * 16;
    for (size_t i = tid; i < head + (total - tail0); i += stride) {
        const size_t at = i < head ? i : tail0 + (i - head);
        dst[at] = (uint8_t)v4;
    }
}

int fill_bytes_async(void *dst, int value, size_t bytes, hipStream_t st) {
    if (bytes == 0) return DOE_OK;
    uint8_t *p = static_cast<uint8_t *>(dst);
    size_t head = (16 - ((uintptr_t)p & 15)) & 15;
    if (head > bytes) head = bytes;
    const size_t n16 = (bytes - head) / 16;
    const uint32_t b = (uint32_t)(value & 0xff);
    size_t blocks = (n16 + 255) / 256;
    blocks = blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
    hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, head, n16, bytes,
                       b * 0x01010101u);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? DOE_OK : hip_fail(e, "fill_bytes_kernel launch");
}

}  // namespace doe

namespace {
// The device's constant-rate wall clock (s_memrealtime) stored by one lane.
__global__ void timestamp_kernel(unsigned long long *dst) {
    if (threadIdx.x == 0) dst[0] = wall_clock64();
}
}  // namespace

extern "C" {

int doe_init(int device) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return doe::hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return doe::set_error(DOE_E_INVALID, "device %d out of range (%d devices)", device, count);
    DOE_HIP_CHECK(hipSetDevice(device));
    hipDeviceProp_t prop;
    DOE_HIP_CHECK(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return doe::set_error(DOE_E_UNSUPPORTED, "device %d is %s; this library is built for gfx950",
                              device, prop.gcnArchName);
    // per-device address of the allocation-free entry point's scratch array
    const int src = doe::attn_scratch_setup(device);
    if (src) return src;
    doe::g_device = device;
    doe::clear_error();
    return DOE_OK;
}

int doe_shutdown(void) {
    if (doe::g_device < 0) return DOE_OK;
    DOE_HIP_CHECK(hipDeviceSynchronize());
    {
        std::lock_guard<std::mutex> lk(doe::g_retired_mu);
        for (void *p : doe::g_retired) DOE_HIP_CHECK(hipFree(p));
        doe::g_retired.clear();
    }
    doe::g_device = -1;
    return DOE_OK;
}

const char *doe_last_error(void) { return doe::g_err; }

int doe_device_info(char *buf, size_t buf_bytes) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(buf != nullptr && buf_bytes > 0, DOE_E_INVALID, "null buffer");
    hipDeviceProp_t p;
    DOE_HIP_CHECK(hipGetDeviceProperties(&p, doe::g_device));
    int n = snprintf(buf, buf_bytes,
                     "{\"device\": %d, \"name\": \"%s\", \"arch\": \"%s\", \"cus\": %d, "
                     "\"clock_khz\": %d, \"mem_clock_khz\": %d, \"bus_width\": %d, "
                     "\"total_mem\": %zu, \"l2_bytes\": %d, \"lds_per_block\": %zu, "
                     "\"max_threads_per_block\": %d, \"warp_size\": %d}",
                     doe::g_device, p.name, p.gcnArchName, p.multiProcessorCount, p.clockRate,
                     p.memoryClockRate, p.memoryBusWidth, (size_t)p.totalGlobalMem, p.l2CacheSize,
                     (size_t)p.sharedMemPerBlock, p.maxThreadsPerBlock, p.warpSize);
    DOE_REQUIRE(n > 0 && (size_t)n < buf_bytes, DOE_E_INVALID, "buffer too small (%d bytes needed)", n);
    return DOE_OK;
}

int doe_device_synchronize(void) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_HIP_CHECK(hipDeviceSynchronize());
    return DOE_OK;
}

int doe_malloc(void **ptr, size_t bytes) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(ptr != nullptr, DOE_E_INVALID, "null out-pointer");
    *ptr = nullptr;
    if (bytes == 0) return DOE_OK;
    DOE_HIP_CHECK(hipMalloc(ptr, bytes));
    return DOE_OK;
}

int doe_free(void *ptr) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (ptr) DOE_HIP_CHECK(hipFree(ptr));
    return DOE_OK;
}

int doe_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (bytes == 0) return DOE_OK;
    DOE_REQUIRE(dst && src, DOE_E_INVALID, "null pointer");
    DOE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return DOE_OK;
}

int doe_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (bytes == 0) return DOE_OK;
    DOE_REQUIRE(dst && src, DOE_E_INVALID, "null pointer");
    DOE_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return DOE_OK;
}

int doe_memcpy_d2d(void *dst, const void *src, size_t bytes, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (bytes == 0) return DOE_OK;
    DOE_REQUIRE(dst && src, DOE_E_INVALID, "null pointer");
    DOE_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return DOE_OK;
}

int doe_memcpy2d_d2d(void *dst, size_t dst_pitch, const void *src, size_t src_pitch, size_t row_bytes,
                     size_t rows, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (row_bytes == 0 || rows == 0) return DOE_OK;
    DOE_REQUIRE(dst && src, DOE_E_INVALID, "null pointer");
    DOE_REQUIRE(row_bytes <= dst_pitch && row_bytes <= src_pitch, DOE_E_INVALID,
                "row of %zu bytes wider than a pitch (dst %zu, src %zu)", row_bytes, dst_pitch, src_pitch);
    DOE_HIP_CHECK(hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, row_bytes, rows, hipMemcpyDeviceToDevice,
                                   (hipStream_t)stream));
    return DOE_OK;
}

int doe_memset(void *dst, int value, size_t bytes, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (bytes == 0) return DOE_OK;
    DOE_REQUIRE(dst, DOE_E_INVALID, "null pointer");
    return doe::fill_bytes_async(dst, value, bytes, (hipStream_t)stream);
}

int doe_stream_create(doe_stream_t *stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(stream, DOE_E_INVALID, "null out-pointer");
    hipStream_t s;
    DOE_HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = (doe_stream_t)s;
    return DOE_OK;
}

int doe_stream_destroy(doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (stream) DOE_HIP_CHECK(hipStreamDestroy((hipStream_t)stream));
    return DOE_OK;
}

int doe_stream_synchronize(doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_HIP_CHECK(hipStreamSynchronize((hipStream_t)stream));
    return DOE_OK;
}

int doe_event_create(doe_event_t *event) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(event, DOE_E_INVALID, "null out-pointer");
    hipEvent_t e;
    DOE_HIP_CHECK(hipEventCreate(&e));
    *event = (doe_event_t)e;
    return DOE_OK;
}

int doe_event_destroy(doe_event_t event) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (event) DOE_HIP_CHECK(hipEventDestroy((hipEvent_t)event));
    return DOE_OK;
}

int doe_event_record(doe_event_t event, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(event, DOE_E_INVALID, "null event");
    DOE_HIP_CHECK(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
    return DOE_OK;
}

int doe_event_synchronize(doe_event_t event) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(event, DOE_E_INVALID, "null event");
    DOE_HIP_CHECK(hipEventSynchronize((hipEvent_t)event));
    return DOE_OK;
}

int doe_event_elapsed_ms(float *ms, doe_event_t start, doe_event_t end) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(ms && start && end, DOE_E_INVALID, "null argument");
    DOE_HIP_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end));
    return DOE_OK;
}

int doe_device_timestamp(uint64_t *dst, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(dst && ((uintptr_t)dst & 7) == 0, DOE_E_INVALID, "timestamp destination must be 8-byte aligned");
    hipLaunchKernelGGL(timestamp_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (unsigned long long *)dst);
    DOE_LAUNCH_CHECK("timestamp_kernel");
    return DOE_OK;
}

int doe_device_timestamp_hz(int64_t *hz) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(hz, DOE_E_INVALID, "null argument");
    int dev = 0, khz = 0;
    DOE_HIP_CHECK(hipGetDevice(&dev));
    DOE_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
    *hz = (int64_t)khz * 1000;
    return DOE_OK;
}

int doe_graph_capture_begin(doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(stream, DOE_E_INVALID, "graph capture needs a created (non-default) stream");
    DOE_HIP_CHECK(hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeRelaxed));
    return DOE_OK;
}

int doe_graph_capture_end(doe_stream_t stream, doe_graph_t *graph) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(stream && graph, DOE_E_INVALID, "null argument");
    hipGraph_t g = nullptr;
    DOE_HIP_CHECK(hipStreamEndCapture((hipStream_t)stream, &g));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return doe::hip_fail(e, "hipGraphInstantiate");
    *graph = (doe_graph_t)exec;
    return DOE_OK;
}

int doe_graph_launch(doe_graph_t graph, doe_stream_t stream) {
    int rc = doe::require_init();
    if (rc) return rc;
    DOE_REQUIRE(graph, DOE_E_INVALID, "null graph");
    DOE_HIP_CHECK(hipGraphLaunch((hipGraphExec_t)graph, (hipStream_t)stream));
    return DOE_OK;
}

int doe_graph_destroy(doe_graph_t graph) {
    int rc = doe::require_init();
    if (rc) return rc;
    if (graph) DOE_HIP_CHECK(hipGraphExecDestroy((hipGraphExec_t)graph));
    return DOE_OK;
}

}  // extern "C"
