// runtime.hip -- device, memory, stream, event and graph glue of the op
// boundary.  Replaces the runtime half of the reference
// (src/ai/cuda_ops.cu:83-231): cuda_init selects device 0 and creates the
// copy stream; memory calls are thin HIP wrappers.  Unlike the reference,
// every HIP status is checked and latched.
#include <atomic>
#include <mutex>
#include <string.h>

#include "common.h"

namespace {

bool g_initialized = false;
hipDeviceProp_t g_props;
hipStream_t g_stream = nullptr;       // library compute stream (null = legacy default)
hipStream_t g_copy_stream = nullptr;  // cuda_memcpy_*_async
int g_cus = 256;
std::atomic<int> g_error{0};

}  // namespace

namespace holo {

hipStream_t stream() { return g_stream; }
hipStream_t copy_stream() { return g_copy_stream ? g_copy_stream : g_stream; }
int num_cus() { return g_cus; }

void latch_error(int code, const char *what, const char *file, int line)
{
    int expected = 0;
    g_error.compare_exchange_strong(expected, code);
    const char *msg = code == HOLO_EINVAL ? "invalid argument" : hipGetErrorString((hipError_t)code);
    fprintf(stderr, "holo_mi355x error %d (%s) at %s:%d: %s\n", code, msg, file, line, what);
}

// One thread per 16-byte piece of the 16-byte-aligned span that covers
// [p, p + n): whole pieces take one vector store, the two end pieces store
// their covered bytes one at a time.
__global__ __launch_bounds__(256) void fill_bytes_k(uint8_t *p, uint32_t byte, size_t n)
{
    const uintptr_t a = (uintptr_t)p, end = a + n;
    const uintptr_t c = (a & ~(uintptr_t)15) + 16 * ((uintptr_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (c >= end) return;
    const uint32_t w = byte * 0x01010101u;
    if (c >= a && c + 16 <= end) {
        *(uint4 *)c = make_uint4(w, w, w, w);
        return;
    }
    for (uintptr_t b = c; b < c + 16; b++)
        if (b >= a && b < end) *(uint8_t *)b = (uint8_t)byte;
}

void fill_bytes(void *p, int value, size_t n)
{
    if (n == 0) return;
    const uintptr_t a = (uintptr_t)p;
    const size_t pieces = (((a + n + 15) & ~(uintptr_t)15) - (a & ~(uintptr_t)15)) / 16;
    hipLaunchKernelGGL(fill_bytes_k, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, g_stream, (uint8_t *)p,
                       (uint32_t)(value & 0xFF), n);
    HOLO_LAUNCH_CHECK();
}

bool stream_capturing()
{
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(g_stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

}  // namespace holo

extern "C" {

int holo_last_error(void) { return g_error.exchange(0); }

const char *holo_error_string(int code)
{
    if (code == 0) return "ok";
    if (code == HOLO_EINVAL) return "invalid argument";
    if (code == HOLO_ECHAIN) return "persistent decode-step launch could not synchronise its workgroups";
    return hipGetErrorString((hipError_t)code);
}

// cuda_ops.cu:95-132
int cuda_init(void)
{
    if (g_initialized) return 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        fprintf(stderr, "holo_mi355x: no HIP device found\n");
        return -1;
    }
    if (hipSetDevice(0) != hipSuccess || hipGetDeviceProperties(&g_props, 0) != hipSuccess) {
        fprintf(stderr, "holo_mi355x: cannot open device 0\n");
        return -1;
    }
    g_cus = g_props.multiProcessorCount > 0 ? g_props.multiProcessorCount : 256;
    if (hipStreamCreateWithFlags(&g_copy_stream, hipStreamNonBlocking) != hipSuccess) {
        fprintf(stderr, "holo_mi355x: cannot create copy stream\n");
        return -1;
    }
    if (!holo::gemv_stream_init()) {
        fprintf(stderr, "holo_mi355x: cannot allocate the GEMV stream barrier\n");
        return -1;
    }
    if (!holo::attention_scratch_init()) {
        fprintf(stderr, "holo_mi355x: cannot allocate the decode-attention scratch\n");
        return -1;
    }
    if (!holo::exact_init()) {
        fprintf(stderr, "holo_mi355x: cannot allocate the batched product's tile counters\n");
        return -1;
    }
    if (!holo::noalloc_scratch()) {
        fprintf(stderr, "holo_mi355x: cannot look up the fixed scratch array\n");
        return -1;
    }
    g_initialized = true;
    return 0;
}

// cuda_ops.cu:134-147
void cuda_cleanup(void)
{
    if (!g_initialized) return;
    hipDeviceSynchronize();
    if (g_copy_stream) hipStreamDestroy(g_copy_stream);
    g_copy_stream = nullptr;
    holo::gemv_stream_release();
    holo::attention_scratch_release();
    holo::panel_workspace_release();
    holo::exact_release();
    g_stream = nullptr;
    g_initialized = false;
}

bool cuda_available(void) { return g_initialized; }  // cuda_ops.cu:149-151

void cuda_print_info(void)  // cuda_ops.cu:153-165
{
    if (!g_initialized) {
        printf("HIP: not initialized\n");
        return;
    }
    printf("HIP device: %s (%s)\n", g_props.name, g_props.gcnArchName);
    printf("  Total memory: %.2f GB\n", g_props.totalGlobalMem / (1024.0 * 1024.0 * 1024.0));
    printf("  Compute units: %d\n", g_props.multiProcessorCount);
    printf("  Max threads/block: %d\n", g_props.maxThreadsPerBlock);
    printf("  Wavefront size: %d\n", g_props.warpSize);
}

int cuda_get_device_count(void)  // cuda_ops.cu:167-171
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

size_t cuda_get_free_memory(void)  // cuda_ops.cu:173-177
{
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) != hipSuccess) return 0;
    return f;
}

const char *cuda_get_device_name(void) { return g_initialized ? g_props.name : "No device"; }

void *cuda_malloc(size_t size)  // cuda_ops.cu:187-191: NULL on failure
{
    void *p = nullptr;
    if (size == 0) return nullptr;
    if (hipMalloc(&p, size) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

void cuda_free(void *ptr)
{
    if (ptr) HOLO_CHECK(hipFree(ptr));
}

// The synchronous copies order after all work on the library stream, as the
// reference's cudaMemcpy orders after the legacy default stream.
void cuda_memcpy_h2d(void *dst, const void *src, size_t size)
{
    if (size == 0) return;
    HOLO_CHECK(hipMemcpyAsync(dst, src, size, hipMemcpyHostToDevice, g_stream));
    HOLO_CHECK(hipStreamSynchronize(g_stream));
}

void cuda_memcpy_d2h(void *dst, const void *src, size_t size)
{
    if (size == 0) return;
    HOLO_CHECK(hipMemcpyAsync(dst, src, size, hipMemcpyDeviceToHost, g_stream));
    HOLO_CHECK(hipStreamSynchronize(g_stream));
}

void cuda_memcpy_d2d(void *dst, const void *src, size_t size)
{
    if (size == 0) return;
    HOLO_CHECK(hipMemcpyAsync(dst, src, size, hipMemcpyDeviceToDevice, g_stream));
    HOLO_CHECK(hipStreamSynchronize(g_stream));
}

void cuda_memcpy_d2d_async(void *dst, const void *src, size_t size)  // cuda_ops.cu:210-212
{
    if (size == 0) return;
    HOLO_CHECK(hipMemcpyAsync(dst, src, size, hipMemcpyDeviceToDevice, holo::copy_stream()));
}

void cuda_memcpy_d2h_async(void *dst, const void *src, size_t size)  // cuda_ops.cu:214-216
{
    if (size == 0) return;
    HOLO_CHECK(hipMemcpyAsync(dst, src, size, hipMemcpyDeviceToHost, holo::copy_stream()));
}

// cuda_ops.cu:220-222.  A fill kernel rather than hipMemsetAsync, so that the
// call may sit inside a graph capture; the synchronisation that makes it
// blocking like the reference's cudaMemset is skipped while capturing (a
// capture cannot synchronise its stream).
void cuda_memset(void *ptr, int value, size_t size)
{
    if (size == 0) return;
    holo::fill_bytes(ptr, value, size);
    if (!holo::stream_capturing()) HOLO_CHECK(hipStreamSynchronize(g_stream));
}

void cuda_sync(void) { HOLO_CHECK(hipDeviceSynchronize()); }  // cuda_ops.cu:222-224

void cuda_sync_copy(void)  // cuda_ops.cu:227-229
{
    if (g_copy_stream) HOLO_CHECK(hipStreamSynchronize(g_copy_stream));
}

// ---- extensions ------------------------------------------------------------

void holo_set_stream(void *s) { g_stream = (hipStream_t)s; }
void *holo_get_stream(void) { return (void *)g_stream; }

void *holo_stream_create(void)
{
    hipStream_t s = nullptr;
    HOLO_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    return (void *)s;
}

void holo_stream_destroy(void *s)
{
    if (s) HOLO_CHECK(hipStreamDestroy((hipStream_t)s));
}

void *holo_event_create(void)
{
    hipEvent_t e = nullptr;
    HOLO_CHECK(hipEventCreate(&e));
    return (void *)e;
}

void holo_event_record(void *ev) { HOLO_CHECK(hipEventRecord((hipEvent_t)ev, g_stream)); }

float holo_event_elapsed_ms(void *start, void *stop)
{
    float ms = 0.0f;
    HOLO_CHECK(hipEventSynchronize((hipEvent_t)stop));
    HOLO_CHECK(hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop));
    return ms;
}

void holo_event_destroy(void *ev)
{
    if (ev) HOLO_CHECK(hipEventDestroy((hipEvent_t)ev));
}

int holo_graph_begin(void)
{
    if (g_stream == nullptr) {
        HOLO_REJECT("holo_graph_begin: set a non-null library stream first");
        return -1;
    }
    hipError_t e = hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) {
        holo::latch_error((int)e, "hipStreamBeginCapture", __FILE__, __LINE__);
        return -1;
    }
    return 0;
}

void *holo_graph_end(void)
{
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipStreamEndCapture(g_stream, &g);
    if (e != hipSuccess) {
        holo::latch_error((int)e, "hipStreamEndCapture", __FILE__, __LINE__);
        return nullptr;
    }
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
        holo::latch_error((int)e, "hipGraphInstantiate", __FILE__, __LINE__);
        return nullptr;
    }
    return (void *)ge;
}

int holo_graph_launch(void *graph_exec)
{
    hipError_t e = hipGraphLaunch((hipGraphExec_t)graph_exec, g_stream);
    if (e != hipSuccess) {
        holo::latch_error((int)e, "hipGraphLaunch", __FILE__, __LINE__);
        return -1;
    }
    return 0;
}

void holo_graph_destroy(void *graph_exec)
{
    if (graph_exec) HOLO_CHECK(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
}

}  // extern "C"
