// common.h -- shared host/device definitions of libholo_mi355x.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/cuda_ops.h"
#include "../../include/holo_mi355x.h"

namespace holo {

// Word 3 of a raw buffer resource (gfx9: 32-bit data format, no swizzle):
// loads past its byte range return zeros.
constexpr uint32_t kRawBufWord3 = 0x00020000u;

// Library stream (null stream unless holo_set_stream was called) and the
// copy stream of cuda_memcpy_*_async (reference cuda_ops.cu:88-89).
hipStream_t stream();
hipStream_t copy_stream();

// Error latch: first error wins until holo_last_error() reads it.
void latch_error(int code, const char *what, const char *file, int line);

// Number of compute units of device 0, read once at init.
int num_cus();

// Barrier words of the persistent decode-step kernel (gemv_stream.hip).
bool gemv_stream_init();
void gemv_stream_release();
// The decode-attention range partials (16 MiB), allocated once by cuda_init;
// without them decode attention runs one range per head.
bool attention_scratch_init();
void attention_scratch_release();
void panel_workspace_release();  // the batched products' panel buffers (prefill.hip)
// The batched products' kept workspaces (prefill.hip): slot 0 weight panels,
// slot 1 activation panels, slot 2 the exact product's split-K partials.  A device buffer of at least `bytes`, grown with
// hipMalloc outside graph capture and reused in stream order; nullptr under
// capture or when growing fails (the caller then allocates stream-ordered).
void *workspace(int slot, size_t bytes);
// The exact batched product (prefill_exact.hip): whether a weight type and
// stream take it, and the product itself (Y[i] = X . W[i]^T, or of silu(X) *
// U, plus R for one matrix).
bool exact_ok(int type, int K, const void *W);
// The exact product's tile counters (split-K form), allocated once by cuda_init.
bool exact_init();
void exact_release();
// With NW, the rows of X are RMS-normed first (weight NW, K <= 16384, 16-byte
// aligned), as holo_rms_norm_rows computes them, inside the activation halves.
void exact_product(float *const *Y, const void *const *W, const int *types, const int *N, int nmat, const float *X,
                   const float *U, const float *R, int M, int K, const float *NW = nullptr, float eps = 0.f);
// The exact route for nmat matrices of rows RMS-normed on the way in, when
// the prefill mode and the shapes take it; false (nothing launched) otherwise.
bool exact_product_normed(float *const *Y, const void *const *W, const int *types, const int *N, int nmat,
                          const float *X, const float *NW, float eps, int M, int K);
// The Q8_0 product on the int8 matrix cores (prefill_i8.hip): whether it takes
// the shapes, its activation panel's bytes (<= the f16 kernel's), and the
// product into a caller-given panel workspace.
bool q8i8_fits(const void *const *W, const int *N, int nmat, int M, int K);
size_t q8i8_panel_bytes(int M, int K);
void q8i8_product(float *const *Y, const void *const *W, const int *N, int nmat, const void *Xq, int M, int K,
                  void *ws);
// Device address of the fixed scratch array of holo_gemm_q4_0_q8_0_noalloc on
// the current device (prefill.hip), looked up once per device; nullptr on failure.
void *noalloc_scratch();

// Events that holo_time_next_launch requested for the next timed kernel
// launch (MFMA GEMV or prefill GEMM): returns them once and clears them.
bool take_launch_events(hipEvent_t *start, hipEvent_t *stop);

// A launch on the library stream that records the events armed by
// holo_time_next_launch, if any, at the kernel's own start and end.
template <typename... KArgs, typename... Args>
inline void launch_timed(void (*kern)(KArgs...), dim3 grid, dim3 block, size_t lds, Args... args)
{
    hipEvent_t e0, e1;
    if (take_launch_events(&e0, &e1))
        hipExtLaunchKernelGGL(kern, grid, block, lds, stream(), e0, e1, 0, args...);
    else
        hipLaunchKernelGGL(kern, grid, block, lds, stream(), args...);
}

// n bytes at p set to `value` by a kernel on the library stream.  Used
// instead of hipMemsetAsync wherever a call may be captured into a graph
// (memset nodes are avoided in captured graphs).
void fill_bytes(void *p, int value, size_t n);

// True while the library stream is being captured into a graph.
bool stream_capturing();

}  // namespace holo

#define HOLO_CHECK(call)                                                        \
    do {                                                                        \
        hipError_t holo_e_ = (call);                                            \
        if (holo_e_ != hipSuccess) holo::latch_error((int)holo_e_, #call, __FILE__, __LINE__); \
    } while (0)

// After a kernel launch: catch launch-configuration errors immediately.
#define HOLO_LAUNCH_CHECK() HOLO_CHECK(hipGetLastError())

#define HOLO_REJECT(msg) holo::latch_error(HOLO_EINVAL, (msg), __FILE__, __LINE__)
