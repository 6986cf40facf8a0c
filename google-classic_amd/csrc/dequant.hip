// dequant.hip -- standalone dequantisation, bit-identical to the reference
// CPU routines (src/ai/quant.c:118-128 Q8_0, 136-153 Q4_0, 277-311 Q4_K,
// 241-271 Q6_K).  They decode with the same helpers as the GEMV kernels, so
// the bit-exact dequant tests also cover the GEMV's realignment and unpack.
//
// Rounding: Q8_0/Q4_0 compute d*q, one exact product.  Q4_K computes
// (d*sc)*q - dmin*m with two roundings as the C source reads, so contraction
// into an FMA is disabled below.  Q6_K computes (d*sc)*q, two roundings.
#include "common.h"
#include "quant_blocks.h"

#include <type_traits>

#pragma clang fp contract(off)

namespace holo {

// Output element: the fp32 dequantised value, or that value rounded to f16
// (round to nearest even: v_cvt_f16_f32), the weight panel of the batched
// f16 product.
template <typename T>
__device__ __forceinline__ T out_of(float v);
template <>
__device__ __forceinline__ float out_of<float>(float v)
{
    return v;
}
template <>
__device__ __forceinline__ _Float16 out_of<_Float16>(float v)
{
    // The empty asm makes v a register value: without it the compiler folds
    // the last multiply and the conversion into v_fma_mixlo_f16(a, b, +0),
    // which rounds the exact product to f16 once (not f32, then f16) and
    // turns a -0 product into +0.
    asm("" : "+v"(v));
    return (_Float16)v;
}

// The 32 values of one block to o: fp32 as 32 stores (o is only 4-byte
// aligned in holo_dequant); f16 packed in pairs and written as four 16-byte
// stores (holo_dequant_f16 requires a 16-byte-aligned panel).
template <typename T>
__device__ __forceinline__ void store32(T *o, const float (&v)[32]);
template <>
__device__ __forceinline__ void store32<float>(float *o, const float (&v)[32])
{
#pragma unroll
    for (int i = 0; i < 32; i++) o[i] = v[i];
}
template <>
__device__ __forceinline__ void store32<_Float16>(_Float16 *o, const float (&v)[32])
{
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const uint32_t lo = __builtin_bit_cast(uint16_t, out_of<_Float16>(v[2 * i]));
        const uint32_t hi = __builtin_bit_cast(uint16_t, out_of<_Float16>(v[2 * i + 1]));
        w[i] = lo | (hi << 16);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) ((uint4 *)o)[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
}

template <typename T>
__global__ __launch_bounds__(256) void dequant_q4_0_kernel(T *__restrict__ y, const uint8_t *__restrict__ W,
                                                            int64_t nblocks)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    Q4_0Unit u = load_q4_0(W, g, nblocks * 18);
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t b = (u.q[i] >> (8 * k)) & 0xFFu;
            v[4 * i + k] = u.d * (float)((int)(b & 15u) - 8);
            v[16 + 4 * i + k] = u.d * (float)((int)(b >> 4) - 8);
        }
    }
    store32<T>(y + g * 32, v);
}

template <typename T>
__global__ __launch_bounds__(256) void dequant_q8_0_kernel(T *__restrict__ y, const uint8_t *__restrict__ W,
                                                            int64_t nblocks)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    Q8_0Unit u = load_q8_0(W, g, nblocks * 34);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            int q = (int)(int8_t)((u.q[i] >> (8 * k)) & 0xFFu);
            v[4 * i + k] = u.d * (float)q;
        }
    }
    store32<T>(y + g * 32, v);
}

// One thread per sub-block (32 weights).
template <typename T>
__global__ __launch_bounds__(256) void dequant_q4_k_kernel(T *__restrict__ y, const uint8_t *__restrict__ W,
                                                            int64_t nunits)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nunits) return;
    Q4_KUnit u = load_q4_k(W, g);
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t b = (u.q[i] >> (8 * k)) & 0xFFu;
            float p0 = u.dsc * (float)(b & 15u);
            float p1 = u.dsc * (float)(b >> 4);
            v[4 * i + k] = p0 - u.dmn;
            v[16 + 4 * i + k] = p1 - u.dmn;
        }
    }
    store32<T>(y + g * 32, v);
}

// One thread per (superblock, half, l): 4 outputs at l, l+32, l+64, l+96 of
// the half (quant.c:252-268).
template <typename T>
__global__ __launch_bounds__(256) void dequant_q6_k_kernel(T *__restrict__ y, const uint8_t *__restrict__ W,
                                                            int64_t nsb)
{
    int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nsb * 64) return;
    int64_t sbi = t >> 6;
    int half = (int)((t >> 5) & 1);
    int l = (int)(t & 31);
    const uint8_t *sb = W + sbi * 210;
    const uint8_t *ql = sb + 64 * half;
    const uint8_t *qh = sb + 128 + 32 * half;
    const int8_t *sc = (const int8_t *)(sb + 192) + 8 * half;
    float d = half_bits_to_float_exact((uint32_t)sb[208] | ((uint32_t)sb[209] << 8));
    int is = l / 16;
    int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
    int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
    int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
    int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
    T *o = y + sbi * 256 + 128 * half;
    o[l] = out_of<T>((d * (float)sc[is + 0]) * (float)q1);
    o[l + 32] = out_of<T>((d * (float)sc[is + 2]) * (float)q2);
    o[l + 64] = out_of<T>((d * (float)sc[is + 4]) * (float)q3);
    o[l + 96] = out_of<T>((d * (float)sc[is + 6]) * (float)q4);
}

// Q6_K to f16 panel values, one thread per (superblock, half h, slice s):
// l = 16s .. 16s + 15 of the half, all four j, i.e. y[256b + 128h + 32j + l]
// = (d * sc[8h + s + 2j]) * (q_j - 32) with both roundings as
// dequantize_row_q6_k (quant.c:252-268), then to f16.  The 64 values come
// from three 16-byte runs (ql low / high part, qh) and leave as eight 16-byte
// stores.
__global__ __launch_bounds__(256) void dequant_q6_k_f16_kernel(_Float16 *__restrict__ y, const uint8_t *__restrict__ W,
                                                               int64_t ntask)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= ntask) return;
    const int64_t b = t >> 2;
    const int h = (int)((t >> 1) & 1), sl = (int)(t & 1);
    const uint8_t *sb = W + b * 210;
    uint32_t qa[4], qb[4], qh[4];
    q6_run16(sb + 64 * h + 16 * sl, qa);
    q6_run16(sb + 64 * h + 32 + 16 * sl, qb);
    q6_run16(sb + 128 + 32 * h + 16 * sl, qh);
    const int8_t *sc = (const int8_t *)(sb + 192) + 8 * h;
    const float d = half_bits_to_float_exact((uint32_t)sb[208] | ((uint32_t)sb[209] << 8));
    _Float16 *o = y + b * 256 + 128 * h + 16 * sl;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t *ql = (j & 1) ? qb : qa;
        const float ds = d * (float)sc[sl + 2 * j];
        uint32_t w[8];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t q = ((ql[c] >> (4 * (j >> 1))) & 0x0F0F0F0Fu) | (((qh[c] >> (2 * j)) & 0x03030303u) << 4);
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = ds * (float)((int)((q >> (8 * k)) & 0xFFu) - 32);
            w[2 * c] = (uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(v[0])) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(v[1])) << 16);
            w[2 * c + 1] = (uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(v[2])) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(v[3])) << 16);
        }
        uint4 *p = (uint4 *)(o + 32 * j);
        p[0] = make_uint4(w[0], w[1], w[2], w[3]);
        p[1] = make_uint4(w[4], w[5], w[6], w[7]);
    }
}

// Q4_K to f16 panel values, four threads per 32-weight unit: thread t of
// unit u writes weights 8t .. 8t + 7, the low nibbles of qs[8t ..] for
// t < 2 and the high nibbles of qs[8(t-2) ..] for t >= 2 (the unit layout of
// dequant_q4_k_kernel), so a wave's 16-byte stores are contiguous.  Same
// arithmetic: (d*sc)*q - dmin*m, both roundings, then f16.
__global__ __launch_bounds__(256) void dequant_q4_k_f16_kernel(_Float16 *__restrict__ y, const uint8_t *__restrict__ W,
                                                               int64_t nthreads)
{
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nthreads) return;
    const int64_t u = g >> 2;
    const int t = (int)(g & 3);
    const uint8_t *sb = W + (u >> 3) * 144;
    const uint32_t j = (uint32_t)(u & 7);
    const u32x4 h = *(const u32x4 *)sb;
    const uint2 q = *(const uint2 *)(sb + 16 + 16 * j + 8 * (t & 1));
    uint32_t sc, mn;
    q4_k_scale_min(h.y, h.z, h.w, j, sc, mn);
    const float dsc = half_bits_to_float(h.x) * (float)sc;
    const float dmn = half_bits_to_float(h.x >> 16) * (float)mn;
    const int shift = t >= 2 ? 4 : 0;
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t word = i < 2 ? q.x : q.y;
        const uint32_t b0 = (word >> (16 * (i & 1) + shift)) & 15u, b1 = (word >> (16 * (i & 1) + 8 + shift)) & 15u;
        const float p0 = dsc * (float)b0, p1 = dsc * (float)b1;
        w[i] = (uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(p0 - dmn)) |
               ((uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(p1 - dmn)) << 16);
    }
    ((uint4 *)(y + u * 32 + 8 * t))[0] = make_uint4(w[0], w[1], w[2], w[3]);
}

// Q4_0 / Q8_0 to f16 panel values, four threads per 32-weight block: thread t
// writes weights 8t .. 8t + 7 as one 16-byte store (contiguous across the
// wave).  Each thread decodes the whole block with the realigning loaders
// (the four loads of a block hit the same lines) and takes its 8 weights:
// Q8_0 qs[8t ..]; Q4_0 the low nibbles of qs[8t ..] for t < 2, the high
// nibbles of qs[8(t-2) ..] for t >= 2.  d*q is exact in fp32, then f16.
template <bool Q8>
__global__ __launch_bounds__(256) void dequant_q8_q4_f16_kernel(_Float16 *__restrict__ y, const uint8_t *__restrict__ W,
                                                                int64_t nthreads, int64_t nblocks)
{
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nthreads) return;
    const int64_t b = g >> 2;
    const int t = (int)(g & 3);
    float v[8];
    if constexpr (Q8) {
        const Q8_0Unit u = load_q8_0(W, b, nblocks * 34);
#pragma unroll
        for (int k = 0; k < 8; k++)
            v[k] = u.d * (float)(int)(int8_t)((u.q[2 * t + (k >> 2)] >> (8 * (k & 3))) & 0xFFu);
    } else {
        const Q4_0Unit u = load_q4_0(W, b, nblocks * 18);
        const int shift = t >= 2 ? 4 : 0;
#pragma unroll
        for (int k = 0; k < 8; k++)
            v[k] = u.d * (float)((int)((u.q[2 * (t & 1) + (k >> 2)] >> (8 * (k & 3) + shift)) & 15u) - 8);
    }
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        w[i] = (uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(v[2 * i])) |
               ((uint32_t)__builtin_bit_cast(uint16_t, out_of<_Float16>(v[2 * i + 1])) << 16);
    ((uint4 *)(y + b * 32 + 8 * t))[0] = make_uint4(w[0], w[1], w[2], w[3]);
}

// F32 rows to f16 (8 per thread; n a multiple of 8).
__global__ __launch_bounds__(256) void f32_to_f16_kernel(_Float16 *__restrict__ y, const float *__restrict__ x,
                                                         int64_t n8)
{
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n8) return;
    const float4 a = ((const float4 *)x)[2 * g], b = ((const float4 *)x)[2 * g + 1];
    _Float16 *o = y + 8 * g;
    o[0] = (_Float16)a.x;
    o[1] = (_Float16)a.y;
    o[2] = (_Float16)a.z;
    o[3] = (_Float16)a.w;
    o[4] = (_Float16)b.x;
    o[5] = (_Float16)b.y;
    o[6] = (_Float16)b.z;
    o[7] = (_Float16)b.w;
}

// Launch the dequant of n weights of `type` into y; false for a type without
// a block kernel here.
template <typename T>
static bool dequant_into(T *y, const uint8_t *W, int64_t n, int type)
{
    switch (type) {
    case HOLO_TYPE_Q4_0:
    case HOLO_TYPE_Q8_0: {
        const int64_t nb = n / 32;
        if (!nb) return true;
        const bool q8 = type == HOLO_TYPE_Q8_0;
        if constexpr (std::is_same<T, _Float16>::value) {
            const dim3 grid((unsigned)((nb * 4 + 255) / 256));
            if (q8) hipLaunchKernelGGL(dequant_q8_q4_f16_kernel<true>, grid, dim3(256), 0, stream(), y, W, nb * 4, nb);
            else hipLaunchKernelGGL(dequant_q8_q4_f16_kernel<false>, grid, dim3(256), 0, stream(), y, W, nb * 4, nb);
        } else {
            const dim3 grid((unsigned)((nb + 255) / 256));
            if (q8) hipLaunchKernelGGL(dequant_q8_0_kernel<T>, grid, dim3(256), 0, stream(), y, W, nb);
            else hipLaunchKernelGGL(dequant_q4_0_kernel<T>, grid, dim3(256), 0, stream(), y, W, nb);
        }
        return true;
    }
    case HOLO_TYPE_Q4_K: {
        const int64_t nu = (n / 256) * 8;
        if (!nu) return true;
        if constexpr (std::is_same<T, _Float16>::value)
            hipLaunchKernelGGL(dequant_q4_k_f16_kernel, dim3((unsigned)((nu * 4 + 255) / 256)), dim3(256), 0,
                               stream(), y, W, nu * 4);
        else
            hipLaunchKernelGGL(dequant_q4_k_kernel<T>, dim3((unsigned)((nu + 255) / 256)), dim3(256), 0, stream(), y,
                               W, nu);
        return true;
    }
    case HOLO_TYPE_Q6_K: {
        const int64_t nsb = n / 256;
        if (!nsb) return true;
        if constexpr (std::is_same<T, _Float16>::value)
            hipLaunchKernelGGL(dequant_q6_k_f16_kernel, dim3((unsigned)((nsb * 4 + 255) / 256)), dim3(256), 0,
                               stream(), y, W, nsb * 4);
        else
            hipLaunchKernelGGL(dequant_q6_k_kernel<T>, dim3((unsigned)((nsb * 64 + 255) / 256)), dim3(256), 0,
                               stream(), y, W, nsb);
        return true;
    }
    default: return false;
    }
}

// Bit-identity holds for every finite scale (zeros, subnormals and normals).
// A NaN or Inf scale gives NaN/Inf weights here as in the reference, but the
// NaN payload bits are not specified.

}  // namespace holo

using namespace holo;

extern "C" void holo_dequant(float *dst, const void *src, int64_t n, int type)
{
    if (n <= 0) return;
    if (!dst || !src) {
        HOLO_REJECT("holo_dequant: null pointer");
        return;
    }
    if (((uintptr_t)src & 3u) != 0) {
        HOLO_REJECT("holo_dequant: source must be 4-byte aligned");
        return;
    }
    if (!dequant_into(dst, (const uint8_t *)src, n, type)) {
        HOLO_REJECT("holo_dequant: unsupported type");
        return;
    }
    HOLO_LAUNCH_CHECK();
}

extern "C" void holo_dequant_f16(void *dst, const void *src, int64_t n, int type)
{
    if (n <= 0) return;
    if (!dst || !src) {
        HOLO_REJECT("holo_dequant_f16: null pointer");
        return;
    }
    const uintptr_t sa = (uintptr_t)src;
    const bool src_ok = type == HOLO_TYPE_F32 ? (sa & 15u) == 0 : type == HOLO_TYPE_F16 ? (sa & 1u) == 0 : (sa & 3u) == 0;
    if (((uintptr_t)dst & 15u) != 0 || !src_ok || n % 32 != 0) {
        HOLO_REJECT("holo_dequant_f16: dst must be 16-byte aligned, src 16- (F32), 2- (F16) or 4-byte aligned "
                    "(blocks), n a multiple of 32");
        return;
    }
    _Float16 *y = (_Float16 *)dst;
    if (type == HOLO_TYPE_F16) {
        HOLO_CHECK(hipMemcpyAsync(y, src, (size_t)n * 2, hipMemcpyDeviceToDevice, stream()));
        return;
    }
    if (type == HOLO_TYPE_F32) {
        const int64_t n8 = n / 8;
        hipLaunchKernelGGL(f32_to_f16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream(), y,
                           (const float *)src, n8);
    } else if (!dequant_into(y, (const uint8_t *)src, n, type)) {
        HOLO_REJECT("holo_dequant_f16: unsupported type");
        return;
    }
    HOLO_LAUNCH_CHECK();
}
