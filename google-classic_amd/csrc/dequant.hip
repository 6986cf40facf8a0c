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

#pragma clang fp contract(off)

namespace holo {

__global__ __launch_bounds__(256) void dequant_q4_0_kernel(float *__restrict__ y, const uint8_t *__restrict__ W,
                                                            int64_t nblocks)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    Q4_0Unit u = load_q4_0(W, g, nblocks * 18);
    float *o = y + g * 32;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t b = (u.q[i] >> (8 * k)) & 0xFFu;
            o[4 * i + k] = u.d * (float)((int)(b & 15u) - 8);
            o[16 + 4 * i + k] = u.d * (float)((int)(b >> 4) - 8);
        }
    }
}

__global__ __launch_bounds__(256) void dequant_q8_0_kernel(float *__restrict__ y, const uint8_t *__restrict__ W,
                                                            int64_t nblocks)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    Q8_0Unit u = load_q8_0(W, g, nblocks * 34);
    float *o = y + g * 32;
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            int q = (int)(int8_t)((u.q[i] >> (8 * k)) & 0xFFu);
            o[4 * i + k] = u.d * (float)q;
        }
    }
}

// One thread per sub-block (32 weights).
__global__ __launch_bounds__(256) void dequant_q4_k_kernel(float *__restrict__ y, const uint8_t *__restrict__ W,
                                                            int64_t nunits)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nunits) return;
    Q4_KUnit u = load_q4_k(W, g);
    float *o = y + g * 32;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t b = (u.q[i] >> (8 * k)) & 0xFFu;
            float p0 = u.dsc * (float)(b & 15u);
            float p1 = u.dsc * (float)(b >> 4);
            o[4 * i + k] = p0 - u.dmn;
            o[16 + 4 * i + k] = p1 - u.dmn;
        }
    }
}

// One thread per (superblock, half, l): 4 outputs at l, l+32, l+64, l+96 of
// the half (quant.c:252-268).
__global__ __launch_bounds__(256) void dequant_q6_k_kernel(float *__restrict__ y, const uint8_t *__restrict__ W,
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
    float *o = y + sbi * 256 + 128 * half;
    o[l] = (d * (float)sc[is + 0]) * (float)q1;
    o[l + 32] = (d * (float)sc[is + 2]) * (float)q2;
    o[l + 64] = (d * (float)sc[is + 4]) * (float)q3;
    o[l + 96] = (d * (float)sc[is + 6]) * (float)q4;
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
    const uint8_t *W = (const uint8_t *)src;
    switch (type) {
    case HOLO_TYPE_Q4_0: {
        int64_t nb = n / 32;
        if (nb) hipLaunchKernelGGL(dequant_q4_0_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, stream(), dst, W, nb);
        break;
    }
    case HOLO_TYPE_Q8_0: {
        int64_t nb = n / 32;
        if (nb) hipLaunchKernelGGL(dequant_q8_0_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, stream(), dst, W, nb);
        break;
    }
    case HOLO_TYPE_Q4_K: {
        int64_t nu = (n / 256) * 8;
        if (nu) hipLaunchKernelGGL(dequant_q4_k_kernel, dim3((unsigned)((nu + 255) / 256)), dim3(256), 0, stream(), dst, W, nu);
        break;
    }
    case HOLO_TYPE_Q6_K: {
        int64_t nsb = n / 256;
        if (nsb) hipLaunchKernelGGL(dequant_q6_k_kernel, dim3((unsigned)((nsb * 64 + 255) / 256)), dim3(256), 0, stream(), dst, W, nsb);
        break;
    }
    default:
        HOLO_REJECT("holo_dequant: unsupported type");
        return;
    }
    HOLO_LAUNCH_CHECK();
}
