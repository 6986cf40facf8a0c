// Wave64 and workgroup reductions shared by the row kernels (RMS norm, the
// normed activation halves of the batched product): one summation order, so
// kernels that reduce the same values get the same bits.
#pragma once
#include <hip/hip_runtime.h>

__device__ __forceinline__ float wave_reduce_sum(float v)
{
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_reduce_max(float v)
{
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// Sum (or max) over the whole workgroup; every thread gets the result.
template <bool MAX>
__device__ float block_reduce(float v, float *scratch)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nw = (blockDim.x + 63) >> 6;
    v = MAX ? wave_reduce_max(v) : wave_reduce_sum(v);
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < nw; w++) r = MAX ? fmaxf(r, scratch[w]) : r + scratch[w];
    return r;
}
