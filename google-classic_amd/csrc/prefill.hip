// prefill.hip -- batched prefill product over Q4_0 weights: activations are
// quantised per row and 32-block to Q8_0, and the int8 x int8 block dots run
// on MFMA (v_mfma_i32_16x16x32_i8, one instruction per 16x16 tile and block).
//
// The reference has no batched path (its prompt loop is one GEMV per token,
// src/ai/llm.c:1049) and no activation quantiser; this is the build's own
// specification, restated on the CPU in oracle/holo_oracle.c
// (oracle_quantize_act_q8_0, oracle_gemm_q4_0_q8_0):
//   quantise  d = f16_rne(amax/127), id = 1/(amax/127) (0 if amax = 0),
//             q = clamp(roundf(x*id), -127, 127)
//   product   Y[m][n] = sum over blocks b, in order, of
//             (float)I[m,n,b] * (f16(dw[n,b]) * f16(dx[m,b])),
//             I = sum_k (qw-8)*qx exact in int32, each step rounded as written
// Every rounding is specified, so the GPU result is bit-identical to the
// CPU restatement (no FMA contraction in this file).
#include "common.h"
#include "quant_blocks.h"

#pragma clang fp contract(off)

namespace holo {

typedef int v4i __attribute__((ext_vector_type(4)));

// ---- activation quantiser: one thread per 32-block --------------------------

__global__ __launch_bounds__(256) void quantize_q8_0_k(uint8_t *__restrict__ out, const float *__restrict__ X,
                                                       int64_t nblocks)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    const float *x = X + g * 32;
    float amax = 0.f;
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t *o = out + g * 34;
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)d);  // v_cvt_f16_f32, round to nearest even
    o[0] = (uint8_t)(h & 0xFF);
    o[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 32; j++) {
        int q = (int)roundf(x[j] * id);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
        o[2 + j] = (uint8_t)(int8_t)q;
    }
}

// ---- GEMM ------------------------------------------------------------------------
// Workgroup: 64 (M) x 64 (N) output tile, 4 waves each owning 32 x 32 (2 x 2
// MFMA tiles of 16 x 16).  Per 32-block of K the tile's 64 activation blocks
// and 64 weight blocks are staged in LDS as 32 int8 per row (weights
// unpacked to q-8) plus the two f16 scales; the next block's raw bytes are
// loaded into registers while the current one is multiplied.
//
// v_mfma_i32_16x16x32_i8 operand layout (wave64): lane l supplies A row
// l%16, k = 8*(l/16) .. +7 and B column l%16, same k range; it receives
// D[i][j] for j = l%16, i = 4*(l/16) + 0..3.

constexpr int kTM = 64, kTN = 64;

struct GemmArgs {
    float *Y;
    const uint8_t *W;   // Q4_0 [N][K/32]
    const uint8_t *Xq;  // Q8_0 [M][K/32]
    int M, N, nb;
};

// Signed bytes (q - 8) of four nibbles held one per byte.
__device__ __forceinline__ uint32_t nib_to_s8(uint32_t nib)
{
    uint32_t t = nib ^ 0x08080808u;                      // 4-bit two's complement of q-8
    uint32_t sign = ((t >> 3) & 0x01010101u) * 0xF0u;    // extend bit 3 into bits 4..7
    return t | sign;
}

__global__ __launch_bounds__(256) void gemm_q4_0_q8_0_k(GemmArgs a)
{
    __shared__ uint4 lA[kTM * 2];  // [m][32 bytes]
    __shared__ uint4 lB[kTN * 2];  // [n][32 bytes]
    __shared__ float lsa[kTM], lsb[kTN];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m_base = blockIdx.y * kTM, n_base = blockIdx.x * kTN;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;

    // staging roles: threads 0..63 -> activation row, 64..127 -> weight row
    const bool stA = tid < 64, stB = tid >= 64 && tid < 128;
    const int srow = tid & 63;
    const int am = min(m_base + srow, a.M - 1), bn = min(n_base + srow, a.N - 1);
    const int64_t a_total = (int64_t)a.M * a.nb * 34, b_total = (int64_t)a.N * a.nb * 18;

    Q8_0Unit ra;
    Q4_0Unit rb;
    auto fetch = [&](int b) {
        if (stA) ra = load_q8_0(a.Xq, (int64_t)am * a.nb + b, a_total);
        if (stB) rb = load_q4_0(a.W, (int64_t)bn * a.nb + b, b_total);
    };

    float acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.f;

    fetch(0);
    for (int b = 0; b < a.nb; b++) {
        __syncthreads();  // previous block's LDS reads are done
        if (stA) {
            lA[srow * 2] = make_uint4(ra.q[0], ra.q[1], ra.q[2], ra.q[3]);
            lA[srow * 2 + 1] = make_uint4(ra.q[4], ra.q[5], ra.q[6], ra.q[7]);
            lsa[srow] = ra.d;
        }
        if (stB) {
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = nib_to_s8(rb.q[i] & 0x0F0F0F0Fu);         // k = 4i .. 4i+3
                hi[i] = nib_to_s8((rb.q[i] >> 4) & 0x0F0F0F0Fu);  // k = 16+4i ..
            }
            lB[srow * 2] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            lB[srow * 2 + 1] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            lsb[srow] = rb.d;
        }
        __syncthreads();
        if (b + 1 < a.nb) fetch(b + 1);

        const uint8_t *pA = (const uint8_t *)lA, *pB = (const uint8_t *)lB;
        const int kq = 8 * (lane >> 4);
#pragma unroll
        for (int mi = 0; mi < 2; mi++) {
            const long av = *(const long *)(pA + (wm + mi * 16 + (lane & 15)) * 32 + kq);
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                const int n0 = wn + ni * 16;
                const long bv = *(const long *)(pB + (n0 + (lane & 15)) * 32 + kq);
                const v4i zero = {0, 0, 0, 0};
                const v4i I = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, zero, 0, 0, 0);
                const float dw = lsb[n0 + (lane & 15)];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float dx = lsa[wm + mi * 16 + 4 * (lane >> 4) + r];
                    const float s = dw * dx;
                    const float t = (float)I[r] * s;
                    acc[mi][ni][r] = acc[mi][ni][r] + t;
                }
            }
        }
    }

#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m_base + wm + mi * 16 + 4 * (lane >> 4) + r;
                const int n = n_base + wn + ni * 16 + (lane & 15);
                if (m < a.M && n < a.N) a.Y[(int64_t)m * a.N + n] = acc[mi][ni][r];
            }
}

}  // namespace holo

using namespace holo;

extern "C" {

void holo_quantize_act_q8_0(void *dst_blocks, const float *X, int rows, int k)
{
    if (rows <= 0 || k < 32) return;
    if (!dst_blocks || !X) {
        HOLO_REJECT("holo_quantize_act_q8_0: null pointer");
        return;
    }
    if (k % 32 != 0) {
        HOLO_REJECT("holo_quantize_act_q8_0: k must be a multiple of 32");
        return;
    }
    const int64_t nb = (int64_t)rows * (k / 32);
    hipLaunchKernelGGL(quantize_q8_0_k, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, stream(),
                       (uint8_t *)dst_blocks, X, nb);
    HOLO_LAUNCH_CHECK();
}

void holo_gemm_q4_0_q8_0(float *Y, const void *W, const void *Xq, int M, int N, int K)
{
    if (M <= 0 || N <= 0) return;
    if (!Y || !W || !Xq || K % 32 != 0 || K <= 0) {
        HOLO_REJECT("holo_gemm_q4_0_q8_0: null pointer or K not a positive multiple of 32");
        return;
    }
    if ((((uintptr_t)W) & 3u) || (((uintptr_t)Xq) & 3u)) {
        HOLO_REJECT("holo_gemm_q4_0_q8_0: W and Xq must be 4-byte aligned");
        return;
    }
    GemmArgs a = {Y, (const uint8_t *)W, (const uint8_t *)Xq, M, N, K / 32};
    dim3 grid((N + kTN - 1) / kTN, (M + kTM - 1) / kTM);
    hipLaunchKernelGGL(gemm_q4_0_q8_0_k, grid, dim3(256), 0, stream(), a);
    HOLO_LAUNCH_CHECK();
}

void holo_matmul_batch_q4_0(float *Y, const void *W, const float *X, int M, int N, int K, void *scratch_q8)
{
    if (M <= 0 || N <= 0) return;
    if (M < 64) {
        for (int m = 0; m < M; m++) cuda_matmul_q4_0(Y + (int64_t)m * N, W, X + (int64_t)m * K, N, K);
        return;
    }
    void *q = scratch_q8;
    if (!q) HOLO_CHECK(hipMallocAsync(&q, (size_t)M * (K / 32) * 34, stream()));
    if (!q) return;
    holo_quantize_act_q8_0(q, X, M, K);
    holo_gemm_q4_0_q8_0(Y, W, q, M, N, K);
    if (!scratch_q8) HOLO_CHECK(hipFreeAsync(q, stream()));
}

}  // extern "C"
