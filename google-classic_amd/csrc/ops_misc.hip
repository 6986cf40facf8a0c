// ops_misc.hip -- the remaining ops of the reference boundary
// (include/cuda_ops.h): vector ops, activations, normalisation, softmax,
// attention, RoPE, embedding lookups, argmax, and the F32 / F16 / Q6_K
// GEMVs.  They are not on the quantized-matmul hot path; they exist so the
// reference inference loop (src/ai/llm_cuda.c) links and runs unchanged.
// Each follows the arithmetic of the reference kernel it replaces (cited per
// function); where the reference has a quirk, it is kept and said so.
#include "common.h"
#include "quant_blocks.h"
#include "block_reduce.h"

#include "../../include/holo_forward.h"

namespace holo {

constexpr int kBlock = 256;

static inline int blocks_for(int n, int per = kBlock) { return (n + per - 1) / per; }

// ---- block-wide reductions: block_reduce.h ----

// ---- elementwise (cuda_ops.cu:237-314, 1401-1455) ------------------------------------

__global__ void vec_add_k(float *d, const float *a, const float *b, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = a[i] + b[i];
}
__global__ void vec_mul_k(float *d, const float *a, const float *b, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = a[i] * b[i];
}
__global__ void vec_scale_k(float *d, const float *a, float s, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) d[i] = a[i] * s;
}
__global__ void silu_k(float *x, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = x[i];
        x[i] = v / (1.0f + expf(-v));
    }
}
__global__ void silu_mul_k(float *d, const float *a, const float *b, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = a[i];
        d[i] = (v / (1.0f + expf(-v))) * b[i];
    }
}
__global__ void gelu_k(float *x, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        float v = x[i];
        x[i] = 0.5f * v * (1.0f + tanhf(0.7978845608f * (v + 0.044715f * v * v * v)));
    }
}
__global__ void relu_k(float *x, int n)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n && x[i] < 0.0f) x[i] = 0.0f;
}

// ---- vec_dot (cuda_ops.cu:316-340): one workgroup, result copied back ------------------

__global__ __launch_bounds__(1024) void vec_dot_k(const float *a, const float *b, int n, float *out)
{
    __shared__ float scratch[16];
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += a[i] * b[i];
    s = block_reduce<false>(s, scratch);
    if (threadIdx.x == 0) out[0] = s;
}

// ---- RMS norm (cuda_ops.cu:1462-1504): dst = (x * (1/sqrt(ss/n + eps))) * w -------------

__global__ __launch_bounds__(1024) void rms_norm_k(float *dst, const float *x, const float *w, int n, float eps)
{
    __shared__ float scratch[16];
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_reduce<false>(ss, scratch);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

// ---- softmax (cuda_ops.cu:1520-1591) -----------------------------------------------------

__global__ __launch_bounds__(1024) void softmax_k(float *dst, const float *x, int n)
{
    __shared__ float scratch[16];
    float m = -1e30f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, x[i]);
    m = block_reduce<true>(m, scratch);
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float e = expf(x[i] - m);
        dst[i] = e;
        s += e;
    }
    s = block_reduce<false>(s, scratch);
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] *= inv;
}

// ---- attention (cuda_ops.cu:1600-1652, 1813-1952, 1960-2096) ------------------------------

__global__ void attention_scores_k(float *dst, const float *Q, const float *K, int seq_len, int kv_len, int hd,
                                   float scale)
{
    int i = blockIdx.y, j = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= seq_len || j >= kv_len) return;
    float s = 0.f;
    for (int d = 0; d < hd; d++) s += Q[(int64_t)i * hd + d] * K[(int64_t)j * hd + d];
    dst[(int64_t)i * kv_len + j] = s * scale;
}

__global__ void attention_apply_k(float *dst, const float *scores, const float *V, int seq_len, int kv_len, int hd)
{
    int i = blockIdx.y, d = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= seq_len || d >= hd) return;
    float s = 0.f;
    for (int j = 0; j < kv_len; j++) s += scores[(int64_t)i * kv_len + j] * V[(int64_t)j * hd + d];
    dst[(int64_t)i * hd + d] = s;
}

// One query head against kv_len cached positions of one KV head:
// scores = (q . k_p) / sqrt(hd), softmax, out = sum_p score_p * v_p.
// `sc` holds kv_len floats (LDS or the caller's buffer).
__device__ void attend_one(float *out, const float *q, const float *kc, const float *vc, int kv_len, int hd,
                           int kv_off, int kv_dim, float *sc, float *scratch)
{
    const float scale = 1.0f / sqrtf((float)hd);
    for (int p = threadIdx.x; p < kv_len; p += blockDim.x) {
        const float *k = kc + (int64_t)p * kv_dim + kv_off;
        float s = 0.f;
        for (int d = 0; d < hd; d++) s += q[d] * k[d];
        sc[p] = s * scale;
    }
    __syncthreads();
    float m = -1e30f;
    for (int p = threadIdx.x; p < kv_len; p += blockDim.x) m = fmaxf(m, sc[p]);
    m = block_reduce<true>(m, scratch);
    float sum = 0.f;
    for (int p = threadIdx.x; p < kv_len; p += blockDim.x) {
        float e = expf(sc[p] - m);
        sc[p] = e;
        sum += e;
    }
    sum = block_reduce<false>(sum, scratch);
    const float inv = 1.0f / sum;
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float o = 0.f;
        for (int p = 0; p < kv_len; p++) o += (sc[p] * inv) * vc[(int64_t)p * kv_dim + kv_off + d];
        out[d] = o;
    }
}

constexpr int kMaxLdsScores = 12288;  // kv_len held in LDS (48 KiB)

__global__ __launch_bounds__(256) void attention_single_k(float *dst, const float *q, const float *kc,
                                                          const float *vc, float *att_buf, int kv_len, int hd,
                                                          int kv_head, int kv_dim)
{
    __shared__ float lsc[kMaxLdsScores];
    __shared__ float scratch[16];
    float *sc = kv_len <= kMaxLdsScores ? lsc : att_buf;
    attend_one(dst, q, kc, vc, kv_len, hd, kv_head * hd, kv_dim, sc, scratch);
}

__global__ __launch_bounds__(256) void mha_k(float *dst, const float *q, const float *kc, const float *vc,
                                             int kv_len, int hd, int n_heads, int n_kv_heads)
{
    __shared__ float lsc[kMaxLdsScores];
    __shared__ float scratch[16];
    const int head = blockIdx.x;
    const int kv_head = head / (n_heads / n_kv_heads);  // GQA grouping, cuda_ops.cu:1834
    attend_one(dst + (int64_t)head * hd, q + (int64_t)head * hd, kc, vc, kv_len, hd, kv_head * hd,
               n_kv_heads * hd, lsc, scratch);
}

// ---- causal prefill attention on the matrix cores ----------------------------------
//
// The same result as attention_prefill_k (softmax((q . k_p) / sqrt(hd)) . v,
// online over key tiles, fp32), for head sizes 32, 64 and 128.  A workgroup
// takes one head and 32 query rows; its 4 waves take the 32-key tiles in turn
// (wave w: tiles w, w + 4, ...) and merge their softmax states through LDS at
// the end.  Both products leave D[i][j] in lane j + 32*((i/4)%2), register
// (i%4) + 4*(i/8).
//   scores, transposed: S^T = K Q^T on v_mfma_f32_32x32x16_f16 with K and Q
//     split into f16 halves (hi*hi + hi*lo + lo*hi, fp32 accumulation): lane
//     l supplies A[l%32][8*(l/32)+t] and B[8*(l/32)+t][l%32], t = 0..7, i.e.
//     half hh of the wave dims 16c + 8hh .. + 7 of its key row (A) and of its
//     query row (B).  Lane j + 32hh then holds query j's scores for keys
//     (r%4) + 8(r/4) + 4hh, r = 0..15: the row maximum is 15 local steps and
//     one exchange with lane j ^ 32.  (On v_mfma_f32_32x32x2_f32 the scores
//     took 64 instructions at head size 128, here 24.)
//   output, transposed: O^T += V^T P^T on v_mfma_f32_32x32x16_f16, V and P
//     split as above.  The contraction runs over the tile's 32 keys in the
//     order the probabilities sit in registers: k-step ks takes registers
//     8ks .. 8ks + 7 of lane j + 32hh (keys (r%4) + 8(r/4) + 4hh), which is
//     its B operand as it stands.  A is V: lane i + 32hh reads dims VB*i ..
//     VB*i + VB - 1 of each of the same 16 keys' rows, and element b of the
//     8 keys of step ks is its A operand for the block of dims VB*i + b.
//     (On v_mfma_f32_32x32x2_f32 this product took 64 instructions of four
//     times the f16 instruction's cycles at head size 128, here 24.)
// Workgroup g runs on XCD g mod 8 (round-robin dispatch): with the head count
// a multiple of 8, XCD x takes heads x H/8 .. (x + 1) H/8 - 1, every query
// block of each, so the XCDs get equal work and each reads its own heads' keys
// and values.  Within an XCD the first half of the query-block ranks go out
// heaviest (most keys) first and the second half lightest first: the second
// workgroup a CU receives then carries about as many key tiles as the first
// is short of the heaviest.
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 af16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 af16x8 __attribute__((ext_vector_type(8)));

// x = hi + lo exactly to 22 bits: hi = f16(x), lo = f16(x - hi) (x - hi is exact
// in fp32).  Products of split operands, hi*hi + hi*lo + lo*hi, keep the fp32
// class of the product (the lo*lo term is below 2^-22 of it).
__device__ __forceinline__ void split_f16(float x, _Float16 &hi, _Float16 &lo)
{
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// The same split of 8 values straight into MFMA operands, two at a time: one
// packed conversion for the two hi, each x - hi by v_fma_mix_f32 reading its
// hi as f16 (one instruction; exact, x - hi is an fp32), one packed
// conversion for the two lo.  Written out: the compiler turns the fused
// form into a conversion and a subtraction.
typedef _Float16 af16x2 __attribute__((ext_vector_type(2)));
typedef float af32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split8_f16(const float x[8], af16x8 &hi, af16x8 &lo)
{
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const af16x2 h = __builtin_convertvector((af32x2){x[2 * i], x[2 * i + 1]}, af16x2);
        const uint32_t hb = __builtin_bit_cast(uint32_t, h);
        af32x2 r;
        asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r.x) : "v"(hb), "v"(x[2 * i]));
        asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r.y) : "v"(hb), "v"(x[2 * i + 1]));
        const af16x2 l = __builtin_convertvector(r, af16x2);
        hi[2 * i] = h.x;
        hi[2 * i + 1] = h.y;
        lo[2 * i] = l.x;
        lo[2 * i + 1] = l.y;
    }
}

template <int HD>
__global__ __launch_bounds__(256, 2) void attn_prefill_mfma_k(float *out, const float *q, const float *kc,
                                                           const float *vc, int rows, int pos0, int n_heads,
                                                           int n_kv_heads, int nqb)
{
    constexpr int NQ = HD / 16;  // 16-dim chunks of a row: the K of one f16 score MFMA
    constexpr int VB = HD / 32;  // output blocks: lane i covers dims VB*i .. VB*i + VB - 1
    extern __shared__ float amf_lds[];
    // the waves' outputs [4 waves][32 queries][HD + 1]: the merge pass reads
    // consecutive dims of a query row (one bank each), the stores from the
    // MFMA layout put the 32 queries of a register on distinct banks
    constexpr int OS = HD + 1;
    float *lo = amf_lds;
    float *lm = lo + 4 * 32 * OS;              // [4][32] running max per query
    float *ll = lm + 4 * 32;                   // [4][64] running sum per lane
    float *lw = ll + 4 * 64;                   // [4][32] merge weight of each wave per query
    // (head, query block) of this workgroup. Query blocks go out by rank k:
    // the first ceil(nqb/2) ranks heaviest first, the rest lightest first, so
    // ranks k and k + ceil(nqb/2), which share CUs as the second workgroup
    // per CU, sum to nqb - 1 blocks and the CUs' key-tile loads come out even
    const int g = blockIdx.x, H = (nqb + 1) >> 1;
    int h, k;
    if (n_heads % 8 == 0) {
        const int hx = n_heads >> 3, i = g >> 3;  // i: the workgroup's place on its XCD
        h = (g & 7) * hx + i % hx;
        k = i / hx;
    } else {
        h = g % n_heads;
        k = g / n_heads;
    }
    const int qb = k < H ? nqb - 1 - k : k - H;
    const int q0 = qb * 32;
    const int lane = threadIdx.x & 63, j = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // uniform: the tiles' resources stay scalar
    const int kvh = h / (n_heads / n_kv_heads);
    const int64_t q_dim = (int64_t)n_heads * HD, kv_dim = (int64_t)n_kv_heads * HD;
    // scores in log2 units: (q . k) / sqrt(hd) * log2(e), so that each
    // probability is one v_exp_f32 (2^x) instead of a full expf
    const float scale = 1.0f / sqrtf((float)HD) * 1.44269504088896341f;
    const int last_key = pos0 + min(q0 + 32, rows) - 1;  // the furthest position a query here sees
    const int ntiles = last_key / 32 + 1;
    const int qpos = pos0 + q0 + j;  // rows past the prompt: computed, not stored

    // The block's 32 query rows in LDS, split into f16 halves ([32][HD + 8]
    // each: the pad puts the rows a 16-byte read pass touches on distinct
    // banks), read per step rather than held in registers: held, the kernel
    // needed more than 256 registers and ran one wave per SIMD.  The rows alias
    // the merge buffer lo, which is written only after every wave has left the
    // loop.
    constexpr int QS = HD + 8;
    _Float16 *qh = (_Float16 *)amf_lds, *ql = qh + 32 * QS;
    for (int e = threadIdx.x; e < 32 * (HD / 4); e += 256) {
        const int r = e / (HD / 4), c4 = e - r * (HD / 4);
        const float4 x = *(const float4 *)(q + (int64_t)min(q0 + r, rows - 1) * q_dim + (int64_t)h * HD + 4 * c4);
        _Float16 hv[4], lv[4];
        split_f16(x.x, hv[0], lv[0]);
        split_f16(x.y, hv[1], lv[1]);
        split_f16(x.z, hv[2], lv[2]);
        split_f16(x.w, hv[3], lv[3]);
        *(af16x4 *)(qh + r * QS + 4 * c4) = af16x4{hv[0], hv[1], hv[2], hv[3]};
        *(af16x4 *)(ql + r * QS + 4 * c4) = af16x4{lv[0], lv[1], lv[2], lv[3]};
    }
    __syncthreads();
    const _Float16 *qhr = qh + j * QS + 8 * hh, *qlr = ql + j * QS + 8 * hh;
    // keys and values through buffer resources based at each tile's first
    // key: the lane offsets are fixed for the launch, the rows' offsets are
    // wave-uniform, and rows past last_key fall outside the range and read
    // zeros (their scores are masked and their probabilities 0)
    const float *khead = kc + (int64_t)kvh * HD, *vhead = vc + (int64_t)kvh * HD;
    const uint32_t rowb = (uint32_t)kv_dim * 4u;
    const uint32_t kvo = (uint32_t)j * rowb + 32u * (uint32_t)hh;          // key j, dims 8hh ..
    const uint32_t vvo = 4u * (uint32_t)hh * rowb + 4u * VB * (uint32_t)j;  // key 4hh + .., dims VB j ..
    float m = -INFINITY, l = 0.f;
    v16f o[VB];
#pragma unroll
    for (int b = 0; b < VB; b++) o[b] = v16f{};

    for (int t = wave; t < ntiles; t += 4) {
        const int key0 = t * 32;
        // Sᵀ = K Qᵀ on v_mfma_f32_32x32x16_f16 with both operands split:
        // lane j + 32hh supplies dims 16c + 8hh .. 16c + 8hh + 7 of key j (A) and
        // of query j (B), as the 32x32x2 f32 layout did for its dims, so the
        // scores land in the same registers
        const int nk = min(32, last_key + 1 - key0);  // keys of the tile inside the range
        const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(khead + (int64_t)key0 * kv_dim), (short)0, (int)((uint32_t)nk * rowb), kRawBufWord3);
        const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
            (void *)(vhead + (int64_t)key0 * kv_dim), (short)0, (int)((uint32_t)nk * rowb), kRawBufWord3);
        float4 kr[2 * NQ];
#pragma unroll
        for (int c = 0; c < NQ; c++) {
            kr[2 * c] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(kvo + 64 * c), 0, 0));
            kr[2 * c + 1] =
                __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)(kvo + 64 * c + 16), 0, 0));
        }
        // the output product's 16 key row pieces, loaded with the keys so that
        // their round trip runs under the scores
        float vv[16][VB];
#pragma unroll
        for (int st = 0; st < 16; st++) {
            const int so = (int)((uint32_t)((st & 3) + 8 * (st >> 2)) * rowb);  // wave-uniform
            if constexpr (VB == 4) {
                const float4 v = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rv, (int)vvo, so, 0));
                vv[st][0] = v.x;
                vv[st][1] = v.y;
                vv[st][2] = v.z;
                vv[st][3] = v.w;
            } else if constexpr (VB == 2) {
                const float2 v = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rv, (int)vvo, so, 0));
                vv[st][0] = v.x;
                vv[st][1] = v.y;
            } else {
                vv[st][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rv, (int)vvo, so, 0));
            }
        }
        v16f s = v16f{};
#pragma unroll
        for (int c = 0; c < NQ; c++) {
            const float kv[8] = {kr[2 * c].x,     kr[2 * c].y,     kr[2 * c].z,     kr[2 * c].w,
                                 kr[2 * c + 1].x, kr[2 * c + 1].y, kr[2 * c + 1].z, kr[2 * c + 1].w};
            af16x8 kh, kl;
            split8_f16(kv, kh, kl);
            const af16x8 bh = *(const af16x8 *)(qhr + 16 * c), bl = *(const af16x8 *)(qlr + 16 * c);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, bh, s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, bl, s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kl, bh, s, 0, 0, 0);
            // one chunk's split and query reads at a time (hoisting them all
            // took the kernel past 256 registers)
            __builtin_amdgcn_sched_barrier(0);
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int key = key0 + (r & 3) + 8 * (r >> 2) + 4 * hh;
            s[r] = key <= qpos ? s[r] * scale : -INFINITY;
            tmax = fmaxf(tmax, s[r]);
        }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        const float mnew = fmaxf(m, tmax);
        // a query with no key yet (every key so far past it) keeps m = -inf, l = 0
        const bool none = mnew == -INFINITY;
        const float corr = none ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            s[r] = none ? 0.f : __builtin_amdgcn_exp2f(s[r] - mnew);
            ps += s[r];
        }
        l = l * corr + ps;
        m = mnew;
#pragma unroll
        for (int b = 0; b < VB; b++) o[b] *= corr;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const float pv[8] = {s[8 * ks],     s[8 * ks + 1], s[8 * ks + 2], s[8 * ks + 3],
                                 s[8 * ks + 4], s[8 * ks + 5], s[8 * ks + 6], s[8 * ks + 7]};
            af16x8 bh, bl;
            split8_f16(pv, bh, bl);
#pragma unroll
            for (int b = 0; b < VB; b++) {
                float v8[8];
#pragma unroll
                for (int t2 = 0; t2 < 8; t2++) v8[t2] = vv[8 * ks + t2][b];
                af16x8 ah, al;
                split8_f16(v8, ah, al);
                o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bh, o[b], 0, 0, 0);
                o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, bl, o[b], 0, 0, 0);
                o[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, bh, o[b], 0, 0, 0);
            }
        }
    }

    // merge the 4 waves: O = sum_w 2^(m_w - M) O_w / L, L = sum_w 2^(m_w - M) l_w
    __syncthreads();  // every wave is done with the query rows in lo
#pragma unroll
    for (int b = 0; b < VB; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int i = (r & 3) + 8 * (r >> 2) + 4 * hh;
            lo[(wave * 32 + j) * OS + VB * i + b] = o[b][r];
        }
    if (hh == 0) lm[wave * 32 + j] = m;
    ll[wave * 64 + lane] = l;
    __syncthreads();
    // each query's four weights 2^(m_w - M) / L, once per query rather than
    // per output element
    if (threadIdx.x < 32) {
        const int qj = threadIdx.x;
        float M = lm[qj];
#pragma unroll
        for (int w = 1; w < 4; w++) M = fmaxf(M, lm[w * 32 + qj]);
        float wg[4], L = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float mw = lm[w * 32 + qj];
            wg[w] = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
            L += wg[w] * (ll[w * 64 + qj] + ll[w * 64 + 32 + qj]);
        }
#pragma unroll
        for (int w = 0; w < 4; w++) lw[w * 32 + qj] = wg[w] / L;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 32 * HD; e += 256) {
        const int qj = e / HD, d = e - qj * HD;  // consecutive threads: consecutive dims of one row
        if (q0 + qj >= rows) continue;
        float O = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) O += lw[w * 32 + qj] * lo[(w * 32 + qj) * OS + d];
        out[(int64_t)(q0 + qj) * q_dim + (int64_t)h * HD + d] = O;
    }
}

template <int HD>
static void launch_attn_prefill_mfma(float *out, const float *q, const float *kc, const float *vc, int rows, int pos0,
                                     int n_heads, int n_kv_heads)
{
    constexpr size_t lds = (size_t)(4 * 32 * (HD + 1) + 4 * 32 + 4 * 64 + 4 * 32) * sizeof(float);
    static bool attr = false;
    if (!attr) {
        HOLO_CHECK(hipFuncSetAttribute((const void *)attn_prefill_mfma_k<HD>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        attr = true;
    }
    const int nqb = (rows + 31) / 32;
    hipLaunchKernelGGL(attn_prefill_mfma_k<HD>, dim3((unsigned)(nqb * n_heads)), dim3(256), lds, stream(), out, q, kc,
                       vc, rows, pos0, n_heads, n_kv_heads, nqb);
    HOLO_LAUNCH_CHECK();
}

// ---- Q6_K GEMV (cuda_matmul_q6_k) ---------------------------------------------------
//
// 210-byte superblocks of 256 weights (quant.h:103-110): ql[128] low
// nibbles, qh[64] high bit pairs, int8 scales[16], f16 d.  dequantize_row_q6_k
// (quant.c:241-271) gives, for half h and l = 0..31, the 4 weights
//   y[128h + 32j + l] = (d * sc[8h + l/16 + 2j]) * (q_j - 32),
//   q_j = ((ql[64h + l + 32(j&1)] >> 4(j>>1)) & 15) | (((qh[32h + l] >> 2j) & 3) << 4).
// Lane task (b, h, s): superblock b, half h, l = 16s .. 16s + 15, all four j:
// 64 weights from three 16-byte runs (ql low part, ql high part, qh), the
// half's 8 scale bytes and d.  The 16 weights of (task, j) share one scale,
// so they contribute (d*sc) * (sum q x - 32 sum x), with q's bytes built in a
// register (and, shift, or) and converted by v_cvt_f32_ubyte.  Each wave takes
// R rows (4, 2 or 1), which share the activation loads.  Measured on MI355X:
// 32000x4096 30.3 us (3.5 TB/s), 11008x4096 13.5 us, 4096x11008 14.9 us
// (2.5 TB/s); issuing the next task's loads ahead of the current task's
// arithmetic (software pipelining) measured slower at every R, and so did
// loading all 64 activations of a task with its weights (one round trip
// instead of four, but 159 registers at R = 4: 39 against 30 us at 32000 rows).

__device__ __forceinline__ float q6_ubyte_dot(uint32_t q, const float4 x)
{
    // (float)((q >> 8k) & 255) compiles to v_cvt_f32_ubyte<k>
    float a = (float)(q & 255u) * x.x;
    a = fmaf((float)((q >> 8) & 255u), x.y, a);
    a = fmaf((float)((q >> 16) & 255u), x.z, a);
    return fmaf((float)(q >> 24), x.w, a);
}

// The weights of the wave's R rows for one task, loaded before the activations.
struct Q6Task {
    uint32_t qa[4], qb[4], qh[4];  // ql[64h + 16s ..], ql[64h + 32 + 16s ..], qh[32h + 16s ..]
    uint32_t sc0, sc1;             // sc[8h .. 8h + 7]
    float d;
};

__device__ __forceinline__ void q6_load_task(const uint8_t *sb, int h, int sl, Q6Task &t)
{
    q6_run16(sb + 64 * h + 16 * sl, t.qa);
    q6_run16(sb + 64 * h + 32 + 16 * sl, t.qb);
    q6_run16(sb + 128 + 32 * h + 16 * sl, t.qh);
    // 8 scale bytes at a 2-byte-aligned offset: at most three dwords, the
    // last ending at the superblock's end
    const uintptr_t a = (uintptr_t)(sb + 192 + 8 * h);
    const uint32_t sh = (uint32_t)(a & 3u);
    const uint32_t *w = (const uint32_t *)(a - sh);
    const uint32_t w0 = w[0], w1 = w[1], w2 = sh ? w[2] : 0u;
    t.sc0 = __builtin_amdgcn_alignbyte(w1, w0, sh);
    t.sc1 = __builtin_amdgcn_alignbyte(w2, w1, sh);
    t.d = half_bits_to_float(*(const uint16_t *)(sb + 208));
}

template <int R>
__global__ __launch_bounds__(256) void gemv_q6_k2_k(float *dst, const uint8_t *M, const float *v, int out, int in)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = (blockIdx.x * 4 + wave) * R;
    if (r0 >= out) return;  // whole wave
    const int nrow = min(R, out - r0);
    const int nsb = in / 256, ntask = nsb * 4;
    const int64_t row_bytes = (int64_t)nsb * 210;
    float acc[R];
#pragma unroll
    for (int rr = 0; rr < R; rr++) acc[rr] = 0.f;
    const uint8_t *rowp[R];
#pragma unroll
    for (int rr = 0; rr < R; rr++) rowp[rr] = M + (int64_t)(r0 + min(rr, nrow - 1)) * row_bytes;  // rows past the end
                                                                                               // repeat the last
    for (int t = lane; t < ntask; t += 64) {
        const int b = t >> 2, h = (t >> 1) & 1, sl = t & 1;
        Q6Task w[R];
#pragma unroll
        for (int rr = 0; rr < R; rr++) q6_load_task(rowp[rr] + (int64_t)b * 210, h, sl, w[rr]);
        const float *xp = v + b * 256 + h * 128 + sl * 16;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float4 x[4];
#pragma unroll
            for (int c = 0; c < 4; c++) x[c] = *(const float4 *)(xp + 32 * j + 4 * c);
            const float sx = ((x[0].x + x[0].y) + (x[0].z + x[0].w)) + ((x[1].x + x[1].y) + (x[1].z + x[1].w)) +
                             ((x[2].x + x[2].y) + (x[2].z + x[2].w)) + ((x[3].x + x[3].y) + (x[3].z + x[3].w));
            const int shq = 4 * (j >> 1);
            // sc[8h + 16s/16 + 2j]: byte s + 2j of the half's 8
            const int k = sl + 2 * j;
#pragma unroll
            for (int rr = 0; rr < R; rr++) {
                const uint32_t *ql = (j & 1) ? w[rr].qb : w[rr].qa;
                float sq = 0.f;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const uint32_t nib = (ql[c] >> shq) & 0x0F0F0F0Fu;
                    const uint32_t hb = (w[rr].qh[c] >> (2 * j)) & 0x03030303u;
                    sq += q6_ubyte_dot(nib | (hb << 4), x[c]);
                }
                const uint32_t scw = k < 4 ? w[rr].sc0 : w[rr].sc1;
                const float sc = (float)(int8_t)(scw >> (8 * (k & 3)));
                acc[rr] = fmaf(w[rr].d * sc, sq - 32.0f * sx, acc[rr]);
            }
        }
    }
#pragma unroll
    for (int rr = 0; rr < R; rr++) {
        const float s = wave_reduce_sum(acc[rr]);
        if (lane == 0 && rr < nrow) dst[r0 + rr] = s;
    }
}

// Rows per wave: the most (of 4, 2, 1) that still give two workgroups per CU
// (MI355X: 4 rows at 32000 and 11008 rows, 2 at 4096).  HOLO_Q6K_ROWS=1|2|4
// forces a value.
static int q6_rows_per_wave(int out_dim)
{
    static const int forced = [] {
        const char *e = getenv("HOLO_Q6K_ROWS");
        const int v = e ? atoi(e) : 0;
        return (v == 1 || v == 2 || v == 4) ? v : 0;
    }();
    if (forced) return forced;
    for (int r = 4; r > 1; r /= 2)
        if ((out_dim + 4 * r - 1) / (4 * r) >= 2 * num_cus()) return r;
    return 1;
}


// ---- decode attention: one query row per head, keys split over workgroups ----------
//
// softmax((q . k_p) / sqrt(hd)) . v over cached positions p < kv_len, as
// cuda_multi_head_attention computes it (cuda_ops.cu:1813-1952), for heads of
// up to 128 dims (a multiple of 4).  The keys are cut into `splits` ranges of
// `chunk` positions, one workgroup per (range, head), so that a decode step
// reads the whole cache with the whole chip rather than one workgroup per head.
// A workgroup takes its range 64 positions at a time: thread (c, g) owns
// 16-byte column c of the head (32 columns) for keys g, g + 8, ..., g + 56, so
// all 8 key and 8 value loads of a thread are issued together and each wave
// instruction reads two whole 512-byte cache rows.  Scores are summed over the
// 32 column lanes, the softmax runs online over the 64-key passes (running
// max and sum), and the 8 key groups' partial outputs are summed in a fixed
// order.  With one range the workgroup writes the output; otherwise it writes
// (unnormalised output, max, sum) and attn_decode_combine_k merges the ranges
// of a head in range order, so the result does not depend on timing.
constexpr int kDecKeys = 64;
constexpr int kDecMaxSplits = 256;  // at most one range per thread of attn_decode_combine_k's 512
constexpr size_t kDecPartFloats = (size_t)4 << 20;  // 16 MiB of range partials, allocated by cuda_init
static float *g_dec_part = nullptr;

__device__ __forceinline__ float half_wave_sum(float v)
{
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) v += __shfl_xor(v, off, 32);
    return v;
}

__global__ __launch_bounds__(256) void attn_decode_k(float *out, float *part, const float *q, const float *kc,
                                                     const float *vc, int kv_len, int hd, int n_heads, int n_kv_heads,
                                                     int chunk)
{
    __shared__ float4 lq[32];
    __shared__ float lsc[kDecKeys];
    __shared__ float4 lo[8][32];
    const int h = blockIdx.y, s = blockIdx.x, splits = gridDim.x;
    const int kvh = h / (n_heads / n_kv_heads);
    const int64_t kv_dim = (int64_t)n_kv_heads * hd;
    const int t = threadIdx.x, lane = t & 63, c = t & 31, g = t >> 5;
    const int hd4 = hd >> 2;
    const bool col = c < hd4;
    const float scale = 1.0f / sqrtf((float)hd);
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < hd4) lq[t] = *(const float4 *)(q + (int64_t)h * hd + 4 * t);
    __syncthreads();
    const float4 q4 = col ? lq[c] : zero;
    const float *kb = kc + (int64_t)kvh * hd + 4 * c;
    const float *vb = vc + (int64_t)kvh * hd + 4 * c;
    const int p_begin = s * chunk, p_end = min(p_begin + chunk, kv_len);
    float m = -INFINITY, l = 0.f;
    float4 o4 = zero;
    for (int p0 = p_begin; p0 < p_end; p0 += kDecKeys) {
        float4 k4[8], v4[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int p = p0 + g + 8 * j;
            k4[j] = zero;
            v4[j] = zero;
            if (col && p < p_end) {
                k4[j] = *(const float4 *)(kb + (int64_t)p * kv_dim);
                v4[j] = *(const float4 *)(vb + (int64_t)p * kv_dim);
            }
        }
        float sj[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            sj[j] = half_wave_sum(q4.x * k4[j].x + q4.y * k4[j].y + q4.z * k4[j].z + q4.w * k4[j].w);
        if (c == 0) {
#pragma unroll
            for (int j = 0; j < 8; j++) lsc[g + 8 * j] = p0 + g + 8 * j < p_end ? sj[j] * scale : -INFINITY;
        }
        __syncthreads();
        // every wave reduces the same 64 scores in the same order, so m and l
        // agree across the workgroup; key p0 + i's weight sits in lane i
        const float sl = lsc[lane];
        const float mnew = fmaxf(m, wave_reduce_max(sl));  // p0 < p_end: finite from the first pass on
        const float corr = expf(m - mnew);
        const float pl = expf(sl - mnew);
        l = l * corr + wave_reduce_sum(pl);
        o4 = make_float4(o4.x * corr, o4.y * corr, o4.z * corr, o4.w * corr);
        m = mnew;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float w = __shfl(pl, g + 8 * j, 64);
            o4 = make_float4(fmaf(w, v4[j].x, o4.x), fmaf(w, v4[j].y, o4.y), fmaf(w, v4[j].z, o4.z),
                             fmaf(w, v4[j].w, o4.w));
        }
        __syncthreads();  // lsc is rewritten by the next pass
    }
    lo[g][c] = o4;
    __syncthreads();
    if (t < hd4) {
        float4 r = lo[0][t];
#pragma unroll
        for (int gg = 1; gg < 8; gg++)
            r = make_float4(r.x + lo[gg][t].x, r.y + lo[gg][t].y, r.z + lo[gg][t].z, r.w + lo[gg][t].w);
        if (splits == 1) {
            const float inv = 1.0f / l;
            *(float4 *)(out + (int64_t)h * hd + 4 * t) = make_float4(r.x * inv, r.y * inv, r.z * inv, r.w * inv);
        } else {
            float *pp = part + ((int64_t)h * splits + s) * (hd + 4);
            *(float4 *)(pp + 4 * t) = r;
            if (t == 0) {
                pp[hd] = m;
                pp[hd + 1] = l;
            }
        }
    }
}

// Merges a head's ranges with weights e^(m_s - M).  512 threads: thread
// (d, g) sums ranges g, g + 4, ... for output dim d, and the 4 groups' sums
// meet in LDS in group order, so the order is fixed.  (Merging in the split
// kernel itself, by the last range of a head to arrive, measured slower: the
// merge becomes a serial tail and every range pays the arrival.)
static_assert(kDecMaxSplits <= 512, "attn_decode_combine_k: one range per thread");
__global__ __launch_bounds__(512) void attn_decode_combine_k(float *out, const float *part, int hd, int splits)
{
    __shared__ float lw[kDecMaxSplits];
    __shared__ float lg[4][128];
    __shared__ float scratch[16];
    const int h = blockIdx.x, t = threadIdx.x, d = t & 127, grp = t >> 7;
    const int stride = hd + 4;
    const float *ph = part + (int64_t)h * splits * stride;
    // one round of loads: the partial outputs of ranges grp, grp + 4, ... (the
    // first kPre of them into registers) together with range t's max and sum,
    // so the reductions below wait for a single round trip
    constexpr int kPre = 16;
    float po[kPre];
#pragma unroll
    for (int i = 0; i < kPre; i++) {
        const int s = grp + 4 * i;
        po[i] = d < hd && s < splits ? ph[(int64_t)s * stride + d] : 0.f;
    }
    const bool mine = t < splits;  // splits <= kDecMaxSplits <= blockDim.x: one range per thread at most
    const float ms = mine ? ph[(int64_t)t * stride + hd] : -INFINITY;
    const float ls = mine ? ph[(int64_t)t * stride + hd + 1] : 0.f;
    const float M = block_reduce<true>(ms, scratch);
    const float w = mine ? expf(ms - M) : 0.f;
    if (mine) lw[t] = w;
    const float L = block_reduce<false>(w * ls, scratch);  // its barriers also publish lw
    if (d < hd) {
        float o = 0.f;
#pragma unroll
        for (int i = 0; i < kPre; i++)
            if (grp + 4 * i < splits) o = fmaf(lw[grp + 4 * i], po[i], o);
        for (int s = grp + 4 * kPre; s < splits; s += 4) o = fmaf(lw[s], ph[(int64_t)s * stride + d], o);
        lg[grp][d] = o;
    }
    __syncthreads();
    if (grp == 0 && d < hd) out[(int64_t)h * hd + d] = (((lg[0][d] + lg[1][d]) + lg[2][d]) + lg[3][d]) * (1.0f / L);
}

// Short caches in one launch: one workgroup per head, SUB groups of 256
// threads, group sg taking positions [sg chunk, (sg + 1) chunk) with
// attn_decode_k's pass (the same loads, scores, online softmax and key-group
// order), every group looping the same number of passes so the barriers are
// the workgroup's.  A group whose range is empty keeps (m, l, o) = (-inf, 0,
// 0) and gets weight 0; the groups merge in group order through LDS, so the
// result does not depend on timing.  No range partials and no second launch.
template <int SUB>
__global__ __launch_bounds__(256 * SUB) void attn_decode_wg_k(float *out, const float *q, const float *kc,
                                                              const float *vc, int kv_len, int hd, int n_heads,
                                                              int n_kv_heads, int chunk)
{
    __shared__ float4 lq[32];
    __shared__ float lsc[SUB][kDecKeys];
    __shared__ float4 lo[SUB][8][32];
    __shared__ float lm[SUB], ll[SUB];
    const int h = blockIdx.x;
    const int kvh = h / (n_heads / n_kv_heads);
    const int64_t kv_dim = (int64_t)n_kv_heads * hd;
    const int t = threadIdx.x, sg = __builtin_amdgcn_readfirstlane(t >> 8), u = t & 255;
    const int lane = u & 63, c = u & 31, g = u >> 5;
    const int hd4 = hd >> 2;
    const bool col = c < hd4;
    const float scale = 1.0f / sqrtf((float)hd);
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t < hd4) lq[t] = *(const float4 *)(q + (int64_t)h * hd + 4 * t);
    __syncthreads();
    const float4 q4 = col ? lq[c] : zero;
    const float *kb = kc + (int64_t)kvh * hd + 4 * c;
    const float *vb = vc + (int64_t)kvh * hd + 4 * c;
    const int p_begin = sg * chunk, p_end = min(p_begin + chunk, kv_len);
    float m = -INFINITY, l = 0.f;
    float4 o4 = zero;
    for (int i0 = 0; i0 < chunk; i0 += kDecKeys) {
        const int p0 = p_begin + i0;
        float4 k4[8], v4[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int p = p0 + g + 8 * j;
            k4[j] = zero;
            v4[j] = zero;
            if (col && p < p_end) {
                k4[j] = *(const float4 *)(kb + (int64_t)p * kv_dim);
                v4[j] = *(const float4 *)(vb + (int64_t)p * kv_dim);
            }
        }
        float sj[8];
#pragma unroll
        for (int j = 0; j < 8; j++)
            sj[j] = half_wave_sum(q4.x * k4[j].x + q4.y * k4[j].y + q4.z * k4[j].z + q4.w * k4[j].w);
        if (c == 0) {
#pragma unroll
            for (int j = 0; j < 8; j++) lsc[sg][g + 8 * j] = p0 + g + 8 * j < p_end ? sj[j] * scale : -INFINITY;
        }
        __syncthreads();
        if (p0 < p_end) {  // uniform per group: a pass with keys in this group's range
            const float sl = lsc[sg][lane];
            const float mnew = fmaxf(m, wave_reduce_max(sl));  // finite: the pass has a key
            const float corr = expf(m - mnew);
            const float pl = expf(sl - mnew);
            l = l * corr + wave_reduce_sum(pl);
            o4 = make_float4(o4.x * corr, o4.y * corr, o4.z * corr, o4.w * corr);
            m = mnew;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float w = __shfl(pl, g + 8 * j, 64);
                o4 = make_float4(fmaf(w, v4[j].x, o4.x), fmaf(w, v4[j].y, o4.y), fmaf(w, v4[j].z, o4.z),
                                 fmaf(w, v4[j].w, o4.w));
            }
        }
        __syncthreads();  // lsc is rewritten by the next pass
    }
    lo[sg][g][c] = o4;
    if (u == 0) {
        lm[sg] = m;
        ll[sg] = l;
    }
    __syncthreads();
    if (t < hd4) {
        float M = lm[0];
#pragma unroll
        for (int k = 1; k < SUB; k++) M = fmaxf(M, lm[k]);  // group 0 always has keys: finite
        float L = 0.f;
        float4 r = zero;
#pragma unroll
        for (int k = 0; k < SUB; k++) {
            const float w = lm[k] == -INFINITY ? 0.f : expf(lm[k] - M);
            float4 rk = lo[k][0][t];
#pragma unroll
            for (int gg = 1; gg < 8; gg++)
                rk = make_float4(rk.x + lo[k][gg][t].x, rk.y + lo[k][gg][t].y, rk.z + lo[k][gg][t].z,
                                 rk.w + lo[k][gg][t].w);
            r = make_float4(fmaf(w, rk.x, r.x), fmaf(w, rk.y, r.y), fmaf(w, rk.z, r.z), fmaf(w, rk.w, r.w));
            L = fmaf(w, ll[k], L);
        }
        const float inv = 1.0f / L;
        *(float4 *)(out + (int64_t)h * hd + 4 * t) = make_float4(r.x * inv, r.y * inv, r.z * inv, r.w * inv);
    }
}
// Up to this many positions (one 64-position pass per group) attn_decode_wg_k:
// 6.6 against 8.0 us at 128 positions, 32 heads of 128.  With two or more
// passes its 32 workgroups wait on each pass in turn, and the split kernel's
// whole-chip read wins (300 / 512 / 1024 positions: 9.8 / 10.8 / 19.4 against
// 8.3 / 8.5 / 10.1 us).
constexpr int kDecWgMaxKeys = 4 * kDecKeys;

// Shapes the split kernel takes: head_dim a multiple of 4 up to 128, 16-byte
// aligned rows.
static bool decode_attention_fits(const float *q, const float *kc, const float *vc, int hd)
{
    return hd >= 4 && hd <= 128 && hd % 4 == 0 && !(((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc) & 15);
}

static void decode_attention(float *dst, const float *q, const float *kc, const float *vc, int kv_len, int hd,
                             int n_heads, int n_kv_heads)
{
    if (kv_len > kDecKeys && kv_len <= kDecWgMaxKeys) {
        // four groups of whole 64-position passes per head
        const int chunk = ((kv_len + 3) / 4 + kDecKeys - 1) / kDecKeys * kDecKeys;
        hipLaunchKernelGGL(attn_decode_wg_k<4>, dim3(n_heads), dim3(1024), 0, stream(), dst, q, kc, vc, kv_len, hd,
                           n_heads, n_kv_heads, chunk);
        HOLO_LAUNCH_CHECK();
        return;
    }
    int splits = (kv_len + kDecKeys - 1) / kDecKeys;
    if (!g_dec_part) splits = 1;
    splits = min(splits, min(kDecMaxSplits, (int)(kDecPartFloats / ((size_t)n_heads * (hd + 4)))));
    splits = max(splits, 1);
    const int chunk = ((kv_len + splits - 1) / splits + kDecKeys - 1) / kDecKeys * kDecKeys;
    splits = (kv_len + chunk - 1) / chunk;  // every range holds at least one key
    hipLaunchKernelGGL(attn_decode_k, dim3(splits, n_heads), dim3(256), 0, stream(), dst, g_dec_part, q, kc, vc,
                       kv_len, hd, n_heads, n_kv_heads, chunk);
    HOLO_LAUNCH_CHECK();
    if (splits > 1) {
        hipLaunchKernelGGL(attn_decode_combine_k, dim3(n_heads), dim3(512), 0, stream(), dst, g_dec_part, hd,
                           splits);
        HOLO_LAUNCH_CHECK();
    }
}

bool attention_scratch_init()
{
    if (g_dec_part) return true;
    if (hipMalloc((void **)&g_dec_part, kDecPartFloats * sizeof(float)) != hipSuccess) {
        g_dec_part = nullptr;
        return false;
    }
    return true;
}

void attention_scratch_release()
{
    if (g_dec_part) (void)hipFree(g_dec_part);
    g_dec_part = nullptr;
}

// ---- RoPE (cuda_ops.cu:2102-2140): pairs (i, i + hd/2), theta = pos / base^(2i/hd) ----------

__device__ __forceinline__ void rope_head(float *q, float *k, int pos, int hd, int n_heads, int n_kv_heads,
                                          float base, int h, int i)
{
    const int half = hd / 2;
    if (i >= half) return;
    const float freq = 1.0f / powf(base, (float)(2 * i) / (float)hd);
    const float th = (float)pos * freq;
    const float c = cosf(th), s = sinf(th);
    if (h < n_heads) {
        float *p = q + (int64_t)h * hd;
        float a = p[i], b = p[i + half];
        p[i] = a * c - b * s;
        p[i + half] = a * s + b * c;
    }
    if (h < n_kv_heads) {
        float *p = k + (int64_t)h * hd;
        float a = p[i], b = p[i + half];
        p[i] = a * c - b * s;
        p[i + half] = a * s + b * c;
    }
}

__global__ void rope_k(float *q, float *k, int pos, int hd, int n_heads, int n_kv_heads, float base)
{
    rope_head(q, k, pos, hd, n_heads, n_kv_heads, base, blockIdx.x, threadIdx.x);
}

// Row r = blockIdx.x of q [rows][n_heads*hd] and k [rows][n_kv_heads*hd] at
// position pos0 + r.  The row's heads, q's then k's, go out in chunks of 4G
// (blockIdx.y) to G groups of hd/2 threads: thread t takes pair index
// i = t mod hd/2 of four heads, loads all four pairs before it stores any,
// and computes the angle of (position, i) once for them.  Same expressions as
// rope_head: the same bits.
__global__ __launch_bounds__(1024) void rope_rows_k(float *__restrict__ q, float *__restrict__ k, int pos0, int hd,
                                                    int n_heads, int n_kv_heads, float base)
{
    const int64_t r = blockIdx.x;
    const int half = hd / 2, G = blockDim.x / half;
    const int i = threadIdx.x % half, g = threadIdx.x / half;
    if (g >= G) return;
    const float freq = 1.0f / powf(base, (float)(2 * i) / (float)hd);
    const float th = (float)(pos0 + (int)r) * freq;
    const float c = cosf(th), s = sinf(th);
    float *qr = q + r * n_heads * hd, *kr = k + r * n_kv_heads * hd;
    const int h0 = (int)blockIdx.y * 4 * G + g;
    float *p[4];
    float a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int h = h0 + u * G;
        p[u] = h < n_heads ? qr + (int64_t)h * hd
               : h < n_heads + n_kv_heads ? kr + (int64_t)(h - n_heads) * hd : nullptr;
        if (p[u]) {
            a[u] = p[u][i];
            b[u] = p[u][i + half];
        }
    }
#pragma unroll
    for (int u = 0; u < 4; u++)
        if (p[u]) {
            p[u][i] = a[u] * c - b[u] * s;
            p[u][i + half] = a[u] * s + b[u] * c;
        }
}

// ---- embedding lookups (cuda_ops.cu:2147-2300) ---------------------------------------------

__global__ void emb_f32_k(float *dst, const float *e, int token, int dim)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < dim) dst[i] = e[(int64_t)token * dim + i];
}
__global__ void emb_f16_k(float *dst, const uint16_t *e, int token, int dim)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < dim) dst[i] = half_bits_to_float_exact(e[(int64_t)token * dim + i]);
}
// One thread per value; byte loads (a token row need not be 4-byte aligned).
__global__ void emb_q8_0_k(float *dst, const uint8_t *e, int token, int dim)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    const uint8_t *b = e + ((int64_t)token * (dim / 32) + i / 32) * 34;
    float d = half_bits_to_float_exact((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    dst[i] = d * (float)(int8_t)b[2 + i % 32];
}
__global__ void emb_q4_0_k(float *dst, const uint8_t *e, int token, int dim)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    const uint8_t *b = e + ((int64_t)token * (dim / 32) + i / 32) * 18;
    float d = half_bits_to_float_exact((uint32_t)b[0] | ((uint32_t)b[1] << 8));
    int j = i % 32;
    uint8_t q = b[2 + (j & 15)];
    int nib = j < 16 ? (q & 15) : (q >> 4);
    dst[i] = d * (float)(nib - 8);
}
// Q6_K value at position j of a 256-value superblock (quant.c:252-268).
__device__ __forceinline__ float q6_k_value(const uint8_t *sb, int j)
{
    const int half = j >> 7, p = j & 127, l = p & 31, quad = p >> 5;
    const uint8_t *ql = sb + 64 * half;
    const uint8_t *qh = sb + 128 + 32 * half;
    const int8_t *sc = (const int8_t *)(sb + 192) + 8 * half;
    const float d = half_bits_to_float_exact((uint32_t)sb[208] | ((uint32_t)sb[209] << 8));
    const int lo = (quad & 1) ? ql[l + 32] : ql[l];
    const int nib = (quad < 2) ? (lo & 0xF) : (lo >> 4);
    const int q = (nib | (((qh[l] >> (2 * quad)) & 3) << 4)) - 32;
    return (d * (float)sc[l / 16 + 2 * quad]) * (float)q;
}
__global__ void emb_q6_k_k(float *dst, const uint8_t *e, int token, int dim)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    const uint8_t *sb = e + ((int64_t)token * (dim / 256) + i / 256) * 210;
    dst[i] = q6_k_value(sb, i % 256);
}

// ---- argmax (cuda_ops.cu:2314-2413): first index of the maximum ---------------------------

__global__ __launch_bounds__(1024) void argmax_k(const float *x, int n, int *out)
{
    __shared__ float sv[1024];
    __shared__ int si[1024];
    float best = -INFINITY;
    int bi = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = x[i];
        if (v > best) {
            best = v;
            bi = i;
        }
    }
    sv[threadIdx.x] = best;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = blockDim.x / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) {
            float v = sv[threadIdx.x + s];
            int j = si[threadIdx.x + s];
            if (v > sv[threadIdx.x] || (v == sv[threadIdx.x] && j < si[threadIdx.x])) {
                sv[threadIdx.x] = v;
                si[threadIdx.x] = j;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[0] = si[0] == 0x7FFFFFFF ? 0 : si[0];
}

// ---- F32 / F16 / Q6_K GEMVs (cuda_ops.cu:511-615, 740-845) ------------------------------------
// One wave per row, 4 rows per workgroup, activations from global memory.

__global__ __launch_bounds__(256) void gemv_f32_k(float *dst, const float *M, const float *v, int out, int in)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= out) return;
    const float *r = M + (int64_t)row * in;
    float s = 0.f;
    for (int j = lane; j < in; j += 64) s += r[j] * v[j];
    s = wave_reduce_sum(s);
    if (lane == 0) dst[row] = s;
}

__global__ __launch_bounds__(256) void gemv_f16_k(float *dst, const uint16_t *M, const float *v, int out, int in)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= out) return;
    const uint16_t *r = M + (int64_t)row * in;
    float s = 0.f;
    for (int j = lane; j < in; j += 64) s += half_bits_to_float(r[j]) * v[j];
    s = wave_reduce_sum(s);
    if (lane == 0) dst[row] = s;
}

// lane = 32*half + l computes the 4 values l, l+32, l+64, l+96 of its half.
__global__ __launch_bounds__(256) void gemv_q6_k_k(float *dst, const uint8_t *M, const float *v, int out, int in)
{
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= out) return;
    const int nsb = in / 256;
    const int half = lane >> 5, l = lane & 31;
    float s = 0.f;
    for (int b = 0; b < nsb; b++) {
        const uint8_t *sb = M + ((int64_t)row * nsb + b) * 210;
        const float *x = v + b * 256 + half * 128;
#pragma unroll
        for (int qd = 0; qd < 4; qd++) s += q6_k_value(sb, half * 128 + qd * 32 + l) * x[qd * 32 + l];
    }
    s = wave_reduce_sum(s);
    if (lane == 0) dst[row] = s;
}

// Device scalars for the two ops that return a value to the host.
static float *g_dot = nullptr;
static int *g_argmax = nullptr;

// ---- row-batched ops of the prefill forward (M activation rows) --------------------------

// RMS norm of each row (the arithmetic of rms_norm_k), one workgroup per row.
__global__ __launch_bounds__(256) void rms_norm_rows_k(float *dst, const float *x, const float *w, int n, float eps)
{
    __shared__ float scratch[16];
    const int64_t off = (int64_t)blockIdx.x * n;
    x += off;
    dst += off;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_reduce<false>(ss, scratch);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = x[i] * scale * (w ? w[i] : 1.0f);
}

// The same with 16-byte loads and the row held in registers between the sum
// of squares and the scaling (rows of up to 1024*NV floats, n % 4 == 0,
// 16-byte-aligned pointers): one read of x instead of two, and no scalar
// load chain.
template <int NV>
__global__ __launch_bounds__(256) void rms_norm_rows4_k(float *dst, const float *x, const float *w, int n, float eps)
{
    __shared__ float scratch[16];
    const int n4 = n >> 2;
    const float4 *x4 = (const float4 *)(x + (int64_t)blockIdx.x * n);
    float4 *d4 = (float4 *)(dst + (int64_t)blockIdx.x * n);
    float4 v[NV], wv[NV];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + 256 * j;
        v[j] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        // the weights load with the row, not after the reduction
        wv[j] = w && i < n4 ? ((const float4 *)w)[i] : make_float4(1.f, 1.f, 1.f, 1.f);
        ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    }
    ss = block_reduce<false>(ss, scratch);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + 256 * j;
        if (i < n4) {
            const float4 w4 = wv[j];
            d4[i] = make_float4(v[j].x * scale * w4.x, v[j].y * scale * w4.y, v[j].z * scale * w4.z,
                                v[j].w * scale * w4.w);
        }
    }
}

// Embedding rows: row r is token tokens[r] of the table, exact dequantisation
// (the per-token lookups above, get_embedding of llm.c:941-1008).
// Weight p (0..31) of a Q4_K unit: (d*sc)*q - dmin*m with both roundings, as
// dequantize_row_q4_k computes it (quant.c:277-311, no contraction).
__device__ __forceinline__ float q4_k_weight(const Q4_KUnit &u, int p)
{
#pragma clang fp contract(off)
    const uint32_t b = (u.q[(p & 15) >> 2] >> (8 * (p & 3))) & 0xFFu;
    const float pv = u.dsc * (float)(p < 16 ? (b & 15u) : (b >> 4));
    return pv - u.dmn;
}

__global__ void emb_rows_k(float *dst, const uint8_t *e, const int *tokens, int dim, int type)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dim) return;
    const int64_t r = blockIdx.y, t = tokens[r];
    float v;
    switch (type) {
    case HOLO_TYPE_F16: v = half_bits_to_float_exact(((const uint16_t *)e)[t * dim + i]); break;
    case HOLO_TYPE_Q8_0: {
        const uint8_t *b = e + (t * (dim / 32) + i / 32) * 34;
        v = half_bits_to_float_exact((uint32_t)b[0] | ((uint32_t)b[1] << 8)) * (float)(int8_t)b[2 + i % 32];
        break;
    }
    case HOLO_TYPE_Q4_0: {
        const uint8_t *b = e + (t * (dim / 32) + i / 32) * 18;
        const int j = i % 32;
        const uint8_t q = b[2 + (j & 15)];
        v = half_bits_to_float_exact((uint32_t)b[0] | ((uint32_t)b[1] << 8)) *
            (float)((j < 16 ? (q & 15) : (q >> 4)) - 8);
        break;
    }
    case HOLO_TYPE_Q6_K: v = q6_k_value(e + (t * (dim / 256) + i / 256) * 210, i % 256); break;
    case HOLO_TYPE_Q4_K: v = q4_k_weight(load_q4_k(e, t * (dim / 32) + i / 32), i % 32); break;
    default: v = ((const float *)e)[t * dim + i]; break;
    }
    dst[r * dim + i] = v;
}

// Causal attention over the prompt.  Query row m (position pos0 + m) of head
// h attends to cached positions 0 .. pos0 + m of KV head h / (n_heads /
// n_kv_heads): softmax((q . k_p) / sqrt(hd)) . v, as cuda_multi_head_attention
// computes it for one query (cuda_ops.cu:1813-1952), with the softmax taken
// online over key tiles (running max and sum, fp32).
// Workgroup: head h, 32 query rows (8 per wave).  Keys and values are staged
// 64 positions at a time in LDS (key rows padded to 132 floats, so the 16-byte
// reads of 16 lanes fall on distinct banks); the next tile's loads are in
// flight in registers (16-byte loads) while the current tile is used.  Lane l
// scores key l of the tile against the wave's 8 queries, reading each 16-byte
// piece of its key once for all 8; the probabilities are then broadcast from
// the lane that holds them (readlane) while lane l accumulates output
// dimensions l and l + 64.
constexpr int kAttQ = 32, kAttKeys = 64, kAttMaxHd = 128, kAttKStride = kAttMaxHd + 4;
constexpr int kAttPieces = kAttKeys * kAttMaxHd / 4 / 256;  // float4 pieces per thread and tile (8)
constexpr size_t kAttLds = (size_t)(kAttQ * kAttMaxHd + kAttKeys * kAttKStride + kAttKeys * kAttMaxHd) * sizeof(float);

__global__ __launch_bounds__(256) void attention_prefill_k(float *out, const float *q, const float *kc,
                                                           const float *vc, int rows, int pos0, int hd, int n_heads,
                                                           int n_kv_heads)
{
    extern __shared__ float att_lds[];
    float *lq = att_lds;                         // [kAttQ][kAttMaxHd]
    float *lk = lq + kAttQ * kAttMaxHd;          // [kAttKeys][kAttKStride]
    float *lv = lk + kAttKeys * kAttKStride;     // [kAttKeys][kAttMaxHd]
    // the causal tiles furthest down the prompt carry the most keys: start them first
    const int h = blockIdx.y, m0 = (gridDim.x - 1 - blockIdx.x) * kAttQ;
    const int kvh = h / (n_heads / n_kv_heads);
    const int64_t q_dim = (int64_t)n_heads * hd, kv_dim = (int64_t)n_kv_heads * hd;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float scale = 1.0f / sqrtf((float)hd);
    const int m_end = min(m0 + kAttQ, rows);
    const int last_key = pos0 + m_end - 1;  // the furthest position any query here attends to
    const int hd4 = hd >> 2;                 // hd is a multiple of 4 (checked by the caller)

    for (int i = tid; i < kAttQ * hd4; i += blockDim.x) {
        const int r = i / hd4, c = i - r * hd4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m0 + r < rows) v = *(const float4 *)(q + (int64_t)(m0 + r) * q_dim + (int64_t)h * hd + 4 * c);
        *(float4 *)(lq + r * kAttMaxHd + 4 * c) = v;
    }
    // the tile at key p0 into registers: piece f = tid + 256 i is key f / hd4,
    // columns 4 (f % hd4) .. +3; pieces past the tile or the last key load zeros
    float4 rk[kAttPieces], rv[kAttPieces];
    auto fetch = [&](int p0) {
#pragma unroll
        for (int i = 0; i < kAttPieces; i++) {
            const int f = tid + 256 * i, r = f / hd4, c = f - r * hd4;
            rk[i] = rv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r < kAttKeys && p0 + r <= last_key) {
                const int64_t o = (int64_t)(p0 + r) * kv_dim + (int64_t)kvh * hd + 4 * c;
                rk[i] = *(const float4 *)(kc + o);
                rv[i] = *(const float4 *)(vc + o);
            }
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < kAttPieces; i++) {
            const int f = tid + 256 * i, r = f / hd4, c = f - r * hd4;
            if (r < kAttKeys) {
                *(float4 *)(lk + r * kAttKStride + 4 * c) = rk[i];
                *(float4 *)(lv + r * kAttMaxHd + 4 * c) = rv[i];
            }
        }
    };

    float mx[8], sm[8], o0[8], o1[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        mx[j] = -INFINITY;
        sm[j] = 0.f;
        o0[j] = 0.f;
        o1[j] = 0.f;
    }
    const int r0 = wave * 8;                               // this wave's first query row in the tile
    const int nq = max(0, min(8, m_end - (m0 + r0)));      // its valid queries (wave-uniform)
    fetch(0);
    for (int p0 = 0; p0 <= last_key; p0 += kAttKeys) {
        __syncthreads();  // the previous tile is consumed (and lq is written, first time)
        stash();
        __syncthreads();
        if (p0 + kAttKeys <= last_key) fetch(p0 + kAttKeys);
        if (nq == 0) continue;
        // scores of key p0 + lane against the wave's queries
        float sc[8];
#pragma unroll
        for (int j = 0; j < 8; j++) sc[j] = 0.f;
        const float *kr = lk + lane * kAttKStride;
#pragma unroll 2
        for (int c = 0; c < hd4; c++) {
            const float4 k4 = *(const float4 *)(kr + 4 * c);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 q4 = *(const float4 *)(lq + (r0 + j) * kAttMaxHd + 4 * c);
                sc[j] += q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
            }
        }
        // All 8 queries are scored, also rows past the prompt (their q rows are
        // zero, their outputs are not written), so the 8 reductions are
        // independent and interleave.  Sums stay per lane until the end.
        const int p = p0 + lane;
        float pr[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int qpos = pos0 + m0 + r0 + j;
            const float s = p <= qpos ? sc[j] * scale : -INFINITY;
            // key 0 <= qpos is in the first tile, so the running max is finite from then on
            const float mnew = fmaxf(mx[j], wave_reduce_max(s));
            pr[j] = p <= qpos ? expf(s - mnew) : 0.f;
            const float corr = expf(mx[j] - mnew);
            sm[j] = sm[j] * corr + pr[j];
            o0[j] *= corr;
            o1[j] *= corr;
            mx[j] = mnew;
        }
        // out += sum_p pr[p] v_p: the weight of key pp comes from lane pp
        const int hi = (lane + 64) & (kAttMaxHd - 1);
        const int kmax = min(kAttKeys, last_key - p0 + 1);  // keys past last_key have weight 0 everywhere
        for (int pp = 0; pp < kmax; pp++) {
            const float va = lv[pp * kAttMaxHd + lane], vb = lv[pp * kAttMaxHd + hi];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float w = __builtin_amdgcn_readlane(__float_as_int(pr[j]), pp) ;
                o0[j] += __int_as_float(w) * va;
                o1[j] += __int_as_float(w) * vb;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) sm[j] = wave_reduce_sum(sm[j]);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int m = m0 + r0 + j;
        if (j >= nq) continue;
        const float inv = 1.0f / sm[j];
        float *o = out + (int64_t)m * q_dim + (int64_t)h * hd;
        if (lane < hd) o[lane] = o0[j] * inv;
        if (lane + 64 < hd) o[lane + 64] = o1[j] * inv;
    }
}

}  // namespace holo

using namespace holo;

extern "C" {

void cuda_vec_add(float *dst, const float *a, const float *b, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(vec_add_k, dim3(blocks_for(n)), dim3(kBlock), 0, stream(), dst, a, b, n);
    HOLO_LAUNCH_CHECK();
}

void cuda_vec_mul(float *dst, const float *a, const float *b, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(vec_mul_k, dim3(blocks_for(n)), dim3(kBlock), 0, stream(), dst, a, b, n);
    HOLO_LAUNCH_CHECK();
}

void cuda_vec_scale(float *dst, const float *a, float scale, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(vec_scale_k, dim3(blocks_for(n)), dim3(kBlock), 0, stream(), dst, a, scale, n);
    HOLO_LAUNCH_CHECK();
}

float cuda_vec_dot(const float *a, const float *b, int n)
{
    if (n <= 0) return 0.0f;
    if (!g_dot) HOLO_CHECK(hipMalloc(&g_dot, sizeof(float)));
    if (!g_dot) return 0.0f;
    hipLaunchKernelGGL(vec_dot_k, dim3(1), dim3(1024), 0, stream(), a, b, n, g_dot);
    HOLO_LAUNCH_CHECK();
    float r = 0.f;
    HOLO_CHECK(hipMemcpyAsync(&r, g_dot, sizeof(float), hipMemcpyDeviceToHost, stream()));
    HOLO_CHECK(hipStreamSynchronize(stream()));
    return r;
}

void cuda_silu(float *x, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(silu_k, dim3(blocks_for(n)), dim3(kBlock), 0, stream(), x, n);
    HOLO_LAUNCH_CHECK();
}

void cuda_silu_mul(float *dst, const float *a, const float *b, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(silu_mul_k, dim3(blocks_for(n)), dim3(kBlock), 0, stream(), dst, a, b, n);
    HOLO_LAUNCH_CHECK();
}

void cuda_gelu(float *x, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(gelu_k, dim3(blocks_for(n)), dim3(kBlock), 0, stream(), x, n);
    HOLO_LAUNCH_CHECK();
}

void cuda_relu(float *x, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(relu_k, dim3(blocks_for(n)), dim3(kBlock), 0, stream(), x, n);
    HOLO_LAUNCH_CHECK();
}

void cuda_rms_norm(float *dst, const float *x, const float *weight, int n, float eps)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(rms_norm_k, dim3(1), dim3(1024), 0, stream(), dst, x, weight, n, eps);
    HOLO_LAUNCH_CHECK();
}

// The reference's layer norm is its RMS norm (cuda_ops.cu:1506-1511, a TODO
// there); kept as is so results match the caller's expectations.
void cuda_layer_norm(float *dst, const float *x, const float *weight, const float *bias, int n, float eps)
{
    (void)bias;
    cuda_rms_norm(dst, x, weight, n, eps);
}

void cuda_softmax(float *dst, const float *x, int n)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(softmax_k, dim3(1), dim3(1024), 0, stream(), dst, x, n);
    HOLO_LAUNCH_CHECK();
}

void cuda_softmax_inplace(float *x, int n) { cuda_softmax(x, x, n); }

void cuda_attention_scores(float *dst, const float *Q, const float *K, int seq_len, int kv_len, int head_dim,
                           float scale)
{
    if (seq_len <= 0 || kv_len <= 0) return;
    hipLaunchKernelGGL(attention_scores_k, dim3(blocks_for(kv_len), seq_len), dim3(kBlock), 0, stream(), dst, Q, K,
                       seq_len, kv_len, head_dim, scale);
    HOLO_LAUNCH_CHECK();
}

void cuda_attention_apply(float *dst, const float *scores, const float *V, int seq_len, int kv_len, int head_dim)
{
    if (seq_len <= 0 || head_dim <= 0) return;
    hipLaunchKernelGGL(attention_apply_k, dim3(blocks_for(head_dim), seq_len), dim3(kBlock), 0, stream(), dst,
                       scores, V, seq_len, kv_len, head_dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_attention_single(float *dst, const float *q, const float *k_cache, const float *v_cache, float *att_buf,
                           int kv_len, int head_dim, int kv_head, int kv_dim)
{
    if (kv_len <= 0 || head_dim <= 0) return;
    if (kv_len > kMaxLdsScores && !att_buf) {
        HOLO_REJECT("cuda_attention_single: kv_len beyond 12288 needs att_buf");
        return;
    }
    hipLaunchKernelGGL(attention_single_k, dim3(1), dim3(256), 0, stream(), dst, q, k_cache, v_cache, att_buf,
                       kv_len, head_dim, kv_head, kv_dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_multi_head_attention(float *dst, const float *q, const float *k_cache, const float *v_cache, int kv_len,
                               int head_dim, int n_heads, int n_kv_heads)
{
    if (kv_len <= 0 || n_heads <= 0) return;
    if (!dst || !q || !k_cache || !v_cache || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) {
        HOLO_REJECT("cuda_multi_head_attention: null pointer or n_heads not a multiple of n_kv_heads");
        return;
    }
    if (decode_attention_fits(q, k_cache, v_cache, head_dim)) {
        decode_attention(dst, q, k_cache, v_cache, kv_len, head_dim, n_heads, n_kv_heads);
        return;
    }
    if (kv_len > kMaxLdsScores) {
        HOLO_REJECT("cuda_multi_head_attention: kv_len <= 12288 required for this head_dim or alignment");
        return;
    }
    hipLaunchKernelGGL(mha_k, dim3(n_heads), dim3(256), 0, stream(), dst, q, k_cache, v_cache, kv_len, head_dim,
                       n_heads, n_kv_heads);
    HOLO_LAUNCH_CHECK();
}

void cuda_rope_apply(float *q, float *k, int pos, int head_dim, int n_heads, int n_kv_heads, float freq_base)
{
    int h = n_heads > n_kv_heads ? n_heads : n_kv_heads;
    if (h <= 0 || head_dim < 2) return;
    if (head_dim / 2 > 1024) {
        HOLO_REJECT("cuda_rope_apply: head_dim > 2048");
        return;
    }
    hipLaunchKernelGGL(rope_k, dim3(h), dim3(head_dim / 2), 0, stream(), q, k, pos, head_dim, n_heads, n_kv_heads,
                       freq_base);
    HOLO_LAUNCH_CHECK();
}

void cuda_get_embedding_f32(float *dst, const float *embeddings, int token, int dim, int vocab_size)
{
    (void)vocab_size;
    if (dim <= 0) return;
    hipLaunchKernelGGL(emb_f32_k, dim3(blocks_for(dim)), dim3(kBlock), 0, stream(), dst, embeddings, token, dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_get_embedding_f16(float *dst, const void *embeddings, int token, int dim, int vocab_size)
{
    (void)vocab_size;
    if (dim <= 0) return;
    hipLaunchKernelGGL(emb_f16_k, dim3(blocks_for(dim)), dim3(kBlock), 0, stream(), dst,
                       (const uint16_t *)embeddings, token, dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_get_embedding_q8_0(float *dst, const void *embeddings, int token, int dim, int vocab_size)
{
    (void)vocab_size;
    if (dim <= 0) return;
    hipLaunchKernelGGL(emb_q8_0_k, dim3(blocks_for(dim)), dim3(kBlock), 0, stream(), dst,
                       (const uint8_t *)embeddings, token, dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_get_embedding_q4_0(float *dst, const void *embeddings, int token, int dim, int vocab_size)
{
    (void)vocab_size;
    if (dim <= 0) return;
    hipLaunchKernelGGL(emb_q4_0_k, dim3(blocks_for(dim)), dim3(kBlock), 0, stream(), dst,
                       (const uint8_t *)embeddings, token, dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_get_embedding_q6_k(float *dst, const void *embeddings, int token, int dim, int vocab_size)
{
    (void)vocab_size;
    if (dim <= 0) return;
    hipLaunchKernelGGL(emb_q6_k_k, dim3(blocks_for(dim)), dim3(kBlock), 0, stream(), dst,
                       (const uint8_t *)embeddings, token, dim);
    HOLO_LAUNCH_CHECK();
}

int cuda_argmax(const float *x, int n)
{
    if (n <= 0) return 0;
    if (!g_argmax) HOLO_CHECK(hipMalloc(&g_argmax, sizeof(int)));
    if (!g_argmax) return 0;
    hipLaunchKernelGGL(argmax_k, dim3(1), dim3(1024), 0, stream(), x, n, g_argmax);
    HOLO_LAUNCH_CHECK();
    int r = 0;
    HOLO_CHECK(hipMemcpyAsync(&r, g_argmax, sizeof(int), hipMemcpyDeviceToHost, stream()));
    HOLO_CHECK(hipStreamSynchronize(stream()));
    return r;
}

void cuda_matmul_f32(float *dst, const float *M, const float *v, int out_dim, int in_dim)
{
    if (out_dim <= 0) return;
    hipLaunchKernelGGL(gemv_f32_k, dim3(blocks_for(out_dim, 4)), dim3(256), 0, stream(), dst, M, v, out_dim, in_dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_matmul_f16(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    if (out_dim <= 0) return;
    hipLaunchKernelGGL(gemv_f16_k, dim3(blocks_for(out_dim, 4)), dim3(256), 0, stream(), dst, (const uint16_t *)M, v,
                       out_dim, in_dim);
    HOLO_LAUNCH_CHECK();
}

void cuda_matmul_q6_k(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    if (out_dim <= 0) return;
    if (!M) {
        // matmul_q with a NULL matrix writes zeros (llm.c:772-775)
        fill_bytes(dst, 0, sizeof(float) * out_dim);
        return;
    }
    if (((uintptr_t)M & 1u) || ((uintptr_t)v & 15u)) {
        // the task kernel needs 2-byte-aligned blocks and 16-byte-aligned activations
        launch_timed(gemv_q6_k_k, dim3(blocks_for(out_dim, 4)), dim3(256), 0, dst, (const uint8_t *)M, v, out_dim,
                     in_dim);
        HOLO_LAUNCH_CHECK();
        return;
    }
    const int R = q6_rows_per_wave(out_dim);
    const dim3 grid((out_dim + 4 * R - 1) / (4 * R));
    const uint8_t *W = (const uint8_t *)M;
    if (R == 4)
        launch_timed(gemv_q6_k2_k<4>, grid, dim3(256), 0, dst, W, v, out_dim, in_dim);
    else if (R == 2)
        launch_timed(gemv_q6_k2_k<2>, grid, dim3(256), 0, dst, W, v, out_dim, in_dim);
    else
        launch_timed(gemv_q6_k2_k<1>, grid, dim3(256), 0, dst, W, v, out_dim, in_dim);
    HOLO_LAUNCH_CHECK();
}

void holo_rms_norm_rows(float *dst, const float *x, const float *weight, int rows, int n, float eps)
{
    if (rows <= 0 || n <= 0) return;
    if (!dst || !x) {
        HOLO_REJECT("holo_rms_norm_rows: null pointer");
        return;
    }
    const bool v4 = n % 4 == 0 && !(((uintptr_t)dst | (uintptr_t)x | (uintptr_t)weight) & 15);
    if (v4 && n <= 1024 * 4)
        hipLaunchKernelGGL(rms_norm_rows4_k<4>, dim3(rows), dim3(256), 0, stream(), dst, x, weight, n, eps);
    else if (v4 && n <= 1024 * 16)
        hipLaunchKernelGGL(rms_norm_rows4_k<16>, dim3(rows), dim3(256), 0, stream(), dst, x, weight, n, eps);
    else
        hipLaunchKernelGGL(rms_norm_rows_k, dim3(rows), dim3(256), 0, stream(), dst, x, weight, n, eps);
    HOLO_LAUNCH_CHECK();
}

void holo_rope_rows(float *q, float *k, int rows, int pos0, int head_dim, int n_heads, int n_kv_heads,
                    float freq_base)
{
    const int h = n_heads > n_kv_heads ? n_heads : n_kv_heads;
    if (rows <= 0 || h <= 0 || head_dim < 2) return;
    if (head_dim / 2 > 1024 || !q || !k) {
        HOLO_REJECT("holo_rope_rows: null pointer or head_dim > 2048");
        return;
    }
    // 256 threads (whole head groups of hd/2 pair indices), or one group when hd/2 > 256;
    // four heads per group
    const int half = head_dim / 2, threads = half <= 256 ? 256 / half * half : half;
    const int per_wg = 4 * (threads / half);
    hipLaunchKernelGGL(rope_rows_k, dim3(rows, (n_heads + n_kv_heads + per_wg - 1) / per_wg), dim3(threads), 0,
                       stream(), q, k, pos0, head_dim, n_heads, n_kv_heads, freq_base);
    HOLO_LAUNCH_CHECK();
}

void holo_embedding_rows(float *dst, const void *embeddings, const int *tokens, int rows, int dim, int type)
{
    if (rows <= 0 || dim <= 0) return;
    if (!dst || !embeddings || !tokens) {
        HOLO_REJECT("holo_embedding_rows: null pointer");
        return;
    }
    if (type != HOLO_TYPE_F32 && type != HOLO_TYPE_F16 && type != HOLO_TYPE_Q8_0 && type != HOLO_TYPE_Q4_0 &&
        type != HOLO_TYPE_Q6_K && type != HOLO_TYPE_Q4_K) {
        HOLO_REJECT("holo_embedding_rows: type without a lookup kernel");
        return;
    }
    hipLaunchKernelGGL(emb_rows_k, dim3(blocks_for(dim), rows), dim3(kBlock), 0, stream(), dst,
                       (const uint8_t *)embeddings, tokens, dim, type);
    HOLO_LAUNCH_CHECK();
}

void holo_attention_prefill(float *out, const float *q, const float *k_cache, const float *v_cache, int rows,
                            int pos0, int head_dim, int n_heads, int n_kv_heads)
{
    if (rows <= 0 || n_heads <= 0) return;
    if (!out || !q || !k_cache || !v_cache || pos0 < 0 || head_dim <= 0 || head_dim > kAttMaxHd || head_dim % 4 ||
        n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache) & 15)) {
        HOLO_REJECT("holo_attention_prefill: null or misaligned pointer, pos0 < 0, head_dim not a multiple of 4 in "
                    "4..128, or heads not grouped");
        return;
    }
    if (rows <= 4) {
        // a decode step (or a few rows): each row on the key-split kernel,
        // row m attending to positions 0 .. pos0 + m
        for (int m = 0; m < rows; m++)
            decode_attention(out + (int64_t)m * n_heads * head_dim, q + (int64_t)m * n_heads * head_dim, k_cache,
                             v_cache, pos0 + m + 1, head_dim, n_heads, n_kv_heads);
        return;
    }
    if (head_dim == 128 || head_dim == 64 || head_dim == 32) {
        if (head_dim == 128) launch_attn_prefill_mfma<128>(out, q, k_cache, v_cache, rows, pos0, n_heads, n_kv_heads);
        else if (head_dim == 64) launch_attn_prefill_mfma<64>(out, q, k_cache, v_cache, rows, pos0, n_heads, n_kv_heads);
        else launch_attn_prefill_mfma<32>(out, q, k_cache, v_cache, rows, pos0, n_heads, n_kv_heads);
        return;
    }
    static bool attr = false;
    if (!attr) {
        HOLO_CHECK(hipFuncSetAttribute((const void *)attention_prefill_k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)kAttLds));
        attr = true;
    }
    hipLaunchKernelGGL(attention_prefill_k, dim3((rows + kAttQ - 1) / kAttQ, n_heads), dim3(256), kAttLds, stream(),
                       out, q, k_cache, v_cache, rows, pos0, head_dim, n_heads, n_kv_heads);
    HOLO_LAUNCH_CHECK();
}

// gpu_matmul of src/ai/llm_cuda.c:140-163: type -> entry point.
void holo_matmul(float *dst, const void *M, const float *v, int out_dim, int in_dim, int type)
{
    switch (type) {
    case HOLO_TYPE_Q8_0: cuda_matmul_q8_0(dst, M, v, out_dim, in_dim); break;
    case HOLO_TYPE_Q4_0: cuda_matmul_q4_0(dst, M, v, out_dim, in_dim); break;
    case HOLO_TYPE_Q4_K: cuda_matmul_q4_k(dst, M, v, out_dim, in_dim); break;
    case HOLO_TYPE_Q6_K: cuda_matmul_q6_k(dst, M, v, out_dim, in_dim); break;
    case HOLO_TYPE_F16: cuda_matmul_f16(dst, M, v, out_dim, in_dim); break;
    default: cuda_matmul_f32(dst, (const float *)M, v, out_dim, in_dim); break;
    }
}

}  // extern "C"
