/*
 * holo_oracle.c -- CPU restatement of the Holo engine's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library under google-classic_amd/.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it, and only as the checker or the
 * timed CPU baseline.  The product path never calls into it.
 *
 * Every routine restates an algorithm of the reference CPU path
 * (privuser2738/google-classic, src/ai) from its source text; the citation is
 * given per function.  It is written from scratch and compiled with
 * -ffp-contract=off and without -ffast-math, so each floating-point
 * expression rounds exactly as the C source of the reference reads.
 *
 * Pinning (see tests/test_oracle.py):
 *   f16 -> f32        all 65536 codes vs numpy.float16 and vs the reference
 *                     build in oracle/_ref (closed form: IEEE binary16)
 *   dequant q8_0/q4_0 one-hot byte sweeps (closed form d*q, d*(nib-8)) and
 *                     bit-exact vs oracle/_ref (strict build)
 *   dequant q4_k      one-hot sweeps over every scale bit and every qs nibble
 *                     and bit-exact vs oracle/_ref (strict build)
 *   matmul_*          fp64 brute force, one-hot and all-ones activations, and
 *                     oracle/_ref matmul_q (release and strict builds)
 *   quantize_act /    build-defined (the reference has no activation
 *   gemm_q4_0_q8_0    quantizer or batched path): pinned by invariants
 *                     |q|<=127, |x-d*q|<=d/2 (+f16 rounding of d), by an
 *                     independent numpy integer restatement and, for the
 *                     block-order fused rescale, by an exact rational
 *                     evaluation of each fmaf step.
 *   gemm_q4_0_f16     build-defined (f16 prefill product): pinned by a closed
 *                     form on inputs exact in f16, by the reference-pinned
 *                     oracle_matmul_q4_0 within the f16 rounding bound, and
 *                     by numpy's own float16 rounding of both operands.
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>
#include <string.h>

#define QK32 32
#define QKK 256

typedef struct { uint16_t d; int8_t qs[32]; } oq8_0;                 /* quant.h:43-48  (34 B) */
typedef struct { uint16_t d; uint8_t qs[16]; } oq4_0;                /* quant.h:54-59  (18 B) */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } oq4_k; /* quant.h:114-120 (144 B) */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } oq6_k; /* quant.h:103-110 (210 B) */

_Static_assert(sizeof(oq8_0) == 34, "q8_0 block size");
_Static_assert(sizeof(oq4_0) == 18, "q4_0 block size");
_Static_assert(sizeof(oq4_k) == 144, "q4_k block size");
_Static_assert(sizeof(oq6_k) == 210, "q6_k block size");

/* ------------------------------------------------------------------------ */
/* f16 -> f32.  quant.c:44-82: exact binary16 decode; subnormals normalised,
 * Inf kept, NaN keeps its payload shifted into the top of the f32 mantissa. */
float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            /* value = m * 2^-24; normalise so the leading one sits at bit 10 */
            int shift = 0;
            while ((m & 0x400u) == 0) { m <<= 1; shift++; }
            m &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 + 1 - shift) << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ------------------------------------------------------------------------ */
/* Dequantisation.                                                          */

/* quant.c:118-128: y[32i+j] = d * qs[j] */
void oracle_dequant_q8_0(const void *src, float *y, int k)
{
    const oq8_0 *x = (const oq8_0 *)src;
    int nb = k / QK32;
    for (int i = 0; i < nb; i++) {
        float d = oracle_f16_to_f32(x[i].d);
        for (int j = 0; j < 32; j++) y[i * 32 + j] = d * (float)x[i].qs[j];
    }
}

/* quant.c:136-153: low nibble of qs[j] -> j, high nibble -> j+16, minus 8 */
void oracle_dequant_q4_0(const void *src, float *y, int k)
{
    const oq4_0 *x = (const oq4_0 *)src;
    int nb = k / QK32;
    for (int i = 0; i < nb; i++) {
        float d = oracle_f16_to_f32(x[i].d);
        for (int j = 0; j < 16; j++) {
            int lo = (x[i].qs[j] & 0x0F) - 8;
            int hi = (x[i].qs[j] >> 4) - 8;
            y[i * 32 + j] = d * (float)lo;
            y[i * 32 + j + 16] = d * (float)hi;
        }
    }
}

/* The 6-bit scale/min unpack of the reference CPU path, quant.c:290-297
 * (same text at quant.c:555-562).  Note the high part of sub-blocks 4..7:
 * the 4-bit field of byte 8+j is shifted left by 2 and the top two bits of
 * byte j (scales) / byte 4+j (mins) fill bits 0..1.  This differs from
 * llama.cpp's get_scale_min_k4; the CPU layout is the parity target. */
void oracle_q4_k_unpack_scales(const uint8_t *sp, uint8_t *sc, uint8_t *mn)
{
    for (int j = 0; j < 4; j++) {
        sc[j] = sp[j] & 0x3F;
        mn[j] = sp[j + 4] & 0x3F;
    }
    for (int j = 0; j < 4; j++) {
        sc[j + 4] = (uint8_t)(((sp[j + 8] & 0x0F) << 2) | (sp[j] >> 6));
        mn[j + 4] = (uint8_t)(((sp[j + 8] >> 4) << 2) | (sp[j + 4] >> 6));
    }
}

/* quant.c:277-311.  Sub-block j reads qs[16j..16j+15]: low nibble -> 32j+l,
 * high nibble -> 32j+l+16.  w = (d*sc)*q - dmin*m, two roundings. */
void oracle_dequant_q4_k(const void *src, float *y, int k)
{
    const oq4_k *x = (const oq4_k *)src;
    int nb = k / QKK;
    for (int i = 0; i < nb; i++) {
        float d = oracle_f16_to_f32(x[i].d);
        float dmin = oracle_f16_to_f32(x[i].dmin);
        uint8_t sc[8], mn[8];
        oracle_q4_k_unpack_scales(x[i].scales, sc, mn);
        for (int j = 0; j < 8; j++) {
            float s = d * (float)sc[j];
            float m = dmin * (float)mn[j];
            for (int l = 0; l < 16; l++) {
                uint8_t b = x[i].qs[16 * j + l];
                float p0 = s * (float)(b & 0x0F);
                float p1 = s * (float)(b >> 4);
                y[i * 256 + 32 * j + l] = p0 - m;
                y[i * 256 + 32 * j + l + 16] = p1 - m;
            }
        }
    }
}

/* quant.c:241-271 (llama.cpp-compatible Q6_K layout). */
void oracle_dequant_q6_k(const void *src, float *y, int k)
{
    const oq6_k *x = (const oq6_k *)src;
    int nb = k / QKK;
    for (int i = 0; i < nb; i++) {
        float d = oracle_f16_to_f32(x[i].d);
        const uint8_t *ql = x[i].ql;
        const uint8_t *qh = x[i].qh;
        const int8_t *sc = x[i].scales;
        float *yy = y + (size_t)i * 256;
        for (int half = 0; half < 2; half++) {
            for (int l = 0; l < 32; l++) {
                int is = l / 16;
                int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                /* d * sc * q evaluates left to right: (d*sc)*q */
                yy[l + 0] = (d * (float)sc[is + 0]) * (float)q1;
                yy[l + 32] = (d * (float)sc[is + 2]) * (float)q2;
                yy[l + 64] = (d * (float)sc[is + 4]) * (float)q3;
                yy[l + 96] = (d * (float)sc[is + 6]) * (float)q4;
            }
            yy += 128;
            ql += 64;
            qh += 32;
            sc += 8;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Matrix-vector products: dst[out] = M[out][in] . v[in], fp32.             */
/* The summation order of each routine is the scalar order of the cited     */
/* reference loop.  Rows are independent, so the OpenMP row split changes   */
/* nothing in the result.                                                    */

/* llm.c:876-890 (scalar Q8_0 branch of matmul_q): one accumulator per row,
 * sum += (scale*q)*v[base+k] for k = 0..31, blocks in order. */
void oracle_matmul_q8_0(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    const oq8_0 *blk = (const oq8_0 *)M;
    int nb = in_dim / QK32;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < out_dim; i++) {
        const oq8_0 *row = blk + (size_t)i * nb;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            float scale = oracle_f16_to_f32(row[b].d);
            for (int k = 0; k < 32; k++) {
                float w = scale * (float)row[b].qs[k];
                sum = sum + w * v[b * 32 + k];
            }
        }
        dst[i] = sum;
    }
}

/* llm.c:893-915 (Q4_0 branch of matmul_q): one accumulator per row; for each
 * block, k = 0..15: sum += (scale*q_lo)*v[base+k]; sum += (scale*q_hi)*v[base+k+16]. */
void oracle_matmul_q4_0(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    const oq4_0 *blk = (const oq4_0 *)M;
    int nb = in_dim / QK32;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < out_dim; i++) {
        const oq4_0 *row = blk + (size_t)i * nb;
        float sum = 0.0f;
        for (int b = 0; b < nb; b++) {
            float scale = oracle_f16_to_f32(row[b].d);
            for (int k = 0; k < 16; k++) {
                int q0 = (row[b].qs[k] & 0xF) - 8;
                int q1 = (row[b].qs[k] >> 4) - 8;
                float w0 = scale * (float)q0;
                float w1 = scale * (float)q1;
                sum = sum + w0 * v[b * 32 + k];
                sum = sum + w1 * v[b * 32 + k + 16];
            }
        }
        dst[i] = sum;
    }
}

/* quant.c:541-580 via mat_vec_q4_k (quant.c:626-633), reached from matmul_q
 * (llm.c:916-918): per row one accumulator; superblock i, sub-block j,
 * l = 0..15: sum += (sc*lo - m)*y[..l]; sum += (sc*hi - m)*y[..l+16]. */
void oracle_matmul_q4_k(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    const oq4_k *blk = (const oq4_k *)M;
    int nb = in_dim / QKK;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < out_dim; r++) {
        const oq4_k *row = blk + (size_t)r * nb;
        float sum = 0.0f;
        for (int i = 0; i < nb; i++) {
            float d = oracle_f16_to_f32(row[i].d);
            float dmin = oracle_f16_to_f32(row[i].dmin);
            uint8_t sc[8], mn[8];
            oracle_q4_k_unpack_scales(row[i].scales, sc, mn);
            for (int j = 0; j < 8; j++) {
                float s = d * (float)sc[j];
                float m = dmin * (float)mn[j];
                int base = i * 256 + j * 32;
                for (int l = 0; l < 16; l++) {
                    uint8_t b = row[i].qs[j * 16 + l];
                    float w0 = s * (float)(b & 0xF);
                    float w1 = s * (float)(b >> 4);
                    w0 = w0 - m;
                    w1 = w1 - m;
                    sum = sum + w0 * v[base + l];
                    sum = sum + w1 * v[base + l + 16];
                }
            }
        }
        dst[r] = sum;
    }
}

/* quant.c:600-606 + 643-646: Q6_K dot = sum over the dequantised superblock. */
void oracle_matmul_q6_k(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    const oq6_k *blk = (const oq6_k *)M;
    int nb = in_dim / QKK;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < out_dim; r++) {
        float tmp[256];
        float sum = 0.0f;
        for (int i = 0; i < nb; i++) {
            oracle_dequant_q6_k(blk + (size_t)r * nb + i, tmp, 256);
            for (int j = 0; j < 256; j++) sum = sum + tmp[j] * v[i * 256 + j];
        }
        dst[r] = sum;
    }
}

/* fp64 truth: the same dequantised weights (bit-exact f32 values from the
 * dequant routines above), products and sums in double. */
void oracle_matmul_f64(double *dst, const float *W, const float *v, int out_dim, int in_dim)
{
#pragma omp parallel for schedule(static)
    for (int i = 0; i < out_dim; i++) {
        const float *row = W + (size_t)i * in_dim;
        double s = 0.0;
        for (int j = 0; j < in_dim; j++) s += (double)row[j] * (double)v[j];
        dst[i] = s;
    }
}

/* ------------------------------------------------------------------------ */
/* Fused Q8_0 multi-GEMV epilogue (cuda_ops.cu:1380-1383): out = silu(g)*u,
 * silu(g) = g / (1 + expf(-g)). */
void oracle_silu_mul(float *out, const float *g, const float *u, int n)
{
    for (int i = 0; i < n; i++) {
        float s = g[i] / (1.0f + expf(-g[i]));
        out[i] = s * u[i];
    }
}

/* ------------------------------------------------------------------------ */
/* Build-defined activation quantiser and batched int8 product.             */
/* The reference has neither (its prompt loop is one GEMV per token,        */
/* llm.c:1049); these restate this build's own specification.               */

/* f32 -> f16, round to nearest even (IEEE 754), with subnormals. */
uint16_t oracle_f32_to_f16_rne(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {                       /* Inf / NaN */
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> Inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: f16 subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;  /* < 2^-25 rounds to 0 (2^-25 ties to even 0) */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        /* value = m * 2^(e-150); f16 subnormal unit = 2^-24 -> q = m * 2^(e-126) */
        uint32_t shift = 126u - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* Q8_0 activation quantiser (build-defined, llama.cpp convention):
 * per 32-block, amax = max|x|, d = amax/127, id = d ? 1/d : 0,
 * q = round-half-away(x*id) clamped to [-127,127] (never exceeds it),
 * stored d = f16_rne(d).  Output: rows*(k/32) blocks of 34 B. */
void oracle_quantize_act_q8_0(const float *x, void *dst, int rows, int k)
{
    oq8_0 *out = (oq8_0 *)dst;
    int nb = k / QK32;
    for (int r = 0; r < rows; r++) {
        for (int b = 0; b < nb; b++) {
            const float *xb = x + (size_t)r * k + b * 32;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) {
                float a = fabsf(xb[j]);
                if (a > amax) amax = a;
            }
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            oq8_0 *o = out + (size_t)r * nb + b;
            o->d = oracle_f32_to_f16_rne(d);
            for (int j = 0; j < 32; j++) {
                float t = xb[j] * id;
                int q = (int)roundf(t);
                if (q > 127) q = 127;
                if (q < -127) q = -127;
                o->qs[j] = (int8_t)q;
            }
        }
    }
}

/* Batched product over Q8_0 activations and Q4_0 weights:
 *   Y[m][n] = sum_b f16(dw[n,b]) * f16(dx[m,b]) * I[m,n,b],
 *   I[m,n,b] = sum_{k<32} (qw[n,b,k]-8) * qx[m,b,k]    (exact in int32)
 * The per-block scale s = dw*dx (a product of two f16 values, exact in fp32)
 * is applied with one fused multiply-add per block, in block order:
 *   acc = fmaf((float)I, s, acc)
 * (I is exact in fp32: |I| <= 32*8*127).  fmaf rounds once (C99 7.12.13). */
void oracle_gemm_q4_0_q8_0(float *Y, const void *W, const void *Xq, int M, int N, int K)
{
    const oq4_0 *w = (const oq4_0 *)W;
    const oq8_0 *xq = (const oq8_0 *)Xq;
    int nb = K / QK32;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int b = 0; b < nb; b++) {
                const oq4_0 *wb = w + (size_t)n * nb + b;
                const oq8_0 *xb = xq + (size_t)m * nb + b;
                int32_t I = 0;
                for (int j = 0; j < 16; j++) {
                    I += ((wb->qs[j] & 0xF) - 8) * xb->qs[j];
                    I += ((wb->qs[j] >> 4) - 8) * xb->qs[j + 16];
                }
                float s = oracle_f16_to_f32(wb->d) * oracle_f16_to_f32(xb->d);
                acc = fmaf((float)I, s, acc);
            }
            Y[(size_t)m * N + n] = acc;
        }
    }
}

/* Batched product over f16 activations and f16-dequantised Q4_0 weights:
 *   Y[m][n] = sum_k x16[m][k] * w16[n][k]
 *   x16 = f16_rne(x),  w16 = f16_rne(f16(dw[n,b]) * (q[n][k] - 8))
 * The products of two f16 values and their sum over k are exact in double up
 * to its own rounding (at these K far below the fp32 accumulation error the
 * GPU is held to), so Y is the truth of the rounded operands.  A[m][n] =
 * sum_k |x16 * w16| scales that error bound.                                */
void oracle_gemm_q4_0_f16(double *Y, double *A, const float *X, const void *W, int M, int N, int K)
{
    const oq4_0 *w = (const oq4_0 *)W;
    int nb = K / QK32;
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            double acc = 0.0, aa = 0.0;
            for (int b = 0; b < nb; b++) {
                const oq4_0 *wb = w + (size_t)n * nb + b;
                const float dw = oracle_f16_to_f32(wb->d);
                for (int j = 0; j < 32; j++) {
                    const int q = j < 16 ? (wb->qs[j] & 0xF) : (wb->qs[j - 16] >> 4);
                    const float wq = oracle_f16_to_f32(oracle_f32_to_f16_rne(dw * (float)(q - 8)));
                    const float xq = oracle_f16_to_f32(oracle_f32_to_f16_rne(X[(size_t)m * K + (size_t)b * 32 + j]));
                    const double p = (double)wq * (double)xq;
                    acc += p;
                    aa += fabs(p);
                }
            }
            Y[(size_t)m * N + n] = acc;
            if (A) A[(size_t)m * N + n] = aa;
        }
    }
}
