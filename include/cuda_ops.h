/*
 * cuda_ops.h -- C ABI of the Holo GPU op boundary, served on MI355X by
 * libholo_mi355x.so (HIP, gfx950).
 *
 * The names, argument order and meaning are those of the reference header
 * include/cuda_ops.h of privuser2738/google-classic; each declaration below
 * cites the line it replaces.  The reference inference loop
 * (src/ai/llm_cuda.c) links against this library unchanged.
 *
 * Conventions (observed in the reference, kept here):
 *  - every pointer argument except host buffers of the memcpy calls is a
 *    device pointer obtained from cuda_malloc;
 *  - quantized matrices are the raw GGUF block stream, row-major
 *    [out_dim][in_dim/QK] blocks, no padding; in_dim is used as
 *    in_dim/QK blocks (truncating), as the reference does;
 *  - dst is fully overwritten; dst must not alias the input vector;
 *  - ops are asynchronous on the library's stream (by default the null
 *    stream, as in the reference); cuda_sync / a blocking cuda_memcpy_d2h
 *    waits for them;
 *  - ops return void; a failed launch or invalid argument is printed to
 *    stderr and latched (holo_last_error() in holo_mi355x.h).
 */
#ifndef HOLO_MI355X_CUDA_OPS_H
#define HOLO_MI355X_CUDA_OPS_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime (reference cuda_ops.h:18-40) ------------------------------- */
int cuda_init(void);                                              /* cuda_ops.h:18 */
void cuda_cleanup(void);                                          /* cuda_ops.h:19 */
bool cuda_available(void);                                        /* cuda_ops.h:20 */
void cuda_print_info(void);                                       /* cuda_ops.h:21 */
int cuda_get_device_count(void);                                  /* cuda_ops.h:24 */
size_t cuda_get_free_memory(void);                                /* cuda_ops.h:25 */
const char *cuda_get_device_name(void);                           /* cuda_ops.h:26 */
void *cuda_malloc(size_t size);                                   /* cuda_ops.h:29 */
void cuda_free(void *ptr);                                        /* cuda_ops.h:30 */
void cuda_memcpy_h2d(void *dst, const void *src, size_t size);    /* cuda_ops.h:31 */
void cuda_memcpy_d2h(void *dst, const void *src, size_t size);    /* cuda_ops.h:32 */
void cuda_memcpy_d2d(void *dst, const void *src, size_t size);    /* cuda_ops.h:33 */
void cuda_memcpy_d2d_async(void *dst, const void *src, size_t size); /* cuda_ops.h:34 */
void cuda_memcpy_d2h_async(void *dst, const void *src, size_t size); /* cuda_ops.h:35 */
void cuda_memset(void *ptr, int value, size_t size);              /* cuda_ops.h:36 */
void cuda_sync(void);                                             /* cuda_ops.h:39 */
void cuda_sync_copy(void);                                        /* cuda_ops.h:40 */

/* ---- quantized matrix-vector products: the hot path ---------------------
 * dst[i] = sum_j W[i][j] * v[j], W dequantised from GGUF blocks, fp32
 * accumulation.  Q4_K uses the CPU layout of src/ai/quant.c:277-311 for every
 * shape.                                                                    */
void cuda_matmul_q8_0(float *dst, const void *M, const float *v, int out_dim, int in_dim); /* cuda_ops.h:54 */
void cuda_matmul_q4_0(float *dst, const void *M, const float *v, int out_dim, int in_dim); /* cuda_ops.h:55 */
void cuda_matmul_q4_k(float *dst, const void *M, const float *v, int out_dim, int in_dim); /* cuda_ops.h:56 */
void cuda_matmul_q6_k(float *dst, const void *M, const float *v, int out_dim, int in_dim); /* cuda_ops.h:57 */
void cuda_matmul_f32(float *dst, const float *M, const float *v, int out_dim, int in_dim); /* cuda_ops.h:50 */
void cuda_matmul_f16(float *dst, const void *M, const float *v, int out_dim, int in_dim);  /* cuda_ops.h:51 */

/* Q, K and V rows in one launch: q_out = Wq.x [q_dim], k_out = Wk.x [kv_dim],
 * v_out = Wv.x [kv_dim].                                   cuda_ops.h:60-62 */
void cuda_batched_qkv_q8_0(float *q_out, float *k_out, float *v_out,
                           const void *Wq, const void *Wk, const void *Wv,
                           const float *x, int q_dim, int kv_dim, int in_dim);
/* out = silu(W1.x) * (W3.x), silu(g) = g/(1+exp(-g)).      cuda_ops.h:65-66 */
void cuda_batched_ffn_gate_up_q8_0(float *out, const void *W1, const void *W3,
                                   const float *x, int ffn_dim, int in_dim);

/* ---- vector, activation and normalisation ops (reference cuda_ops.h:43-80) */
void cuda_vec_add(float *dst, const float *a, const float *b, int n);   /* cuda_ops.h:43 */
void cuda_vec_mul(float *dst, const float *a, const float *b, int n);   /* cuda_ops.h:44 */
void cuda_vec_scale(float *dst, const float *a, float scale, int n);    /* cuda_ops.h:45 */
float cuda_vec_dot(const float *a, const float *b, int n);              /* cuda_ops.h:46 */
void cuda_silu(float *x, int n);                                        /* cuda_ops.h:69 */
void cuda_silu_mul(float *dst, const float *a, const float *b, int n);  /* cuda_ops.h:70 */
void cuda_gelu(float *x, int n);                                        /* cuda_ops.h:71 */
void cuda_relu(float *x, int n);                                        /* cuda_ops.h:72 */
void cuda_rms_norm(float *dst, const float *x, const float *weight, int n, float eps); /* cuda_ops.h:75 */
void cuda_layer_norm(float *dst, const float *x, const float *weight, const float *bias,
                     int n, float eps);                                 /* cuda_ops.h:76 */
void cuda_softmax(float *dst, const float *x, int n);                   /* cuda_ops.h:79 */
void cuda_softmax_inplace(float *x, int n);                             /* cuda_ops.h:80 */

/* ---- attention, RoPE, embedding, sampling (reference cuda_ops.h:83-133) -- */
void cuda_attention_scores(float *dst, const float *Q, const float *K,
                           int seq_len, int kv_len, int head_dim, float scale);   /* cuda_ops.h:83 */
void cuda_attention_apply(float *dst, const float *scores, const float *V,
                          int seq_len, int kv_len, int head_dim);                 /* cuda_ops.h:85 */
void cuda_attention_single(float *dst, const float *q, const float *k_cache, const float *v_cache,
                           float *att_buf, int kv_len, int head_dim, int kv_head, int kv_dim); /* cuda_ops.h:100 */
void cuda_multi_head_attention(float *dst, const float *q, const float *k_cache, const float *v_cache,
                               int kv_len, int head_dim, int n_heads, int n_kv_heads); /* cuda_ops.h:112 */
void cuda_rope_apply(float *q, float *k, int pos, int head_dim, int n_heads,
                     int n_kv_heads, float freq_base);                              /* cuda_ops.h:117 */
void cuda_get_embedding_f32(float *dst, const float *embeddings, int token, int dim, int vocab_size); /* cuda_ops.h:121 */
void cuda_get_embedding_f16(float *dst, const void *embeddings, int token, int dim, int vocab_size);  /* cuda_ops.h:123 */
void cuda_get_embedding_q8_0(float *dst, const void *embeddings, int token, int dim, int vocab_size); /* cuda_ops.h:125 */
void cuda_get_embedding_q4_0(float *dst, const void *embeddings, int token, int dim, int vocab_size); /* cuda_ops.h:127 */
void cuda_get_embedding_q6_k(float *dst, const void *embeddings, int token, int dim, int vocab_size); /* cuda_ops.h:129 */
int cuda_argmax(const float *x, int n);                                   /* cuda_ops.h:133 */

#ifdef __cplusplus
}
#endif

#endif /* HOLO_MI355X_CUDA_OPS_H */
