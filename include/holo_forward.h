/*
 * holo_forward.h -- the Llama forward over a prompt of M tokens in one pass:
 * row-batched ops and a driver that runs all M rows through every layer at
 * once.
 *
 * The reference processes a prompt one token at a time: llm_forward runs
 * every layer for token t before token t+1 (src/ai/llm.c:1015-1270, CPU), and
 * the GPU loop does the same with one GEMV per matrix and token
 * (src/ai/llm_cuda.c:574-891).  holo_llama_forward computes the same result
 * for tokens[0..n) at positions pos0..pos0+n-1:
 *   - each matrix multiplies all n rows at once (holo_matmul_rows: the MFMA
 *     prefill GEMM with n >= 64 -- Q4_0 unpacked in the GEMM, the other
 *     types over an f16 panel dequantised first -- otherwise one GEMV per
 *     row);
 *   - RoPE, the KV-cache writes and the norms take all rows in one launch;
 *   - attention is causal over the prompt (holo_attention_prefill): row m sees
 *     positions 0..pos0+m, as token pos0+m does in the reference.
 * The logits of the last token are written, as after the reference's loop.
 * n = 1 is one decode step.
 *
 * Supported: the Llama layer of llm.c (attention norm, q/k/v/o, SwiGLU FFN,
 * final norm, output head); no QKV biases, QK-norm, post-norms or embedding
 * scaling (the Qwen/Gemma branches of llm.c), head_dim <= 128.
 */
#ifndef HOLO_FORWARD_H
#define HOLO_FORWARD_H

#include "holo_gguf.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- row-batched ops ---------------------------------------------------------
 * rows consecutive vectors; each row as the single-vector op would compute it. */

/* cuda_rms_norm (cuda_ops.h:75) on each of rows rows of n floats.            */
void holo_rms_norm_rows(float *dst, const float *x, const float *weight, int rows, int n, float eps);
/* cuda_rope_apply (cuda_ops.h:117) with row r at position pos0 + r; q rows of
 * n_heads*head_dim floats, k rows of n_kv_heads*head_dim.                    */
void holo_rope_rows(float *q, float *k, int rows, int pos0, int head_dim, int n_heads, int n_kv_heads,
                    float freq_base);
/* cuda_get_embedding_* (cuda_ops.h:121-129) for tokens[0..rows) (a device
 * array of int): F32, F16, Q8_0, Q4_0, Q6_K; and Q4_K, which has no lookup
 * op in the reference, as the bit-exact dequantize_row_q4_k of each row
 * (quant.c:277-311), as llm.c:998-1003 looks Q4_K rows up.                 */
void holo_embedding_rows(float *dst, const void *embeddings, const int *tokens, int rows, int dim, int type);
/* Causal attention: row m of q (position pos0 + m) against positions
 * 0..pos0+m of this layer's caches [pos][n_kv_heads*head_dim], which must
 * already hold those positions; head h reads KV head h / (n_heads /
 * n_kv_heads) (cuda_multi_head_attention, cuda_ops.h:112, per row).           */
void holo_attention_prefill(float *out, const float *q, const float *k_cache, const float *v_cache, int rows,
                            int pos0, int head_dim, int n_heads, int n_kv_heads);
/* Y[rows][out] = X[rows][in] . W^T for any GEMV type (holo_matmul per row).
 * rows >= 64 with in_dim whole blocks takes the batched MFMA product
 * (holo_matmul_batch) unless `exact` is set.                                  */
void holo_matmul_rows(float *Y, const void *W, const float *X, int rows, int out_dim, int in_dim, int type,
                      int exact);

/* ---- the model --------------------------------------------------------------- */

typedef struct {
    const float *attn_norm;  /* [dim] F32, or NULL (no norm) */
    const void *wq, *wk, *wv, *wo;
    int wq_type, wk_type, wv_type, wo_type;
    const float *ffn_norm;   /* [dim] F32, or NULL */
    const void *w1, *w2, *w3; /* gate [ffn][dim], down [dim][ffn], up [ffn][dim] */
    int w1_type, w2_type, w3_type;
} holo_llama_layer_t;

typedef struct {
    int n_layers, dim, n_heads, n_kv_heads, head_dim, ffn_dim;
    int vocab;               /* rows of the output head (logits written) */
    int max_seq;             /* positions held by the caches */
    float rms_eps, rope_base;
    const void *tok_emb;     /* [vocab][dim] blocks */
    int emb_type;
    const float *out_norm;   /* [dim] F32, or NULL */
    const void *output;      /* [vocab][dim] */
    int out_type;
    float *key_cache, *value_cache;   /* device, [n_layers][max_seq][n_kv_heads*head_dim] */
    const holo_llama_layer_t *layers; /* host array of n_layers */
} holo_llama_t;

#define HOLO_FORWARD_EXACT 1 /* every matmul as fp32-activation GEMVs (no Q8_0 activations) */

/* Runs tokens[0..n) (host array) at positions pos0..pos0+n-1, writes the
 * caches' rows pos0..pos0+n-1 of every layer and the last token's logits
 * (device, [vocab]).  0, or HOLO_EINVAL for a model or shape outside the
 * supported set (nothing launched).  Scratch is stream-ordered.               */
int holo_llama_forward(const holo_llama_t *m, const int *tokens, int n, int pos0, float *logits, int flags);

/* holo_prefill_prepare for every Q6_K layer matrix of m (q, k, v, o, gate,
 * down, up; the output head runs the GEMV), and holo_prefill_release for
 * them: the prompt forward then reads their repacked copies (1 byte per
 * weight of those matrices) instead of repacking each one per call.  No
 * reference counterpart.  0, or the first failing holo_prefill_prepare's
 * code (the matrices prepared before it are released).                      */
int holo_llama_prepare(const holo_llama_t *m);
void holo_llama_release(const holo_llama_t *m);

/* Fills m and layers[0..n_layers) from an uploaded GGUF file
 * (holo_gguf_upload), with the reference loader's tensor names and model
 * parameters (llm.c:344-533, 617-660): token_embd, blk.N.{attn_norm,
 * attn_q, attn_k, attn_v, attn_output, ffn_norm, ffn_gate, ffn_down,
 * ffn_up}, output_norm, output (tied to token_embd when absent).  vocab is
 * token_embd's row count.  The caller sets max_seq and the caches.
 * 0, or -1 when a required tensor is missing, n_layers > max_layers, or
 * holo_llama_gguf_check rejects the file.                                   */
int holo_llama_from_gguf(const holo_gguf_t *g, holo_llama_t *m, holo_llama_layer_t *layers, int max_layers);
/* 0 when a parsed GGUF file (host-side parse is enough) is the plain Llama
 * body this forward runs; -1 when it needs a branch of the reference's
 * forward that is not built here: a Gemma architecture (general.architecture
 * contains "gemma"), or any blk.N.attn_{q,k,v}.bias, attn_{q,k}_norm.weight,
 * post_attention_norm.weight or post_ffw_norm.weight tensor (the Qwen and
 * Gemma branches of llm.c:451-521, 1037-1133).                               */
int holo_llama_gguf_check(const holo_gguf_t *g);

#ifdef __cplusplus
}
#endif

#endif /* HOLO_FORWARD_H */
