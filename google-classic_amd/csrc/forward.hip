// forward.hip -- the Llama forward over n prompt tokens in one pass (host
// driver over the row-batched ops), and the model descriptor from a GGUF file.
//
// Per layer, with all n rows at once (the reference runs this body once per
// token: llm.c:1063-1247 on the CPU, llm_cuda.c:598-880 on the GPU):
//   xb = rms_norm(x); q = Wq xb; cache rows pos0 + r: k = Wk xb, v = Wv xb
//   (written in place); rope(q, k) at pos0 + r; att = causal attention;
//   x += Wo att;
//   xb = rms_norm(x); h = silu(W1 xb) * (W3 xb); x += W2 h
// then the last row: rms_norm, output head -> logits (llm.c:1249-1263).
#include "common.h"

#include "../../include/holo_forward.h"

#include <string.h>

#include <string>

using namespace holo;

namespace {

bool rows_type_ok(int t)
{
    return t == HOLO_TYPE_F32 || t == HOLO_TYPE_F16 || t == HOLO_TYPE_Q4_0 || t == HOLO_TYPE_Q8_0 ||
           t == HOLO_TYPE_Q4_K || t == HOLO_TYPE_Q6_K;
}

bool layer_ok(const holo_llama_layer_t &l)
{
    return l.wq && l.wk && l.wv && l.wo && l.w1 && l.w2 && l.w3 && rows_type_ok(l.wq_type) && rows_type_ok(l.wk_type) &&
           rows_type_ok(l.wv_type) && rows_type_ok(l.wo_type) && rows_type_ok(l.w1_type) &&
           rows_type_ok(l.w2_type) && rows_type_ok(l.w3_type);
}

// A layer without a norm weight passes x through unchanged (llm.c:1084-1086,
// 1223-1225, 1251-1254).
void norm_or_copy(float *dst, const float *x, const float *w, int rows, int n, float eps)
{
    if (w)
        holo_rms_norm_rows(dst, x, w, rows, n, eps);
    else
        HOLO_CHECK(hipMemcpyAsync(dst, x, (size_t)rows * n * sizeof(float), hipMemcpyDeviceToDevice, stream()));
}

bool fused_gemv_type(int t) { return t == HOLO_TYPE_Q4_0 || t == HOLO_TYPE_Q8_0 || t == HOLO_TYPE_Q4_K; }

// The batched product takes the rows: at least 64, not in exact mode, in_dim
// whole blocks of the type (holo_matmul_batch: Q4_0 on its own kernels, the
// other types on a dequantised f16 panel).
bool gemm_rows(int type, int rows, int in_dim, int exact)
{
    if (rows < 64 || exact) return false;
    switch (type) {
    case HOLO_TYPE_Q4_0:
    case HOLO_TYPE_Q8_0:
    case HOLO_TYPE_F16:
    case HOLO_TYPE_F32: return in_dim % 32 == 0;
    case HOLO_TYPE_Q4_K:
    case HOLO_TYPE_Q6_K: return in_dim % 256 == 0;
    default: return false;
    }
}

// q, k, v of n rows of xb.  One GEMM over the three matrices when the rows
// go to the prefill GEMM (one quantisation, one launch); the fused q/k/v GEMV
// per row when the three share a GEMV format; otherwise one call per matrix.
void matmul_qkv(float *q, float *k, float *v, const holo_llama_layer_t &L, const float *xb, int n, int q_dim,
                int kv_dim, int dim, int exact)
{
    const int t = L.wq_type;
    const bool same = L.wk_type == t && L.wv_type == t;
    if (same && gemm_rows(t, n, dim, exact) && q_dim % 128 == 0 && kv_dim % 128 == 0) {
        float *Y[3] = {q, k, v};
        const void *W[3] = {L.wq, L.wk, L.wv};
        const int N[3] = {q_dim, kv_dim, kv_dim};
        holo_matmul_batch_multi(Y, W, N, 3, xb, n, dim, t);
        return;
    }
    if (!same && gemm_rows(t, n, dim, exact) && gemm_rows(L.wk_type, n, dim, exact) &&
        gemm_rows(L.wv_type, n, dim, exact) && q_dim % 128 == 0 && kv_dim % 128 == 0) {
        // mixed types (Q4_K_M: Q6_K v): one launch over the three dequantised panels
        float *Y[3] = {q, k, v};
        const void *W[3] = {L.wq, L.wk, L.wv};
        const int T[3] = {L.wq_type, L.wk_type, L.wv_type};
        const int N[3] = {q_dim, kv_dim, kv_dim};
        holo_matmul_batch_multi_types(Y, W, T, N, 3, xb, n, dim);
        return;
    }
    if (same && fused_gemv_type(t) && !gemm_rows(t, n, dim, exact)) {
        for (int r = 0; r < n; r++)
            holo_batched_qkv(q + (int64_t)r * q_dim, k + (int64_t)r * kv_dim, v + (int64_t)r * kv_dim, L.wq, L.wk, L.wv,
                             xb + (int64_t)r * dim, q_dim, kv_dim, dim, t);
        return;
    }
    holo_matmul_rows(q, L.wq, xb, n, q_dim, dim, L.wq_type, exact);
    holo_matmul_rows(k, L.wk, xb, n, kv_dim, dim, L.wk_type, exact);
    holo_matmul_rows(v, L.wv, xb, n, kv_dim, dim, L.wv_type, exact);
}

// q, k, v of the rows of x RMS-normed by nw, the norm inside the exact
// product's activation halves (one launch for the three matrices); false
// when that route does not take these rows, and nothing ran.
bool qkv_normed(float *q, float *k, float *v, const holo_llama_layer_t &L, const float *x, const float *nw, float eps,
                int n, int q_dim, int kv_dim, int dim, int exact)
{
    if (!nw || !gemm_rows(L.wq_type, n, dim, exact) || !gemm_rows(L.wk_type, n, dim, exact) ||
        !gemm_rows(L.wv_type, n, dim, exact))
        return false;
    float *Y[3] = {q, k, v};
    const void *W[3] = {L.wq, L.wk, L.wv};
    const int T[3] = {L.wq_type, L.wk_type, L.wv_type};
    const int N[3] = {q_dim, kv_dim, kv_dim};
    return exact_product_normed(Y, W, T, N, 3, x, nw, eps, n, dim);
}

// h = silu(W1 xb) * (W3 xb) of n rows (h2: scratch of the same size), by the
// same three routes; the fused GEMV applies silu * in its epilogue.
void matmul_gate_up(float *h, float *h2, const holo_llama_layer_t &L, const float *xb, int n, int ffn, int dim,
                    int exact)
{
    const int t = L.w1_type;
    const bool same = L.w3_type == t;
    if (same && gemm_rows(t, n, dim, exact) && ffn % 128 == 0) {
        float *Y[2] = {h, h2};
        const void *W[2] = {L.w1, L.w3};
        const int N[2] = {ffn, ffn};
        holo_matmul_batch_multi(Y, W, N, 2, xb, n, dim, t);
    } else if (same && fused_gemv_type(t) && !gemm_rows(t, n, dim, exact)) {
        for (int r = 0; r < n; r++)
            holo_batched_ffn_gate_up(h + (int64_t)r * ffn, L.w1, L.w3, xb + (int64_t)r * dim, ffn, dim, t);
        return;
    } else {
        holo_matmul_rows(h, L.w1, xb, n, ffn, dim, L.w1_type, exact);
        holo_matmul_rows(h2, L.w3, xb, n, ffn, dim, L.w3_type, exact);
    }
    cuda_silu_mul(h, h, h2, n * ffn);
}

}  // namespace

extern "C" {

void holo_matmul_rows(float *Y, const void *W, const float *X, int rows, int out_dim, int in_dim, int type,
                      int exact)
{
    if (rows <= 0 || out_dim <= 0) return;
    if (gemm_rows(type, rows, in_dim, exact)) {
        holo_matmul_batch(Y, W, X, rows, out_dim, in_dim, type);
        return;
    }
    for (int r = 0; r < rows; r++)
        holo_matmul(Y + (int64_t)r * out_dim, W, X + (int64_t)r * in_dim, out_dim, in_dim, type);
}

int holo_llama_forward(const holo_llama_t *m, const int *tokens, int n, int pos0, float *logits, int flags)
{
    if (!m || !tokens || !logits || n <= 0 || pos0 < 0 || m->n_layers <= 0 || !m->layers || !m->tok_emb ||
        !m->output || !m->key_cache || !m->value_cache || m->dim <= 0 || m->n_heads <= 0 || m->n_kv_heads <= 0 ||
        m->n_heads % m->n_kv_heads != 0 || m->head_dim <= 0 || m->head_dim > 128 || m->head_dim % 2 ||
        m->ffn_dim <= 0 || m->vocab <= 0 || pos0 + n > m->max_seq || !rows_type_ok(m->out_type) ||
        !(rows_type_ok(m->emb_type) || m->emb_type == HOLO_TYPE_Q4_K)) {
        HOLO_REJECT("holo_llama_forward: model or shape outside the supported set");
        return HOLO_EINVAL;
    }
    for (int l = 0; l < m->n_layers; l++)
        if (!layer_ok(m->layers[l])) {
            HOLO_REJECT("holo_llama_forward: layer with a missing matrix or an unsupported type");
            return HOLO_EINVAL;
        }
    for (int t = 0; t < n; t++)
        if (tokens[t] < 0 || tokens[t] >= m->vocab) {
            HOLO_REJECT("holo_llama_forward: token outside the vocabulary");
            return HOLO_EINVAL;
        }
    const int dim = m->dim, hd = m->head_dim, ffn = m->ffn_dim;
    const int q_dim = m->n_heads * hd, kv_dim = m->n_kv_heads * hd;
    const int exact = flags & HOLO_FORWARD_EXACT;
    const int64_t layer_cache = (int64_t)m->max_seq * kv_dim;

    // stream-ordered scratch: token ids, x, xb, q, att, hb, hb2 (k and v are
    // written straight into the caches)
    const size_t rowsz = (size_t)n * sizeof(float);
    const size_t sz_tok = ((size_t)n * sizeof(int) + 255) & ~(size_t)255;
    const size_t sizes[] = {sz_tok, rowsz * dim, rowsz * dim, rowsz * q_dim, rowsz * q_dim, rowsz * ffn, rowsz * ffn};
    constexpr int kBufs = sizeof(sizes) / sizeof(sizes[0]);
    size_t total = 0;
    for (size_t s : sizes) total += (s + 255) & ~(size_t)255;
    void *ws = nullptr;
    HOLO_CHECK(hipMallocAsync(&ws, total, stream()));
    if (!ws) return HOLO_EINVAL;
    uint8_t *p = (uint8_t *)ws;
    void *bufs[kBufs];
    for (int i = 0; i < kBufs; i++) {
        bufs[i] = p;
        p += (sizes[i] + 255) & ~(size_t)255;
    }
    int *dtok = (int *)bufs[0];
    float *x = (float *)bufs[1], *xb = (float *)bufs[2], *q = (float *)bufs[3], *att = (float *)bufs[4];
    float *hb = (float *)bufs[5], *hb2 = (float *)bufs[6];

    // embeddings: all n rows in one launch
    HOLO_CHECK(hipMemcpyAsync(dtok, tokens, (size_t)n * sizeof(int), hipMemcpyHostToDevice, stream()));
    holo_embedding_rows(x, m->tok_emb, dtok, n, dim, m->emb_type);

    for (int l = 0; l < m->n_layers; l++) {
        const holo_llama_layer_t &L = m->layers[l];
        float *kc = m->key_cache + l * layer_cache, *vc = m->value_cache + l * layer_cache;
        // this call's rows of the caches: the k and v products land there
        // directly ([pos][kv_dim] is their row-major output layout)
        float *k = kc + (int64_t)pos0 * kv_dim, *v = vc + (int64_t)pos0 * kv_dim;
        // One row (a decode step): the norms run inside the q/k/v and gate/up
        // GEMVs and the residual adds inside the o and down GEMVs.
        const bool one = n == 1;
        const bool qkv1 = one && L.attn_norm && fused_gemv_type(L.wq_type) && L.wk_type == L.wq_type &&
                          L.wv_type == L.wq_type;
        const bool ffn1 = one && L.ffn_norm && fused_gemv_type(L.w1_type) && L.w3_type == L.w1_type;
        // attention block
        if (qkv1) {
            holo_batched_qkv_norm(q, k, v, L.wq, L.wk, L.wv, x, L.attn_norm, m->rms_eps, xb, q_dim, kv_dim, dim,
                                  L.wq_type);
        } else if (!qkv_normed(q, k, v, L, x, L.attn_norm, m->rms_eps, n, q_dim, kv_dim, dim, exact)) {
            norm_or_copy(xb, x, L.attn_norm, n, dim, m->rms_eps);
            matmul_qkv(q, k, v, L, xb, n, q_dim, kv_dim, dim, exact);
        }
        holo_rope_rows(q, k, n, pos0, hd, m->n_heads, m->n_kv_heads, m->rope_base);  // k rotated in the cache
        holo_attention_prefill(att, q, kc, vc, n, pos0, hd, m->n_heads, m->n_kv_heads);
        if (one && fused_gemv_type(L.wo_type)) {
            holo_matmul_add(x, L.wo, att, x, dim, q_dim, L.wo_type);
        } else if (gemm_rows(L.wo_type, n, q_dim, exact)) {
            holo_matmul_batch_add(x, L.wo, att, x, n, dim, q_dim, L.wo_type);  // the add in the GEMM's store
        } else {
            holo_matmul_rows(xb, L.wo, att, n, dim, q_dim, L.wo_type, exact);
            cuda_vec_add(x, x, xb, n * dim);
        }
        // FFN block
        if (ffn1) {
            holo_batched_ffn_gate_up_norm(hb, L.w1, L.w3, x, L.ffn_norm, m->rms_eps, xb, ffn, dim, L.w1_type);
        } else {
            if (L.w3_type == L.w1_type && gemm_rows(L.w1_type, n, dim, exact) && ffn % 128 == 0 &&
                gemm_rows(L.w2_type, n, ffn, exact)) {
                // gate and up in one GEMM (the norm in its activation halves
                // when it takes the exact route); the SwiGLU goes into the down
                // GEMM's activation panel and the residual add into its store
                float *Y[2] = {hb, hb2};
                const void *W[2] = {L.w1, L.w3};
                const int N[2] = {ffn, ffn};
                const int T[2] = {L.w1_type, L.w3_type};
                if (!L.ffn_norm || !exact_product_normed(Y, W, T, N, 2, x, L.ffn_norm, m->rms_eps, n, dim)) {
                    norm_or_copy(xb, x, L.ffn_norm, n, dim, m->rms_eps);
                    holo_matmul_batch_multi(Y, W, N, 2, xb, n, dim, L.w1_type);
                }
                holo_matmul_batch_swiglu_add(x, L.w2, hb, hb2, x, n, dim, ffn, L.w2_type);
                continue;
            }
            norm_or_copy(xb, x, L.ffn_norm, n, dim, m->rms_eps);
            matmul_gate_up(hb, hb2, L, xb, n, ffn, dim, exact);
        }
        if (one && fused_gemv_type(L.w2_type)) {
            holo_matmul_add(x, L.w2, hb, x, dim, ffn, L.w2_type);
        } else if (gemm_rows(L.w2_type, n, ffn, exact)) {
            holo_matmul_batch_add(x, L.w2, hb, x, n, dim, ffn, L.w2_type);
        } else {
            holo_matmul_rows(xb, L.w2, hb, n, dim, ffn, L.w2_type, exact);
            cuda_vec_add(x, x, xb, n * dim);
        }
    }
    // the last token: final norm and the output head
    float *xl = x + (int64_t)(n - 1) * dim;
    norm_or_copy(xb, xl, m->out_norm, 1, dim, m->rms_eps);
    holo_matmul(logits, m->output, xb, m->vocab, dim, m->out_type);
    HOLO_CHECK(hipFreeAsync(ws, stream()));
    return 0;
}

// Every layer matrix of m with its shape [out][in]: q, k, v, o, gate, down, up.
static void layer_mats(const holo_llama_t *m, int l, const void *W[7], int T[7], int O[7], int I[7])
{
    const holo_llama_layer_t &L = m->layers[l];
    const int q_dim = m->n_heads * m->head_dim, kv_dim = m->n_kv_heads * m->head_dim, d = m->dim, f = m->ffn_dim;
    const void *w[7] = {L.wq, L.wk, L.wv, L.wo, L.w1, L.w2, L.w3};
    const int t[7] = {L.wq_type, L.wk_type, L.wv_type, L.wo_type, L.w1_type, L.w2_type, L.w3_type};
    const int o[7] = {q_dim, kv_dim, kv_dim, d, f, d, f}, in[7] = {d, d, d, q_dim, d, f, d};
    for (int i = 0; i < 7; i++) {
        W[i] = w[i];
        T[i] = t[i];
        O[i] = o[i];
        I[i] = in[i];
    }
}

int holo_llama_prepare(const holo_llama_t *m)
{
    if (!m || !m->layers || m->n_layers <= 0) {
        HOLO_REJECT("holo_llama_prepare: null model");
        return HOLO_EINVAL;
    }
    for (int l = 0; l < m->n_layers; l++) {
        const void *W[7];
        int T[7], O[7], I[7];
        layer_mats(m, l, W, T, O, I);
        for (int i = 0; i < 7; i++) {
            if (T[i] != HOLO_TYPE_Q6_K || !W[i] || I[i] % 256 != 0 || I[i] > 16384) continue;
            const int rc = holo_prefill_prepare(W[i], O[i], I[i], T[i]);
            if (rc != 0) {
                holo_llama_release(m);
                return rc;
            }
        }
    }
    return 0;
}

void holo_llama_release(const holo_llama_t *m)
{
    if (!m || !m->layers) return;
    for (int l = 0; l < m->n_layers; l++) {
        const void *W[7];
        int T[7], O[7], I[7];
        layer_mats(m, l, W, T, O, I);
        for (int i = 0; i < 7; i++)
            if (T[i] == HOLO_TYPE_Q6_K && W[i]) holo_prefill_release(W[i]);
    }
}

// This forward is the plain Llama body.  The reference also runs Gemma
// (embedding scale, post-norms, a 1M RoPE base on global layers) and Qwen
// (q/k/v biases, QK-norm) variants (llm.c:451-475, 480-485, 516-521,
// 1037-1133); a file that needs one of them is rejected rather than run with
// the wrong arithmetic.
int holo_llama_gguf_check(const holo_gguf_t *g)
{
    if (!g) return -1;
    const holo_gguf_model_t *p = holo_gguf_model(g);
    if (strstr(p->arch, "gemma") || strstr(p->arch, "Gemma")) return -1;
    static const char *const kUnsupported[] = {"attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_q_norm.weight",
                                               "attn_k_norm.weight", "post_attention_norm.weight",
                                               "post_ffw_norm.weight"};
    for (int l = 0; l < (int)p->block_count; l++)
        for (const char *suffix : kUnsupported) {
            const std::string name = "blk." + std::to_string(l) + "." + suffix;
            if (holo_gguf_find_tensor(g, name.c_str())) return -1;
        }
    return 0;
}

int holo_llama_from_gguf(const holo_gguf_t *g, holo_llama_t *m, holo_llama_layer_t *layers, int max_layers)
{
    if (!g || !m || !layers || !holo_gguf_device_base(g)) return -1;
    const holo_gguf_model_t *p = holo_gguf_model(g);
    const int n_layers = (int)p->block_count;
    if (n_layers <= 0 || n_layers > max_layers) return -1;
    if (holo_llama_gguf_check(g) != 0) return -1;
    memset(m, 0, sizeof(*m));
    memset(layers, 0, sizeof(*layers) * (size_t)n_layers);
    auto find = [&](const std::string &name, int *type) -> const void * {
        const holo_gguf_tensor_t *t = holo_gguf_find_tensor(g, name.c_str());
        if (!t) return nullptr;
        if (type) *type = t->type;
        return holo_gguf_device_ptr(g, t);
    };
    m->n_layers = n_layers;
    m->dim = (int)p->embedding_length;
    m->n_heads = (int)p->attention_head_count;
    m->n_kv_heads = (int)p->attention_head_count_kv;
    m->head_dim = (int)p->attention_key_length;
    m->ffn_dim = (int)p->feed_forward_length;
    m->rms_eps = p->rms_norm_eps;
    m->rope_base = p->rope_freq_base;
    const holo_gguf_tensor_t *emb = holo_gguf_find_tensor(g, "token_embd.weight");
    if (!emb) return -1;
    m->tok_emb = holo_gguf_device_ptr(g, emb);
    m->emb_type = emb->type;
    m->vocab = (int)emb->dims[1];  // g_emb_vocab_size (llm.c:368)
    m->out_norm = (const float *)find("output_norm.weight", nullptr);
    m->output = find("output.weight", &m->out_type);
    if (!m->output) {  // tied embeddings (llm.c:387-390)
        m->output = m->tok_emb;
        m->out_type = m->emb_type;
    }
    for (int l = 0; l < n_layers; l++) {
        const std::string b = "blk." + std::to_string(l) + ".";
        holo_llama_layer_t &L = layers[l];
        L.attn_norm = (const float *)find(b + "attn_norm.weight", nullptr);
        L.wq = find(b + "attn_q.weight", &L.wq_type);
        L.wk = find(b + "attn_k.weight", &L.wk_type);
        L.wv = find(b + "attn_v.weight", &L.wv_type);
        L.wo = find(b + "attn_output.weight", &L.wo_type);
        L.ffn_norm = (const float *)find(b + "ffn_norm.weight", nullptr);
        L.w1 = find(b + "ffn_gate.weight", &L.w1_type);
        L.w2 = find(b + "ffn_down.weight", &L.w2_type);
        L.w3 = find(b + "ffn_up.weight", &L.w3_type);
        if (!L.wq || !L.wk || !L.wv || !L.wo || !L.w1 || !L.w2 || !L.w3) return -1;
    }
    m->layers = layers;
    return 0;
}

}  // extern "C"
