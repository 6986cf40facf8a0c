/*
 * ref_forward.c -- TEST INFRASTRUCTURE.  Runs the reference's own CPU
 * forward on a GGUF file: llm_load (src/ai/llm.c:617) then llm_forward over
 * the tokens (llm.c:1015), and hands back the logits after the last token and
 * the KV caches.  Compiled by oracle/Makefile together with the reference
 * sources, where they lie, into oracle/_ref/libholo_ref_forward.so; loaded
 * only by tests/ (and tests/golden/ to write fixtures), as the checker of the
 * prompt forward.
 */
#include <string.h>

#include "llm.h"

/* Returns 0 and fills logits[0..n_logits) and, when not NULL, the first
 * cache_floats floats of the key and value caches ([layer][max_seq][kv_dim]);
 * *max_seq receives the caches' position count.  -1 if the file does not
 * load or the forward fails.                                                */
int ref_forward(const char *path, const int *tokens, int n, float *logits, int n_logits, float *key_cache,
                float *value_cache, long cache_floats, int *max_seq)
{
    llm_ctx_t *ctx = llm_load(path);
    if (!ctx) return -1;
    int rc = llm_forward(ctx, tokens, n);
    if (rc == 0) {
        if (n_logits > ctx->config.vocab_size) n_logits = ctx->config.vocab_size;
        memcpy(logits, ctx->state.logits, (size_t)n_logits * sizeof(float));
        const llm_kv_cache_t *kv = &ctx->kv_cache;
        long total = (long)kv->n_layers * kv->max_seq_len * kv->n_kv_heads * kv->head_dim;
        long c = cache_floats < total ? cache_floats : total;
        if (key_cache) memcpy(key_cache, kv->key_cache, (size_t)c * sizeof(float));
        if (value_cache) memcpy(value_cache, kv->value_cache, (size_t)c * sizeof(float));
        if (max_seq) *max_seq = kv->max_seq_len;
    }
    llm_free(ctx);
    return rc;
}
