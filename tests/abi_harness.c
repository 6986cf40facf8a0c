/* abi_harness.c -- a C caller of libholo_mi355x.so through include/cuda_ops.h
 * only, with the call sequence of the reference's GPU decode loop
 * (src/ai/llm_cuda.c:604-918: gpu_matmul -> cuda_matmul_q4_0 for each of the
 * seven layer matrices, cuda_rms_norm, cuda_silu_mul, cuda_vec_add, then the
 * loop's cudaDeviceSynchronize and a blocking cuda_memcpy_d2h).  No Python and
 * no extension header in the loop: it shows that a C engine drives the
 * drop-in boundary as the reference does.
 *
 * The step is the Llama decode dataflow at position 0 (RoPE is the identity
 * and attention over the one cached position returns v):
 *   xb = rms(x) * w_att; q = Wq xb; k = Wk xb; v = Wv xb; x += Wo v;
 *   xb = rms(x) * w_ffn; h = silu(W1 xb) * (W3 xb); x += W2 h
 *
 * usage: holo_abi_harness DIR
 *   DIR/meta.txt          "dim ffn layers"
 *   DIR/x.bin             dim fp32, the input vector
 *   DIR/norm.bin          2 * layers * dim fp32: w_att, w_ffn of each layer
 *   DIR/L<l>_<name>.bin   Q4_0 blocks of layer l, name in q k v o gate up down
 * writes DIR/out.bin (dim fp32, x after the layers) and DIR/h.bin (ffn fp32,
 * the last layer's h).  Exit status 0, or 1 with a message on stderr. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "cuda_ops.h"

static void *read_file(const char *dir, const char *name, size_t want)
{
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "abi_harness: cannot open %s\n", path);
        exit(1);
    }
    void *buf = malloc(want);
    if (!buf || fread(buf, 1, want, f) != want) {
        fprintf(stderr, "abi_harness: %s is shorter than %zu bytes\n", path, want);
        exit(1);
    }
    fclose(f);
    return buf;
}

static void write_file(const char *dir, const char *name, const void *buf, size_t n)
{
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(buf, 1, n, f) != n) {
        fprintf(stderr, "abi_harness: cannot write %s\n", path);
        exit(1);
    }
    fclose(f);
}

/* a device copy of a host buffer, as llm_cuda.c uploads tensors
 * (cuda_malloc + cuda_memcpy_h2d) */
static void *upload(const void *host, size_t n)
{
    void *d = cuda_malloc(n);
    if (!d) {
        fprintf(stderr, "abi_harness: cuda_malloc(%zu) failed\n", n);
        exit(1);
    }
    cuda_memcpy_h2d(d, host, n);
    return d;
}

int main(int argc, char **argv)
{
    if (argc != 2) {
        fprintf(stderr, "usage: %s DIR\n", argv[0]);
        return 1;
    }
    const char *dir = argv[1];
    int dim = 0, ffn = 0, layers = 0;
    {
        char path[4096];
        snprintf(path, sizeof path, "%s/meta.txt", dir);
        FILE *f = fopen(path, "r");
        if (!f || fscanf(f, "%d %d %d", &dim, &ffn, &layers) != 3 || dim <= 0 || ffn <= 0 || layers <= 0 ||
            dim % 32 || ffn % 32) {
            fprintf(stderr, "abi_harness: bad %s\n", path);
            return 1;
        }
        fclose(f);
    }
    if (cuda_init() != 0) {
        fprintf(stderr, "abi_harness: cuda_init failed\n");
        return 1;
    }
    static const char *names[7] = {"q", "k", "v", "o", "gate", "up", "down"};
    const size_t row_dim = (size_t)dim / 32 * 18, row_ffn = (size_t)ffn / 32 * 18;
    const size_t bytes[7] = {dim * row_dim, dim * row_dim, dim * row_dim, dim * row_dim,
                             ffn * row_dim, ffn * row_dim, dim * row_ffn};
    void **W = calloc((size_t)layers * 7, sizeof(void *));
    for (int l = 0; l < layers; l++)
        for (int m = 0; m < 7; m++) {
            char name[64];
            snprintf(name, sizeof name, "L%d_%s.bin", l, names[m]);
            void *h = read_file(dir, name, bytes[m]);
            W[7 * l + m] = upload(h, bytes[m]);
            free(h);
        }
    float *hx = read_file(dir, "x.bin", sizeof(float) * dim);
    float *hn = read_file(dir, "norm.bin", sizeof(float) * 2 * layers * dim);
    float *x = upload(hx, sizeof(float) * dim);
    float *nw = upload(hn, sizeof(float) * 2 * layers * dim);
    float *xb = cuda_malloc(sizeof(float) * dim), *q = cuda_malloc(sizeof(float) * dim);
    float *k = cuda_malloc(sizeof(float) * dim), *v = cuda_malloc(sizeof(float) * dim);
    float *o = cuda_malloc(sizeof(float) * dim), *g = cuda_malloc(sizeof(float) * ffn);
    float *u = cuda_malloc(sizeof(float) * ffn), *h = cuda_malloc(sizeof(float) * ffn);
    if (!xb || !q || !k || !v || !o || !g || !u || !h) {
        fprintf(stderr, "abi_harness: cuda_malloc failed\n");
        return 1;
    }
    for (int l = 0; l < layers; l++) {
        void **L = W + 7 * l;
        cuda_rms_norm(xb, x, nw + (size_t)2 * l * dim, dim, 1e-5f);
        cuda_matmul_q4_0(q, L[0], xb, dim, dim);
        cuda_matmul_q4_0(k, L[1], xb, dim, dim);
        cuda_matmul_q4_0(v, L[2], xb, dim, dim);
        cuda_matmul_q4_0(o, L[3], v, dim, dim); /* attention at position 0 returns v */
        cuda_vec_add(x, x, o, dim);
        cuda_rms_norm(xb, x, nw + (size_t)(2 * l + 1) * dim, dim, 1e-5f);
        cuda_matmul_q4_0(g, L[4], xb, ffn, dim);
        cuda_matmul_q4_0(u, L[5], xb, ffn, dim);
        cuda_silu_mul(h, g, u, ffn);
        cuda_matmul_q4_0(o, L[6], h, dim, ffn);
        cuda_vec_add(x, x, o, dim);
    }
    cuda_sync(); /* the decode loop's cudaDeviceSynchronize (llm_cuda.c:922) */
    float *out = malloc(sizeof(float) * dim), *hh = malloc(sizeof(float) * ffn);
    cuda_memcpy_d2h(out, x, sizeof(float) * dim); /* blocking, as llm_cuda.c:926 */
    cuda_memcpy_d2h(hh, h, sizeof(float) * ffn);
    write_file(dir, "out.bin", out, sizeof(float) * dim);
    write_file(dir, "h.bin", hh, sizeof(float) * ffn);
    for (int i = 0; i < 7 * layers; i++) cuda_free(W[i]);
    cuda_free(x);
    cuda_free(nw);
    cuda_free(xb);
    cuda_free(q);
    cuda_free(k);
    cuda_free(v);
    cuda_free(o);
    cuda_free(g);
    cuda_free(u);
    cuda_free(h);
    cuda_cleanup();
    free(W);
    free(hx);
    free(hn);
    free(out);
    free(hh);
    return 0;
}
