/*
 * holo_mi355x.h -- extensions of libholo_mi355x.so beyond the reference's
 * cuda_ops.h.  None of these replaces a reference symbol; each says what in
 * the reference it relates to.  Existing cuda_ops.h signatures are unchanged.
 */
#ifndef HOLO_MI355X_EXT_H
#define HOLO_MI355X_EXT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids of the formats served (reference src/ai/quant.h:19-33). */
#define HOLO_TYPE_F32  0
#define HOLO_TYPE_F16  1
#define HOLO_TYPE_Q4_0 2
#define HOLO_TYPE_Q8_0 8
#define HOLO_TYPE_Q4_K 12
#define HOLO_TYPE_Q6_K 14

/* ---- errors ---------------------------------------------------------------
 * The reference ops return void and print (cuda_ops.cu:21-37).  This library
 * prints too, and latches the first error code until it is read:
 * 0 = ok, otherwise a hipError_t value, or HOLO_EINVAL for a rejected
 * argument.  holo_last_error() returns and clears the latch.               */
#define HOLO_EINVAL 100001
#define HOLO_ECHAIN 100002  /* a persistent decode-step launch could not synchronise */
int holo_last_error(void);
const char *holo_error_string(int code);

/* ---- stream, events, graphs ----------------------------------------------
 * All ops launch on one library stream (default: the null stream, as the
 * reference).  Events are recorded on that stream.  A graph captures every
 * op issued between begin and end on that stream (stream capture), so a
 * decode step of many GEMVs replays with one launch.                        */
void holo_set_stream(void *hip_stream);
void *holo_get_stream(void);
void *holo_event_create(void);
void holo_event_record(void *ev);
float holo_event_elapsed_ms(void *start, void *stop); /* synchronises on stop */
void holo_event_destroy(void *ev);
void *holo_stream_create(void);                 /* default priority */
void holo_stream_destroy(void *s);
int holo_graph_begin(void);                     /* library stream must not be the null stream */
void *holo_graph_end(void);                     /* returns an executable graph or NULL */
int holo_graph_launch(void *graph_exec);
void holo_graph_destroy(void *graph_exec);

/* ---- generic dispatch -------------------------------------------------------
 * The reference's gpu_matmul switch (src/ai/llm_cuda.c:140-163) as one call. */
void holo_matmul(float *dst, const void *M, const float *v, int out_dim, int in_dim, int type);

/* ---- GEMV activation mode ------------------------------------------------------
 * All modes hold the dot products to fp32 accuracy and accumulate across
 * blocks in fp32.
 * HOLO_XMODE_MFMA (default): activations are held per 32-block as 22-bit
 * fixed point, xi = rint(x * 63*65536/amax), |x - d*xi| <= amax*2^-23, in
 * three int8 planes, and each block's three exact integer dots run on the
 * int8 matrix cores (v_mfma_i32_16x16x64_i8).  Taken for Q4_0, Q4_K and Q8_0
 * rows with in_dim a multiple of 256 up to 16384 and 16-byte aligned
 * matrices; other shapes run HOLO_XMODE_F32.
 * HOLO_XMODE_F32: every weight is multiplied by the fp32 activation itself
 * (v_cvt_f32_ubyte + FMA).
 * HOLO_XMODE_I24: the MFMA mode's arithmetic on v_dot4_i32_i8.
 * Rows longer than the LDS staging holds (in_dim > 14880 for F32) switch to
 * I24, and beyond 18880 to fp32 read from global memory.  Applies to every
 * GEMV entry point.                                                        */
#define HOLO_XMODE_F32 0
#define HOLO_XMODE_I24 1
#define HOLO_XMODE_MFMA 2      /* default: MFMA for Q4_0, Q4_K and Q8_0      */
#define HOLO_XMODE_MFMA_ALL 3  /* the same as HOLO_XMODE_MFMA                */
/* MFMA for Q4_0 and Q4_K, Q8_0 rows up to 8192 on the F32 kernel (the
 * former default; 4096x4096 Q8_0: 6.2 against 5.9 us on MFMA)              */
#define HOLO_XMODE_MFMA_Q8F32 4
void holo_gemv_set_xmode(int xmode);
/* Launch shape of the GEMV kernels: rows per work item (1, 2 or 4; 0 = the
 * default, 1; F32/I24 modes only) and workgroups per CU (0 = the default:
 * F32/I24 use 1 when the grid has at most 2 tiles per CU, else 2; MFMA
 * uses 1 or 2 by how evenly the rows fill its tiles).  A tuning knob.      */
void holo_gemv_set_launch(int rows_per_item, int wg_per_cu);
/* ---- a decode step's GEMV stages in one persistent launch ---------------------
 * A plan of dependent GEMV stages (every layer's q/k/v, o, gate/up and down of a
 * decode step), run by holo_gemv_stream_launch as ONE kernel launch.  Each
 * stage is the GEMV of cuda_matmul_<type> over 1-3 matrices sharing x
 * (gate_up = 0: y[m] = W[m] x), or the fused gate/up (gate_up = 1: y[0] =
 * silu(W[0] x) * (W[1] x)); with norm_w its input is rms_norm(x) * norm_w
 * (cuda_rms_norm's formula, eps), and with r (one plain matrix) its output is
 * y[0] = r + W x (r may alias y[0]).  A stage may read an earlier stage's
 * output as x or r, when it names that output's address exactly; outputs hand
 * over to later stages through exchange words (value and a launch/stage tag
 * in one 64-bit store) that the consumers poll, not a grid barrier, and the
 * first later stage that reads an output as x (its in_dim = the output's
 * rows, all of the producing stage's matrices with rows a multiple of 16)
 * receives it as plane records: the reader's int8 activation planes, made by
 * the producer.  Every stage output has exchange buffers of its own, so a
 * later stage may rewrite a vector that earlier stages still read.  Rejected:
 * an input overlapping an earlier output other than exactly, or reading past
 * the rows its last writer stored; an output overlapping its own stage's x or
 * another output.  The
 * activations are 22-bit fixed point per 16 values (the separate GEMV calls:
 * per 32), so results match the separate MFMA-path calls to about 1e-6
 * normwise per stage and the CPU reference within the 1e-3 bar.  The weight
 * loads of later stages are issued ahead, across the stage boundaries.  Q4_0
 * or Q4_K (HOLO_TYPE_*), in_dim a multiple of 256 up to 18432 (and within the
 * 160 KB of LDS), 16-byte aligned matrices, vectors and norm weights, at most
 * 16 tiles of 16 rows per CU and stage.  An output row that a later stage
 * writes again is stored in plain fp32 only by the last one (the final
 * contents are those of running the stages in order).  No reference
 * counterpart: it replaces the per-matrix launches of the decode loop
 * (src/ai/llm_cuda.c:604-918).
 * create: copies the stage table to the device and allocates the exchange
 *   buffers (not under graph capture); NULL, with the error latched, for
 *   anything outside the set.
 * launch: one launch on the library stream (capturable); 0 or HOLO_EINVAL.
 *   Launches of one plan must not overlap (they share its exchange buffers).
 * status: HOLO_ECHAIN (and clears it) if a launch's exchange wait gave up
 *   (bounded at ~0.3 s; the results of that launch are then wrong), else 0. */
typedef struct {
    const void *W[3];
    float *y[3];
    int rows[3];
    int nmat;            /* matrices of a plain stage: 1..3 */
    int gate_up;         /* 1: W[0] = gate, W[1] = up, output y[0] */
    const float *x;
    int in_dim;
    const float *norm_w; /* NULL, or the stage multiplies rms_norm(x) * norm_w */
    float eps;
    const float *r;      /* NULL, or y[0] = r + W x (one plain matrix) */
} holo_stream_stage_t;
void *holo_gemv_stream_create(const holo_stream_stage_t *stages, int nstages, int type);
int holo_gemv_stream_launch(void *plan);
void holo_gemv_stream_destroy(void *plan);
int holo_gemv_stream_status(void);

/* Times one kernel: the next launch of the MFMA GEMV path or of the prefill
 * GEMM kernel (holo_gemm_q4_0_q8_0) records start_event
 * when its first wave starts and stop_event when its last wave ends
 * (hipExtLaunchKernelGGL), so the events span the kernel alone, without the
 * dispatch latency an event pair around the call includes.  One launch only;
 * a launch that takes another path leaves the request pending.              */
void holo_time_next_launch(void *start_event, void *stop_event);

/* ---- dequantisation ---------------------------------------------------------
 * dst[n] = the fp32 weights of n/QK blocks, bit-identical to the reference
 * CPU routines dequantize_row_q8_0 / q4_0 / q4_k / q6_k
 * (src/ai/quant.c:118-128, 136-153, 277-311, 241-271).                     */
void holo_dequant(float *dst, const void *src, int64_t n, int type);
/* dst[n] (f16) = f16_rne of the same values, for Q8_0 / Q4_0 / Q4_K / Q6_K
 * blocks, and of F32 (16-byte aligned) and F16 (copied) rows: the weight panel
 * of the batched f16 product.  dst 16-byte aligned, src 4-byte aligned (F32:
 * 16, F16: 2), n a multiple of 32.
 * No reference counterpart (the reference dequantises to fp32 only).       */
void holo_dequant_f16(void *dst, const void *src, int64_t n, int type);

/* ---- fused multi-GEMV for every served format --------------------------------
 * Same contract as cuda_batched_qkv_q8_0 / cuda_batched_ffn_gate_up_q8_0
 * (reference cuda_ops.h:60-66) for type Q8_0, Q4_0 or Q4_K.                */
void holo_batched_qkv(float *q_out, float *k_out, float *v_out,
                      const void *Wq, const void *Wk, const void *Wv,
                      const float *x, int q_dim, int kv_dim, int in_dim, int type);
void holo_batched_ffn_gate_up(float *out, const void *W1, const void *W3,
                              const float *x, int ffn_dim, int in_dim, int type);

/* ---- decode-layer fusions (no reference counterpart) ------------------------
 * The reference's decode layer runs rms_norm before q/k/v and gate/up and a
 * residual add after o and down, each its own launch (llm_cuda.c:598-880).
 * These fold them into the GEMVs:
 *   holo_batched_qkv_norm / holo_batched_ffn_gate_up_norm: the product of
 *     rms_norm(x) * norm_w (as cuda_rms_norm with eps) -- the norm is applied
 *     in the GEMV's activation staging for Q4_0/Q4_K with in_dim <= 8192 and a
 *     16-byte-aligned norm_w; otherwise cuda_rms_norm writes xb (in_dim
 *     floats, required then; NULL allowed when the fused path applies) and
 *     the plain fused GEMV runs on it.
 *   holo_matmul_add: y = r + W.v, the add in the GEMV's output store; y may
 *     alias r (in place) for Q8_0, Q4_0 and Q4_K.                          */
void holo_batched_qkv_norm(float *q_out, float *k_out, float *v_out,
                           const void *Wq, const void *Wk, const void *Wv,
                           const float *x, const float *norm_w, float eps, float *xb,
                           int q_dim, int kv_dim, int in_dim, int type);
void holo_batched_ffn_gate_up_norm(float *out, const void *W1, const void *W3,
                                   const float *x, const float *norm_w, float eps, float *xb,
                                   int ffn_dim, int in_dim, int type);
void holo_matmul_add(float *y, const void *M, const float *v, const float *r,
                     int out_dim, int in_dim, int type);

/* ---- batched prefill --------------------------------------------------------
 * The reference has no batched path (one GEMV per prompt token,
 * src/ai/llm.c:1049).  Activations X[M][K] fp32 are quantised per row and
 * 32-block to Q8_0: d = f16_rne(amax/127), q = round-half-away(x*127/amax)
 * (d=0 -> q=0).  Y[M][N] accumulates, over blocks b in order,
 *   acc = fmaf((float)I_b, f16(dw)*f16(dx), acc)
 * with the exact integer block dot I_b (the scale product is exact in fp32).
 * holo_gemm_q4_0_q8_0 stages the activations as f16 in a workspace of
 * M*K*2 + M*(K/32)*2 bytes: a device buffer the library keeps and grows
 * outside graph capture, a stream-ordered allocation under capture.       */
void holo_quantize_act_q8_0(void *dst_blocks, const float *X, int rows, int k);
void holo_gemm_q4_0_q8_0(float *Y, const void *W, const void *Xq, int M, int N, int K);
/* The same product with no allocation anywhere in the call: no hipMalloc,
 * hipFree or allocating library routine.  No counterpart in the reference;
 * it is for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  The activation
 * panel (M*K*2 + M*K/16 bytes, rounded up to 256) is staged in a fixed
 * 24 MiB device array that the library holds on each device until the
 * process ends, so M*K*33/16 must fit in 24 MiB (M = 512 takes K up to
 * 23,831: every config-4 shape); larger calls are rejected (HOLO_EINVAL,
 * nothing launched).  Returns 0 or HOLO_EINVAL.  The array keeps the last
 * call's contents and every call on a device shares it: calls that overlap
 * on one device (issued on two streams) race.                              */
int holo_gemm_q4_0_q8_0_noalloc(float *Y, const void *W, const void *Xq, int M, int N, int K);
/* The matrix cores the Q8_0 product above (and its multi, no-allocation and
 * Q8_0-mode batched forms) runs on, with the same specification and bits:
 * HOLO_Q8_KERNEL_F16 (the default: the integers as f16 on
 * v_mfma_f32_32x32x16_f16) or HOLO_Q8_KERNEL_I8 (v_mfma_i32_32x32x32_i8 for
 * each block's integer dot, the -8 of the weights in the accumulator input,
 * then acc = fmaf((float)I, s, acc); slower, kept for comparison).  The int8
 * kernel takes K/32 even, 4-byte aligned matrices and, with several
 * matrices, every N but the last a multiple of 64; other calls run the f16
 * kernel.  No reference counterpart.                                       */
#define HOLO_Q8_KERNEL_F16 0
#define HOLO_Q8_KERNEL_I8 1
void holo_prefill_set_q8_kernel(int kind);
int holo_prefill_get_q8_kernel(void);
/* Y[M][N] = X[M][K] . W[N][K]^T for W in Q4_0.  M >= 64 runs, by the mode
 * set below: the exact product (HOLO_PREFILL_EXACT, the default: each row of
 * X scaled by a power of two and split into two f16 halves, x - xh - xl
 * within 2^-22 |x|, times the block's integers, exact in f16, on the f16
 * matrix cores, block scales applied in fp32 in block order; fp32 accuracy,
 * within 1e-3 of the CPU path; X 16-byte aligned and K <= 16384, else M
 * GEMVs; the K blocks of each row of tiles are dealt evenly to about two
 * workgroups per CU, and a tile whose blocks two or more workgroups share
 * is the sum of their parts in K order, so the result depends on the
 * launch's shape and the CU count but not on timing), the f16 product below
 * (HOLO_PREFILL_F16) or the Q8_0
 * product above (HOLO_PREFILL_Q8_0: X quantised to Q8_0).  M < 64 runs M
 * GEMVs.                                                                     */
void holo_matmul_batch_q4_0(float *Y, const void *W, const float *X, int M, int N, int K,
                            void *scratch_q8);
/* The same over nmat = 1..3 Q4_0 matrices that multiply the same X in one
 * launch, sharing one quantisation and one staged panel (for example q/k/v,
 * or gate and up): Y[i][M][N[i]] = X . W[i]^T.  With more than one matrix
 * every N[i] must be a multiple of 128.  Each output is bit-identical to the
 * single-matrix call.  No reference counterpart (the reference multiplies one
 * matrix by one token at a time, llm.c:1049); the batched analogue of
 * holo_batched_qkv / holo_batched_ffn_gate_up.                              */
void holo_gemm_q4_0_q8_0_multi(float *const *Y, const void *const *W, const int *N, int nmat,
                               const void *Xq, int M, int K);
/* The f16 product: no activation quantisation.  x16 = f16_rne(x), w16 =
 * f16_rne(f16(dw) * (q - 8)), Y = sum_k x16 * w16 accumulated in fp32 on the
 * matrix cores (order of the hardware: within the fp32 accumulation bound of
 * the float64 sum of the rounded operands, not bit-reproducible on the CPU).
 * X[M][K] fp32, 16-byte aligned, K a multiple of 32; a workspace of M*K*2
 * bytes, as above.  No reference counterpart (build-defined, like
 * the Q8_0 product).                                                       */
void holo_gemm_q4_0_f16(float *Y, const void *W, const float *X, int M, int N, int K);
void holo_gemm_q4_0_f16_multi(float *const *Y, const void *const *W, const int *N, int nmat,
                              const float *X, int M, int K);
/* Which product every batched matmul (holo_matmul_batch*, the prompt
 * forward) runs for M >= 64: HOLO_PREFILL_EXACT (default), HOLO_PREFILL_F16
 * (Q4_0: the f16 product; other types: their f16 weight panel) or
 * HOLO_PREFILL_Q8_0 (Q4_0 only: the Q8_0 product; other types as F16).    */
/* The prompt layer's residual products (no reference counterpart; the batched
 * analogue of holo_matmul_add): Y = R + X . W^T, and Y = R + (silu(G) * U) .
 * W^T with silu(g) * u as cuda_silu_mul computes it -- the add in the
 * GEMM's output store, the SwiGLU in its f16 activation panel.  Y may alias
 * R.  M < 64 runs GEMVs; outside the f16 product (Q8_0 mode, misaligned G/U,
 * M < 64) the SwiGLU is stored into G first, so G's contents are not kept. */
void holo_matmul_batch_q4_0_add(float *Y, const void *W, const float *X, const float *R, int M, int N, int K);
void holo_matmul_batch_q4_0_swiglu_add(float *Y, const void *W, float *G, const float *U, const float *R,
                                       int M, int N, int K);
#define HOLO_PREFILL_F16 0
#define HOLO_PREFILL_Q8_0 1
#define HOLO_PREFILL_EXACT 2
void holo_prefill_set_mode(int mode);
int holo_prefill_get_mode(void);
void holo_matmul_batch_q4_0_multi(float *const *Y, const void *const *W, const int *N, int nmat,
                                  const float *X, int M, int K, void *scratch_q8);
/* The batched products for any weight type the GEMVs serve (Q4_0, Q8_0, Q4_K,
 * Q6_K, F16, F32), with the contracts of the Q4_0 calls above.  Q4_0 goes to
 * them.  Every other type, for M >= 64 and K whole blocks (Q4_K, Q6_K: K a
 * multiple of 256) up to 16384, runs the exact product by default (the block
 * integers against the two f16 halves of X, block scales in fp32); in
 * HOLO_PREFILL_F16 mode it is dequantised into an f16 panel
 * (holo_dequant_f16, N*K*2 bytes per matrix) and multiplied on the f16
 * product.  Workspaces live in device buffers the library keeps and grows
 * (hipMalloc, outside graph capture; under capture a stream-ordered
 * allocation per call); calls on one stream reuse them in order.  Otherwise
 * one holo_matmul GEMV per row.  The multi forms take up to 3 matrices
 * sharing X (with several, every N a multiple of 128); an output equals the
 * single call's bit for bit when neither launch shares a tile's K blocks
 * between workgroups (for Q4_0, Q8_0, Q4_K, Q6_K and F16 that is when the K
 * blocks per row of tiles split evenly into whole tiles per workgroup; Q6_K
 * matrices are first repacked into the workspace), else it is
 * within the product's error bound.  No reference counterpart (the
 * reference runs one GEMV per token,
 * llm.c:1049).                                                              */
void holo_matmul_batch(float *Y, const void *W, const float *X, int M, int N, int K, int type);
void holo_matmul_batch_multi(float *const *Y, const void *const *W, const int *N, int nmat, const float *X,
                             int M, int K, int type);
/* The multi form with a type per matrix (q/k/v of a Q4_K_M file: Q4_K, Q4_K,
 * Q6_K); one type throughout is holo_matmul_batch_multi.  In the exact
 * product (the default) the matrices share one activation split and run one
 * launch per weight type (Q4_K q and k together, Q6_K v on its own); in
 * HOLO_PREFILL_F16 mode they share one activation panel and one launch,
 * every weight matrix dequantised to its f16 panel (Q4_0 too, to the same
 * f16 values its own kernel unpacks).                                       */
void holo_matmul_batch_multi_types(float *const *Y, const void *const *W, const int *types, const int *N, int nmat,
                                   const float *X, int M, int K);
void holo_matmul_batch_add(float *Y, const void *W, const float *X, const float *R, int M, int N, int K, int type);
void holo_matmul_batch_swiglu_add(float *Y, const void *W, float *G, const float *U, const float *R, int M, int N,
                                  int K, int type);
/* Q6_K matrices repacked once instead of per call (no reference counterpart;
 * the load-time step of this library's own exact product).  The exact
 * product reads Q6_K through a layout of its own (1 byte per weight, the
 * superblocks' bits rearranged), which every batched call otherwise builds
 * in its workspace first.  holo_prefill_prepare allocates that copy of W
 * [N][K] (N*K bytes, hipMalloc), writes it, waits for it, and keeps it until
 * holo_prefill_release(W): every later exact batched product on W with the
 * same N and K reads the copy, with the same bits as the per-call form.  W
 * must not change and must not be freed while registered, and a graph
 * captured while W was registered reads the copy: destroy such graphs
 * before releasing W.  Returns 0 (also
 * for a W already registered with this shape), or HOLO_EINVAL (not Q6_K, K
 * not a multiple of 256 up to 16384, W not 2-byte aligned, N*K >= 2^31, a W
 * registered with another shape, or under graph capture), or the hipError_t
 * of the allocation.  Release of an unregistered W does nothing; release
 * waits for the library stream.  cuda_cleanup releases every copy.         */
int holo_prefill_prepare(const void *W, int N, int K, int type);
void holo_prefill_release(const void *W);

#ifdef __cplusplus
}
#endif

#endif /* HOLO_MI355X_EXT_H */
