// prefill.hip -- batched prefill product over Q4_0 weights: activations are
// quantised per row and 32-block to Q8_0, and the block dots run on the f16
// matrix cores (v_mfma_f32_32x32x16_f16), where every operand is a small
// integer and every block dot is therefore exact.
//
// The reference has no batched path (its prompt loop is one GEMV per token,
// src/ai/llm.c:1049) and no activation quantiser; this is the build's own
// specification, restated on the CPU in oracle/holo_oracle.c
// (oracle_quantize_act_q8_0, oracle_gemm_q4_0_q8_0):
//   quantise  d = f16_rne(amax/127), id = 1/(amax/127) (0 if amax = 0),
//             q = clamp(roundf(x*id), -127, 127)
//   product   Y[m][n]: acc = fmaf((float)I[m,n,b], f16(dw[n,b]) * f16(dx[m,b]), acc)
//             over blocks b in order, I = sum_k (qw-8)*qx exact
// Every rounding is specified, so the GPU result is bit-identical to the
// CPU restatement (no contraction in this file: the one fused multiply-add
// is written as fmaf).
//
// The f16 product (the default of holo_matmul_batch_q4_0) keeps the
// activations instead of quantising them, and dequantises the weights as
// they are staged:
//   x16 = f16_rne(x),  w16 = f16_rne(f16(dw) * (q - 8)),
//   Y[m][n] = sum_k x16 * w16, accumulated in fp32 on the matrix cores
// (restated in float64 by oracle_gemm_q4_0_f16; the GPU is held to the fp32
// accumulation bound).  No per-block rescale is left, so each 32-block costs
// two MFMAs per tile and no VALU, and both operands keep 11 significant bits
// where the Q8_0 activations keep 8.
#include "common.h"
#include "quant_blocks.h"

#include <hip/hip_ext.h>
#include <limits.h>
#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

#pragma clang fp contract(off)

namespace holo {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

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

// ---- activation panel: Q8_0 blocks -> f16 values + f16 scale bits ------------
// P[m][k] = (f16)qx (exact, |qx| <= 127), D[m][b] = the block's d bits.  Block
// g = m*nb + b lands at P + 32*g, so P is the row-major [M][K] matrix.

__global__ __launch_bounds__(256) void q8_panel_k(uint4 *__restrict__ P, uint16_t *__restrict__ D,
                                                  const uint8_t *__restrict__ Xq, int64_t nblocks, int64_t total)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    const Q8_0Unit u = load_q8_0(Xq, g, total);
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int8_t lo = (int8_t)(u.q[i] >> (16 * j)), hi = (int8_t)(u.q[i] >> (16 * j + 8));
            const h2 v = {(_Float16)lo, (_Float16)hi};
            w[2 * i + j] = __builtin_bit_cast(uint32_t, v);
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) P[g * 4 + j] = make_uint4(w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]);
    D[g] = (uint16_t)u.dh;
}

// ---- f16 activation panel: P[m][k] = f16_rne(X[m][k]), 8 values per thread ----

__global__ __launch_bounds__(256) void x16_panel_k(uint4 *__restrict__ P, const float *__restrict__ X, int64_t n8)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n8) return;
    const float4 a = ((const float4 *)X)[2 * g], b = ((const float4 *)X)[2 * g + 1];
    const h2 v0 = {(_Float16)a.x, (_Float16)a.y}, v1 = {(_Float16)a.z, (_Float16)a.w};
    const h2 v2 = {(_Float16)b.x, (_Float16)b.y}, v3 = {(_Float16)b.z, (_Float16)b.w};
    P[g] = make_uint4(__builtin_bit_cast(uint32_t, v0), __builtin_bit_cast(uint32_t, v1),
                      __builtin_bit_cast(uint32_t, v2), __builtin_bit_cast(uint32_t, v3));
}

// The same from the SwiGLU of two activation matrices: P = f16_rne(silu(g) * u)
// with silu(g) * u as cuda_silu_mul computes it (cuda_ops.cu:304-314).

__global__ __launch_bounds__(256) void x16_swiglu_panel_k(uint4 *__restrict__ P, const float *__restrict__ G,
                                                          const float *__restrict__ U, int64_t n8)
{
    int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n8) return;
    float v[8], u[8];
    *(float4 *)&v[0] = ((const float4 *)G)[2 * g];
    *(float4 *)&v[4] = ((const float4 *)G)[2 * g + 1];
    *(float4 *)&u[0] = ((const float4 *)U)[2 * g];
    *(float4 *)&u[4] = ((const float4 *)U)[2 * g + 1];
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const float a = (v[2 * j] / (1.0f + expf(-v[2 * j]))) * u[2 * j];
        const float b = (v[2 * j + 1] / (1.0f + expf(-v[2 * j + 1]))) * u[2 * j + 1];
        const h2 h = {(_Float16)a, (_Float16)b};
        o[j] = __builtin_bit_cast(uint32_t, h);
    }
    P[g] = make_uint4(o[0], o[1], o[2], o[3]);
}

// ---- GEMM ------------------------------------------------------------------------
// Workgroup: 4 waves in a 2 x 2 grid, each wave owning WM x WN tiles of
// 32 x 32 outputs; the workgroup tile is TM = 64*WM rows (activations) by
// TN = 64*WN columns (weights).  K advances in stages of S blocks; a stage
// is staged in LDS as f16 rows (activations copied from the panel, weights
// unpacked to q-8) plus the f16 scale bits, double-buffered, so one barrier
// per stage separates the writes of stage s+1 from the reads of stage s-1.
// The next stage's global loads are issued before the current stage's
// products and land in registers.
//
// v_mfma_f32_32x32x16_f16 (wave64): lane l supplies A[l%32][8*(l/32)+t] and
// B[8*(l/32)+t][l%32], t = 0..7; D[i][j] lands in lane j + 32*((i/4)%2),
// register (i%4) + 4*(i/8).  Per block and tile: two instructions give the
// exact block dot I (k = 0..15, 16..31; integer partial sums < 2^24), and a
// third, whose only non-zero operands are A[i][0] = dx[i] and B[0][j] = dw[j],
// gives s[i][j] = dx[i]*dw[j] exactly in the same register layout, leaving
// one VALU instruction (the fmaf) per output and block.

// Up to three weight matrices share one launch and one activation panel:
// matrix i holds columns [n_end[i-1], n_end[i]) of the concatenated product
// and writes its own Y[i] ([M][N_i]).  Every column tile lies in one matrix
// (the host checks N_i % TN == 0 when there are several).
constexpr int kPrefillMats = 3;

struct PrefillArgs {
    float *Y[kPrefillMats];
    const uint8_t *W[kPrefillMats];  // Q4_0 [N_i][nb]
    int n_end[kPrefillMats];         // prefix sums of N_i; unused entries INT_MAX
    const _Float16 *P;               // f16 [M][K]
    const uint16_t *D;               // f16 bits [M][nb]
    int M, N, nb;                    // N: all matrices' columns
    int ntm, tiles;                  // row tiles, all tiles
    const float *R;                  // one matrix only: Y = R + product (R [M][N], may be Y)
};

// The matrix of a column tile, its first column and its width.
struct PrefillMat {
    const uint8_t *W;
    float *Y;
    int nbase, N;
    int64_t w_bytes;
};

// WGM x WGN waves per workgroup (4 or 8), each owning WM x WN 32x32 tiles.
template <int WM, int WN, int S, int WGM = 2, int WGN = 2>
struct PGeo {
    static constexpr int NT = 64 * WGM * WGN;  // threads
    static constexpr int TM = 32 * WM * WGM, TN = 32 * WN * WGN;
    static constexpr int ROW = 32 * S + 8;  // f16 per LDS row; the 16-byte pad spreads rows over the banks
    static constexpr int A_OFF = 0;
    static constexpr int B_OFF = A_OFF + TM * ROW * 2;
    static constexpr int AD_OFF = B_OFF + TN * ROW * 2;
    static constexpr int BD_OFF = AD_OFF + ((TM * S * 2 + 15) & ~15);
    static constexpr int STAGE = BD_OFF + ((TN * S * 2 + 15) & ~15);
    static constexpr int LDS = 2 * STAGE;
    static constexpr int NA = TM * S * 4 / NT;         // 16-byte activation pieces per thread
    static constexpr int ND = (TM * S + NT - 1) / NT;  // activation scales per thread
    static constexpr int NB = (TN * S + NT - 1) / NT;  // weight blocks per thread
    static constexpr int NWP = TN * S * 4 / NT;        // 16-byte weight-panel pieces per thread
    static_assert((TM * S * 4) % NT == 0, "activation pieces must split evenly over the threads");
    static_assert((TN * S * 4) % NT == 0, "weight-panel pieces must split evenly over the threads");
};

// f16 (q - 8) of the eight nibbles of x = qs[4j..4j+3]: lo[0..1] hold k = 4j..4j+3
// (low nibbles), hi[0..1] k = 16+4j..16+4j+3 (high nibbles).  v_perm pairs a
// nibble byte with 0x64, giving the f16 value 1024 + q; subtracting 1032 is
// exact.
__device__ __forceinline__ void nib_f16(uint32_t x, uint32_t lo[2], uint32_t hi[2])
{
    const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const uint32_t t0 = x & 0x0F0F0F0Fu, t1 = (x >> 4) & 0x0F0F0F0Fu;
    const uint32_t c64 = 0x64646464u;
    lo[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(c64, t0, 0x04010400u)) + off);
    lo[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(c64, t0, 0x04030402u)) + off);
    hi[0] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(c64, t1, 0x04010400u)) + off);
    hi[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(c64, t1, 0x04030402u)) + off);
}

// Per-thread load addresses of a tile, computed once: each piece's row (and
// its column within a block) at block 0, and its block within the stage.  A
// stage's fetch then only adds the block offset (clamped to the last block).
// Rows past the last row or column re-read the last one (in bounds, never used).
template <int WM, int WN, int S, bool XF16, int WGM = 2, int WGN = 2, bool WP = false>
struct PAddr {
    using G = PGeo<WM, WN, S, WGM, WGN>;
    static constexpr int NWI = WP ? G::NWP : G::NB;
    const uint8_t *pa[G::NA];            // activation piece i: its row, column (c % 4) * 8
    int ka[G::NA];                       // its block within the stage
    const uint16_t *pd[XF16 ? 1 : G::ND];  // activation scales: the row of scale i
    int kd[XF16 ? 1 : G::ND];
    int64_t ow[NWI];                     // weights: byte offset of the piece's row (+ column) at block 0
    int kw[NWI];

    __device__ __forceinline__ PAddr(const PrefillArgs &a, const PrefillMat &w, int tid, int m0, int n0)
    {
        const int nb = a.nb;
        const int64_t K = (int64_t)nb * 32;
#pragma unroll
        for (int i = 0; i < G::NA; i++) {
            const int p = tid + G::NT * i, r = p / (4 * S), c = p % (4 * S);
            pa[i] = (const uint8_t *)(a.P + (int64_t)min(m0 + r, a.M - 1) * K + (c % 4) * 8);
            ka[i] = c / 4;
        }
        if constexpr (!XF16) {
#pragma unroll
            for (int i = 0; i < G::ND; i++) {
                const int v = min(tid + G::NT * i, G::TM * S - 1);
                pd[i] = a.D + (int64_t)min(m0 + v / S, a.M - 1) * nb;
                kd[i] = v % S;
            }
        }
#pragma unroll
        for (int i = 0; i < NWI; i++) {
            if constexpr (WP) {
                const int p = tid + G::NT * i, n = p / (4 * S), c = p % (4 * S);
                ow[i] = (int64_t)min(n0 + n, w.N - 1) * K * 2 + (c % 4) * 16;
                kw[i] = c / 4;
            } else {
                const int v = min(tid + G::NT * i, G::TN * S - 1);
                ow[i] = (int64_t)min(n0 + v / S, w.N - 1) * nb * 18;
                kw[i] = v % S;
            }
        }
    }
};

// Registers of one stage in flight between its global loads and its LDS
// writes: blocks kb0 .. kb0+S-1 of the workgroup's rows and columns; block
// indices past the row's last block read the last block again (in bounds,
// never used).
// XF16: f16 activations without scales, weights dequantised to f16 as they
// are staged (the f16 product); otherwise the Q8_0 product.  WP (with XF16):
// the weights are an f16 panel [N][K] already (any block format, dequantised
// by holo_dequant_f16), fetched and staged as the activations are.
template <int WM, int WN, int S, bool XF16, int WGM = 2, int WGN = 2, bool WP = false>
struct PStage {
    using G = PGeo<WM, WN, S, WGM, WGN>;
    static_assert(!WP || XF16, "a weight panel needs f16 activations");
    v4u ra[G::NA];
    uint16_t rd[G::ND];  // as loaded: a widening here would wait for the load
    Q4_0Raw rb[WP ? 1 : G::NB];
    v4u rw[WP ? G::NWP : 1];

    __device__ __forceinline__ void fetch(const PrefillArgs &a, const PrefillMat &w,
                                          const PAddr<WM, WN, S, XF16, WGM, WGN, WP> &ad, int kb0)
    {
        const int nb = a.nb;
#pragma unroll
        for (int i = 0; i < G::NA; i++)
            ra[i] = *(const v4u *)(ad.pa[i] + (int64_t)min(kb0 + ad.ka[i], nb - 1) * 64);
        if constexpr (!XF16) {
#pragma unroll
            for (int i = 0; i < G::ND; i++) rd[i] = ad.pd[i][min(kb0 + ad.kd[i], nb - 1)];
        }
        if constexpr (WP) {
#pragma unroll
            for (int i = 0; i < G::NWP; i++)
                rw[i] = *(const v4u *)((const uint8_t *)w.W + ad.ow[i] + (int64_t)min(kb0 + ad.kw[i], nb - 1) * 64);
            return;
        }
#pragma unroll
        for (int i = 0; i < G::NB; i++)
            rb[i] = load_q4_0_raw(w.W, ad.ow[i] + (int64_t)min(kb0 + ad.kw[i], nb - 1) * 18, w.w_bytes);
    }

    // registers -> one LDS stage buffer (weights unpacked to f16 q-8)
    __device__ __forceinline__ void stash(uint8_t *base, int tid) const
    {
#pragma unroll
        for (int i = 0; i < G::NA; i++) {
            const int p = tid + G::NT * i, r = p / (4 * S), c = p % (4 * S);
            *(v4u *)(base + G::A_OFF + (r * G::ROW + c * 8) * 2) = ra[i];
        }
        if constexpr (!XF16) {
#pragma unroll
            for (int i = 0; i < G::ND; i++) {
                const int v = tid + G::NT * i;
                if (v < G::TM * S) ((uint16_t *)(base + G::AD_OFF))[v] = rd[i];
            }
        }
        if constexpr (WP) {
            // the same k order as the unpacked blocks below: row n, k = 8c .. 8c + 7
#pragma unroll
            for (int i = 0; i < G::NWP; i++) {
                const int p = tid + G::NT * i, n = p / (4 * S), c = p % (4 * S);
                *(v4u *)(base + G::B_OFF + (n * G::ROW + c * 8) * 2) = rw[i];
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < G::NB; i++) {
            const int v = tid + G::NT * i, n = v / S, s = v % S;
            if (v < G::TN * S) {
                const Q4_0Unit u = q4_0_unit(rb[i]);
                uint32_t lo[8], hi[8];
#pragma unroll
                for (int j = 0; j < 4; j++) nib_f16(u.q[j], &lo[2 * j], &hi[2 * j]);
                if constexpr (XF16) {
                    // w16 = f16_rne(dw * (q - 8)): one packed f16 multiply per pair
                    const _Float16 dw = __builtin_bit_cast(_Float16, (uint16_t)u.dh);
                    const h2 d2 = {dw, dw};
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        lo[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, lo[j]) * d2);
                        hi[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, hi[j]) * d2);
                    }
                }
                v4u *dst = (v4u *)(base + G::B_OFF + (n * G::ROW + s * 32) * 2);
                dst[0] = v4u{lo[0], lo[1], lo[2], lo[3]};  // k = 0..7
                dst[1] = v4u{lo[4], lo[5], lo[6], lo[7]};  // k = 8..15
                dst[2] = v4u{hi[0], hi[1], hi[2], hi[3]};  // k = 16..23
                dst[3] = v4u{hi[4], hi[5], hi[6], hi[7]};  // k = 24..31
                if constexpr (!XF16) ((uint16_t *)(base + G::BD_OFF))[v] = (uint16_t)u.dh;
            }
        }
    }
};

// D: stages of global loads in flight (1 or 2); OCC: workgroups per CU the
// register allocation is bounded for.
template <int WM, int WN, int S, int D, int OCC, bool XF16, int WGM = 2, int WGN = 2, bool WP = false>
__global__ __launch_bounds__(64 * WGM * WGN, OCC) void gemm_q4_0_f16_k(PrefillArgs a)
{
    using G = PGeo<WM, WN, S, WGM, WGN>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, c32 = lane & 31;

    // Tile of this workgroup.  Workgroups go to the 8 XCDs round-robin; when
    // the tile count allows, XCD x takes a contiguous run of tiles, so the
    // row tiles sharing a weight tile share that XCD's L2.
    const int g = blockIdx.x;
    const int t = (a.tiles & 7) ? g : (g & 7) * (a.tiles >> 3) + (g >> 3);
    const int m0 = (t % a.ntm) * G::TM, ng = (t / a.ntm) * G::TN;
    // the tile's matrix (constant indices into the argument arrays: selects)
    const int sel = (ng >= a.n_end[0]) + (ng >= a.n_end[1]);
    PrefillMat w;
    w.W = sel == 2 ? a.W[2] : sel == 1 ? a.W[1] : a.W[0];
    w.Y = sel == 2 ? a.Y[2] : sel == 1 ? a.Y[1] : a.Y[0];
    w.nbase = sel == 2 ? a.n_end[1] : sel == 1 ? a.n_end[0] : 0;
    w.N = (sel == 2 ? a.n_end[2] : sel == 1 ? a.n_end[1] : a.n_end[0]) - w.nbase;
    w.w_bytes = (int64_t)w.N * a.nb * 18;
    const int n0 = ng - w.nbase;
    const int wm0 = (wave / WGN) * 32 * WM, wn0 = (wave % WGN) * 32 * WN;
    const int nb = a.nb;
    const int nst = (nb + S - 1) / S;
    v16f acc[WM][WN];
#pragma unroll
    for (int mi = 0; mi < WM; mi++)
#pragma unroll
        for (int ni = 0; ni < WN; ni++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;

    // Scale operands of v_mfma_f32_32x32x8_f16 (lane l supplies A[l%32][4*(l/32)+t],
    // B[4*(l/32)+t][l%32], t = 0..3): the f16 scale in element 0 of lanes 0..31,
    // zero everywhere else, so the product is the single term dx[i]*dw[j].
    v2u as[WM], bs[WN];
#pragma unroll
    for (int mi = 0; mi < WM; mi++) as[mi] = v2u{0u, 0u};
#pragma unroll
    for (int ni = 0; ni < WN; ni++) bs[ni] = v2u{0u, 0u};

    auto compute = [&](int buf, int kb0) {
        const uint8_t *base = lds + buf * G::STAGE;
        const _Float16 *lA = (const _Float16 *)(base + G::A_OFF);
        const _Float16 *lB = (const _Float16 *)(base + G::B_OFF);
        const uint16_t *lAd = (const uint16_t *)(base + G::AD_OFF);
        const uint16_t *lBd = (const uint16_t *)(base + G::BD_OFF);
        const v16f zero = {};
#pragma unroll
        for (int s = 0; s < S; s++) {
            if (kb0 + s >= nb) break;
            v8h a0[WM], a1[WM], b0[WN], b1[WN];
#pragma unroll
            for (int mi = 0; mi < WM; mi++) {
                const int r = wm0 + 32 * mi + c32;
                const _Float16 *pa = lA + r * G::ROW + s * 32 + 8 * h;
                a0[mi] = *(const v8h *)pa;
                a1[mi] = *(const v8h *)(pa + 16);
                if constexpr (!XF16) as[mi].x = h ? 0u : (uint32_t)lAd[r * S + s];
            }
#pragma unroll
            for (int ni = 0; ni < WN; ni++) {
                const int n = wn0 + 32 * ni + c32;
                const _Float16 *pb = lB + n * G::ROW + s * 32 + 8 * h;
                b0[ni] = *(const v8h *)pb;
                b1[ni] = *(const v8h *)(pb + 16);
                if constexpr (!XF16) bs[ni].x = h ? 0u : (uint32_t)lBd[n * S + s];
            }
#pragma unroll
            for (int mi = 0; mi < WM; mi++)
#pragma unroll
                for (int ni = 0; ni < WN; ni++) {
                    if constexpr (XF16) {
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0[mi], b0[ni], acc[mi][ni], 0, 0, 0);
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[mi], b1[ni], acc[mi][ni], 0, 0, 0);
                        continue;
                    }
                    v16f I = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0[mi], b0[ni], zero, 0, 0, 0);
                    I = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[mi], b1[ni], I, 0, 0, 0);
                    const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(__builtin_bit_cast(v4h, as[mi]),
                                                                         __builtin_bit_cast(v4h, bs[ni]), zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[mi][ni][r] = __builtin_fmaf(I[r], sc[r], acc[mi][ni][r]);
                }
        }
    };

    // Ring of D register stages: set d holds stage k with k % D == d.
    // Stages past the last block re-read the last one (fetch clamps every
    // index) and compute skips their blocks, so every slot issues the same
    // loads and the loop has one exit, at its latch, with a trip count known
    // up front: the compiler's wait before each stash is then exactly that
    // stage's own loads (a conditional fetch made it wait for every load in
    // flight, the other set's too).
    const PAddr<WM, WN, S, XF16, WGM, WGN, WP> ad(a, w, tid, m0, n0);
    PStage<WM, WN, S, XF16, WGM, WGN, WP> st[D];
#pragma unroll
    for (int d = 0; d < D; d++) st[d].fetch(a, w, ad, d * S);
    st[0].stash(lds, tid);
    st[0].fetch(a, w, ad, D * S);
    __syncthreads();
    const int rounds = (nst + D - 1) / D;
    for (int q = 0; q < rounds; q++) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int k = q * D + d;
            compute(k & 1, k * S);
            // stage k + 1 (register set (d + 1) % D) into the other buffer,
            // then that set fetches stage k + 1 + D
            st[(d + 1) % D].stash(lds + ((k + 1) & 1) * G::STAGE, tid);
            st[(d + 1) % D].fetch(a, w, ad, (k + 1 + D) * S);
            __syncthreads();
        }
    }

#pragma unroll
    for (int mi = 0; mi < WM; mi++)
#pragma unroll
        for (int ni = 0; ni < WN; ni++) {
            const int n = n0 + wn0 + 32 * ni + c32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + wm0 + 32 * mi + (r & 3) + 4 * h + 8 * (r >> 2);
                if (m < a.M && n < w.N) {
                    const int64_t o = (int64_t)m * w.N + n;
                    w.Y[o] = a.R ? a.R[o] + acc[mi][ni][r] : acc[mi][ni][r];
                }
            }
        }
}

// Tile per problem: the 128 x 128 workgroup tile (64 x 64 per wave) reads
// the least LDS per product and is used when it yields at least one tile per
// CU; otherwise the 64 x 64 tile gives four times the workgroups.
static int prefill_tn(int M, int N)
{
    const int cus = num_cus() > 0 ? num_cus() : 256;
    const long tiles128 = (long)((M + 127) / 128) * ((N + 127) / 128);
    return tiles128 >= cus ? 128 : 64;
}

template <int WM, int WN, int S, int D, int OCC, bool XF16, int WGM = 2, int WGN = 2, bool WP = false>
static void launch_prefill(PrefillArgs a)
{
    using G = PGeo<WM, WN, S, WGM, WGN>;
    a.ntm = (a.M + G::TM - 1) / G::TM;
    a.tiles = a.ntm * ((a.N + G::TN - 1) / G::TN);
    auto kern = gemm_q4_0_f16_k<WM, WN, S, D, OCC, XF16, WGM, WGN, WP>;
    static bool attr = false;
    if (!attr) {
        HOLO_CHECK(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS));
        attr = true;
    }
    hipEvent_t e0, e1;
    if (take_launch_events(&e0, &e1))
        hipExtLaunchKernelGGL(kern, dim3(a.tiles), dim3(G::NT), G::LDS, stream(), e0, e1, 0, a);
    else
        hipLaunchKernelGGL(kern, dim3(a.tiles), dim3(G::NT), G::LDS, stream(), a);
    HOLO_LAUNCH_CHECK();
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

}  // extern "C"

// Workspaces of the batched products: slot 0 holds the weight panels
// (gemm_panel), slot 1 the activation panel (gemm_multi).  Each is one device
// buffer kept by the library and grown (outside graph capture) to the largest
// request, reused in stream order by every call.  Per-call stream-ordered
// allocations of these sizes (tens to hundreds of MB, interleaved) made single
// prompts stall for up to 15 ms while the pool mapped memory.  Under graph
// capture, or when growing fails, the call allocates stream-ordered instead.  Calls
// that overlap on different streams would share a buffer: the library issues
// on one stream.
static void *g_ws[3] = {nullptr, nullptr, nullptr};
static size_t g_ws_bytes[3] = {0, 0, 0};

namespace holo {
void *workspace(int slot, size_t bytes)
{
    // never under capture: a graph must not hold a buffer a later growth frees
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream(), &st) != hipSuccess || st != hipStreamCaptureStatusNone) return nullptr;
    if (bytes <= g_ws_bytes[slot]) return g_ws[slot];
    HOLO_CHECK(hipStreamSynchronize(stream()));  // earlier calls may still use the old buffer
    if (g_ws[slot]) HOLO_CHECK(hipFree(g_ws[slot]));
    g_ws[slot] = nullptr;
    g_ws_bytes[slot] = 0;
    if (hipMalloc(&g_ws[slot], bytes) != hipSuccess) {
        (void)hipGetLastError();
        g_ws[slot] = nullptr;
        return nullptr;
    }
    g_ws_bytes[slot] = bytes;
    return g_ws[slot];
}
}  // namespace holo

// One launch over nmat matrices (holo_gemm_q4_0_q8_0 and its multi-matrix form).
// Xq (Q8_0 blocks): the Q8_0 product; otherwise X (fp32, 16-byte aligned):
// the f16 product, of silu(X) * U when U is given.  R: Y = R + product (one
// matrix).  wp: W[i] are f16 panels [N_i][K] (f16 product only), otherwise
// Q4_0 block streams.
// Bytes of the activation panel (and, for the Q8_0 product, its scale
// array) that gemm_multi stages M x K activations into.
static size_t act_panel_bytes(int M, int K, bool xf16)
{
    const int64_t nblk = (int64_t)M * (K / 32);
    return (size_t)nblk * 64 + (xf16 ? 0 : (((size_t)nblk * 2 + 255) & ~(size_t)255));
}

// Which matrix cores the Q8_0 product runs on (holo_prefill_set_q8_kernel):
// f16 by default, measured faster (config 4: 125 / 131 us against 185 / 285 us
// on int8, whose extra convert per output and block adds to the epilogue that
// bounds this specification).
static int g_q8_kernel = HOLO_Q8_KERNEL_F16;

// ws_given: a caller-provided workspace of at least act_panel_bytes bytes
// (nothing is allocated); otherwise the library's kept workspace.
static void gemm_multi(float *const *Y, const void *const *W, const int *N, int nmat, const void *Xq, const float *X,
                       int M, int K, const float *U = nullptr, const float *R = nullptr, bool wp = false,
                       void *ws_given = nullptr)
{
    const bool xf16 = Xq == nullptr;
    const int nb = K / 32;
    const int64_t nblk = (int64_t)M * nb;
    int ntot = 0;
    for (int i = 0; i < nmat; i++) ntot += N[i];
    const size_t pbytes = (size_t)nblk * 64, dbytes = act_panel_bytes(M, K, xf16) - pbytes;
    void *ws = ws_given ? ws_given : workspace(1, pbytes + dbytes);
    const bool own = ws == nullptr;
    if (own) HOLO_CHECK(hipMallocAsync(&ws, pbytes + dbytes, stream()));
    if (!ws) return;
    // the Q8_0 product on the int8 matrix cores (its panel fits the f16 one's space)
    if (!xf16 && !R && g_q8_kernel == HOLO_Q8_KERNEL_I8 && q8i8_fits(W, N, nmat, M, K)) {
        q8i8_product(Y, W, N, nmat, Xq, M, K, ws);
        if (own) HOLO_CHECK(hipFreeAsync(ws, stream()));
        return;
    }
    uint4 *P = (uint4 *)ws;
    uint16_t *D = xf16 ? nullptr : (uint16_t *)((uint8_t *)ws + pbytes);
    if (xf16) {
        const int64_t n8 = nblk * 4;
        if (U)
            hipLaunchKernelGGL(x16_swiglu_panel_k, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream(), P, X,
                               U, n8);
        else
            hipLaunchKernelGGL(x16_panel_k, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, stream(), P, X, n8);
    } else {
        hipLaunchKernelGGL(q8_panel_k, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, stream(), P, D,
                           (const uint8_t *)Xq, nblk, nblk * 34);
    }
    HOLO_LAUNCH_CHECK();
    PrefillArgs a = {};
    int acc = 0;
    for (int i = 0; i < kPrefillMats; i++) {
        if (i < nmat) {
            acc += N[i];
            a.Y[i] = Y[i];
            a.W[i] = (const uint8_t *)W[i];
            a.n_end[i] = acc;
        } else {
            a.Y[i] = Y[0];
            a.W[i] = (const uint8_t *)W[0];
            a.n_end[i] = INT_MAX;
        }
    }
    a.P = (const _Float16 *)P;
    a.D = D;
    a.M = M;
    a.N = ntot;
    a.nb = nb;
    a.R = nmat == 1 ? R : nullptr;
    // Variant per shape (measured at the prompt-forward shapes, M = 512):
    // 128 x 128 tiles with 2-block stages when there are at least as many
    // such tiles as CUs (q/k/v, gate/up), with two stages of loads in flight
    // for the f16 product (95 and 181 us; gate/up, two tiles per CU and more,
    // on 8 waves of 64 x 32: 166 us) and one for the Q8_0 product, whose extra
    // scale registers leave no room for a second (137 and 254 us);
    // otherwise 64 x 64 tiles, 4-block stages, two in flight (o, down: f16
    // 47 and 113 us, Q8_0 58 and 142 us, against 90 and 223 us on the 128 x 64
    // tile).  HOLO_PREFILL_CFG=<tile rows>,<tile columns>,<stage blocks>,
    // <stages in flight>,<waves per EU>[,<waves per workgroup>] selects one
    // of the compiled variants (128,128,2,1,2  128,128,2,2,2 (f16 only)
    // 128,128,2,2,2,8  128,64,2,2,2  64,64,4,1,2  64,64,4,2,2) instead.
    static int cfg = -1;
    if (cfg < 0) {
        const char *e = getenv("HOLO_PREFILL_CFG");
        int tm = 0, tn = 0, st = 0, d = 0, o = 0, w = 4;
        const int got = e ? sscanf(e, "%d,%d,%d,%d,%d,%d", &tm, &tn, &st, &d, &o, &w) : 0;
        cfg = got >= 5 ? (w == 8 ? 100000 : 0) + (tm / 64) * 10000 + (tn / 64) * 1000 + st * 100 + d * 10 + o : 0;
    }
    auto go = [&](auto xfc, auto wpc) {
        constexpr bool XF = decltype(xfc)::value, WP = decltype(wpc)::value;
        static_assert(!WP || XF, "a weight panel needs the f16 product");
        const int tiles128 = ((M + 127) / 128) * ((ntot + 127) / 128);
        const int def = prefill_tn(M, ntot) != 128 ? 11422
                        : !XF                       ? 22212
                        : tiles128 >= 2 * num_cus() ? 122222
                                                    : 22222;
        switch (cfg ? cfg : def) {
        case 21222: launch_prefill<2, 1, 2, 2, 2, XF, 2, 2, WP>(a); break;
        case 122222: launch_prefill<2, 1, 2, 2, 2, XF, 2, 4, WP>(a); break;
        case 11412: launch_prefill<1, 1, 4, 1, 2, XF, 2, 2, WP>(a); break;
        case 11422: launch_prefill<1, 1, 4, 2, 2, XF, 2, 2, WP>(a); break;
        case 22222:  // the Q8_0 product has no registers for a second stage: one
            if constexpr (XF) launch_prefill<2, 2, 2, 2, 2, true, 2, 2, WP>(a);
            else launch_prefill<2, 2, 2, 1, 2, false>(a);
            break;
        default: launch_prefill<2, 2, 2, 1, 2, XF, 2, 2, WP>(a); break;
        }
    };
    if (wp) go(std::true_type{}, std::true_type{});
    else if (xf16) go(std::true_type{}, std::false_type{});
    else go(std::false_type{}, std::false_type{});
    if (own) HOLO_CHECK(hipFreeAsync(ws, stream()));
}

// Several matrices in one launch: each N_i a multiple of 128 (a column tile
// never straddles two matrices), at most three.
static bool multi_fits(const int *N, int nmat)
{
    if (nmat < 1 || nmat > kPrefillMats) return false;
    if (nmat == 1) return N[0] > 0;
    for (int i = 0; i < nmat; i++)
        if (N[i] <= 0 || N[i] % 128) return false;
    return true;
}

static bool gemm_args_ok(const void *Xq, int K)
{
    if (!Xq || K % 32 != 0 || K <= 0 || (((uintptr_t)Xq) & 3u)) {
        HOLO_REJECT("holo_gemm_q4_0_q8_0_multi: Xq null or not 4-byte aligned, or K not a positive multiple of 32");
        return false;
    }
    return true;
}

// ---- the allocation-free variant of holo_gemm_q4_0_q8_0 ---------------------------
//
// Its activation panel lives in `scratch`, a file-scope device array of
// kNoAllocScratchBytes that every device the library runs on holds from
// module load until the process ends.  In host code `scratch` names a
// host-side stand-in, not device memory: its device address is taken once
// per device with hipGetSymbolAddress (cuda_init for device 0, or the entry
// point's first call on another device) and only that address is used.
// Every call on one device shares the array, and the last call's contents
// stay there: the panel kernel overwrites every byte a call reads, so nothing
// needs clearing; calls that overlap on one device (two streams) race.
constexpr size_t kNoAllocScratchBytes = (size_t)24 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
constexpr int kMaxDevices = 64;
static void *g_scratch_dev[kMaxDevices];

namespace holo {
// The device address of `scratch` on the current device, looked up once per
// device; nullptr if the lookup fails.
void *noalloc_scratch()
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    if (!g_scratch_dev[dev]) {
        void *ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            latch_error((int)e, "hipGetSymbolAddress(scratch)", __FILE__, __LINE__);
            return nullptr;
        }
        g_scratch_dev[dev] = ptr;
    }
    return g_scratch_dev[dev];
}
}  // namespace holo

extern "C" {

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
    gemm_multi(&Y, &W, &N, 1, Xq, nullptr, M, K);
}

int holo_gemm_q4_0_q8_0_noalloc(float *Y, const void *W, const void *Xq, int M, int N, int K)
{
    if (M <= 0 || N <= 0) return 0;
    if (!Y || !W || !Xq || K % 32 != 0 || K <= 0) {
        HOLO_REJECT("holo_gemm_q4_0_q8_0_noalloc: null pointer or K not a positive multiple of 32");
        return HOLO_EINVAL;
    }
    if ((((uintptr_t)W) & 3u) || (((uintptr_t)Xq) & 3u)) {
        HOLO_REJECT("holo_gemm_q4_0_q8_0_noalloc: W and Xq must be 4-byte aligned");
        return HOLO_EINVAL;
    }
    if (act_panel_bytes(M, K, false) > kNoAllocScratchBytes) {
        HOLO_REJECT("holo_gemm_q4_0_q8_0_noalloc: M*K too large for the fixed scratch (M*K*33/16 bytes must fit "
                    "in 24 MiB)");
        return HOLO_EINVAL;
    }
    void *ws = noalloc_scratch();
    if (!ws) return HOLO_EINVAL;
    gemm_multi(&Y, &W, &N, 1, Xq, nullptr, M, K, nullptr, nullptr, false, ws);
    return 0;
}

void holo_gemm_q4_0_q8_0_multi(float *const *Y, const void *const *W, const int *N, int nmat, const void *Xq, int M,
                               int K)
{
    if (M <= 0) return;
    if (!Y || !W || !N || !multi_fits(N, nmat)) {
        HOLO_REJECT("holo_gemm_q4_0_q8_0_multi: null array, or not 1..3 matrices whose N are multiples of 128");
        return;
    }
    for (int i = 0; i < nmat; i++)
        if (!Y[i] || !W[i] || (((uintptr_t)W[i]) & 3u)) {
            HOLO_REJECT("holo_gemm_q4_0_q8_0_multi: null or misaligned matrix or output");
            return;
        }
    if (!gemm_args_ok(Xq, K)) return;
    gemm_multi(Y, W, N, nmat, Xq, nullptr, M, K);
}

void holo_gemm_q4_0_f16_multi(float *const *Y, const void *const *W, const int *N, int nmat, const float *X, int M,
                              int K)
{
    if (M <= 0) return;
    if (!Y || !W || !N || !multi_fits(N, nmat)) {
        HOLO_REJECT("holo_gemm_q4_0_f16_multi: null array, or not 1..3 matrices whose N are multiples of 128");
        return;
    }
    for (int i = 0; i < nmat; i++)
        if (!Y[i] || !W[i] || (((uintptr_t)W[i]) & 3u)) {
            HOLO_REJECT("holo_gemm_q4_0_f16_multi: null or misaligned matrix or output");
            return;
        }
    if (!X || ((uintptr_t)X & 15u) || K % 32 != 0 || K <= 0) {
        HOLO_REJECT("holo_gemm_q4_0_f16_multi: X null or not 16-byte aligned, or K not a positive multiple of 32");
        return;
    }
    gemm_multi(Y, W, N, nmat, nullptr, X, M, K);
}

void holo_gemm_q4_0_f16(float *Y, const void *W, const float *X, int M, int N, int K)
{
    if (M <= 0 || N <= 0) return;
    holo_gemm_q4_0_f16_multi(&Y, &W, &N, 1, X, M, K);
}

static int g_prefill_mode = HOLO_PREFILL_EXACT;

void holo_prefill_set_mode(int mode)
{
    if (mode != HOLO_PREFILL_F16 && mode != HOLO_PREFILL_Q8_0 && mode != HOLO_PREFILL_EXACT) {
        HOLO_REJECT("holo_prefill_set_mode: HOLO_PREFILL_EXACT, HOLO_PREFILL_F16 or HOLO_PREFILL_Q8_0");
        return;
    }
    g_prefill_mode = mode;
}

}  // extern "C"

// Exact mode (the default): the exact product (prefill_exact.hip) when every
// operand fits it; otherwise the callers run fp32-activation GEMVs per row,
// never a lower-precision product.
static bool exact_fits(const void *const *W, const int *types, int nmat, const float *X, const float *U, int M, int K)
{
    // the product addresses each activation half (M*K f16) with 32-bit byte offsets
    if (!X || ((uintptr_t)X & 15u) || ((uintptr_t)U & 15u) || (int64_t)M * K > (1LL << 30)) return false;
    for (int i = 0; i < nmat; i++)
        if (!W[i] || !exact_ok(types[i], K, W[i])) return false;
    return true;
}

static bool exact_mode() { return g_prefill_mode == HOLO_PREFILL_EXACT; }

extern "C" {

void holo_prefill_set_q8_kernel(int kind)
{
    if (kind != HOLO_Q8_KERNEL_F16 && kind != HOLO_Q8_KERNEL_I8) {
        HOLO_REJECT("holo_prefill_set_q8_kernel: HOLO_Q8_KERNEL_F16 or HOLO_Q8_KERNEL_I8");
        return;
    }
    g_q8_kernel = kind;
}

int holo_prefill_get_q8_kernel(void) { return g_q8_kernel; }

}  // extern "C"

namespace holo {

bool exact_product_normed(float *const *Y, const void *const *W, const int *types, const int *N, int nmat,
                          const float *X, const float *NW, float eps, int M, int K)
{
    if (M < 64 || !exact_mode() || !Y || !W || !types || !N || !NW || ((uintptr_t)NW & 15u) || K > 1024 * 16 ||
        !multi_fits(N, nmat) || !exact_fits(W, types, nmat, X, nullptr, M, K))
        return false;
    for (int i = 0; i < nmat; i++)
        if (!Y[i]) return false;
    exact_product(Y, W, types, N, nmat, X, nullptr, nullptr, M, K, NW, eps);
    return true;
}

}  // namespace holo

extern "C" {

int holo_prefill_get_mode(void) { return g_prefill_mode; }

void holo_matmul_batch_q4_0(float *Y, const void *W, const float *X, int M, int N, int K, void *scratch_q8)
{
    if (M <= 0 || N <= 0) return;
    const int t = HOLO_TYPE_Q4_0;
    if (M >= 64 && exact_mode() && exact_fits(&W, &t, 1, X, nullptr, M, K)) {
        exact_product(&Y, &W, &t, &N, 1, X, nullptr, nullptr, M, K);
        return;
    }
    if (M < 64 || exact_mode()) {
        for (int m = 0; m < M; m++) cuda_matmul_q4_0(Y + (int64_t)m * N, W, X + (int64_t)m * K, N, K);
        return;
    }
    if (g_prefill_mode == HOLO_PREFILL_F16 && !((uintptr_t)X & 15u) && K % 32 == 0) {
        holo_gemm_q4_0_f16(Y, W, X, M, N, K);
        return;
    }
    void *q = scratch_q8;
    if (!q) HOLO_CHECK(hipMallocAsync(&q, (size_t)M * (K / 32) * 34, stream()));
    if (!q) return;
    holo_quantize_act_q8_0(q, X, M, K);
    holo_gemm_q4_0_q8_0(Y, W, q, M, N, K);
    if (!scratch_q8) HOLO_CHECK(hipFreeAsync(q, stream()));
}

void holo_matmul_batch_q4_0_add(float *Y, const void *W, const float *X, const float *R, int M, int N, int K)
{
    if (M <= 0 || N <= 0) return;
    if (!Y || !W || !X || !R || K % 32 != 0 || K <= 0) {
        HOLO_REJECT("holo_matmul_batch_q4_0_add: null pointer or K not a positive multiple of 32");
        return;
    }
    const int t = HOLO_TYPE_Q4_0;
    if (M >= 64 && exact_mode() && exact_fits(&W, &t, 1, X, nullptr, M, K)) {
        exact_product(&Y, &W, &t, &N, 1, X, nullptr, R, M, K);
        return;
    }
    if (M < 64 || exact_mode()) {
        for (int m = 0; m < M; m++)
            holo_matmul_add(Y + (int64_t)m * N, W, X + (int64_t)m * K, R + (int64_t)m * N, N, K, HOLO_TYPE_Q4_0);
        return;
    }
    if (g_prefill_mode == HOLO_PREFILL_F16 && !((uintptr_t)X & 15u)) {
        gemm_multi(&Y, &W, &N, 1, nullptr, X, M, K, nullptr, R);
        return;
    }
    void *q = nullptr;
    HOLO_CHECK(hipMallocAsync(&q, (size_t)M * (K / 32) * 34, stream()));
    if (!q) return;
    holo_quantize_act_q8_0(q, X, M, K);
    gemm_multi(&Y, &W, &N, 1, q, nullptr, M, K, nullptr, R);
    HOLO_CHECK(hipFreeAsync(q, stream()));
}

void holo_matmul_batch_q4_0_swiglu_add(float *Y, const void *W, float *G, const float *U, const float *R, int M,
                                       int N, int K)
{
    if (M <= 0 || N <= 0) return;
    if (!Y || !W || !G || !U || !R || K % 32 != 0 || K <= 0) {
        HOLO_REJECT("holo_matmul_batch_q4_0_swiglu_add: null pointer or K not a positive multiple of 32");
        return;
    }
    const int t = HOLO_TYPE_Q4_0;
    if (M >= 64 && exact_mode() && exact_fits(&W, &t, 1, G, U, M, K)) {
        exact_product(&Y, &W, &t, &N, 1, G, U, R, M, K);
        return;
    }
    if (M >= 64 && g_prefill_mode == HOLO_PREFILL_F16 && !(((uintptr_t)G | (uintptr_t)U) & 15u)) {
        gemm_multi(&Y, &W, &N, 1, nullptr, G, M, K, U, R);
        return;
    }
    cuda_silu_mul(G, G, U, M * K);
    holo_matmul_batch_q4_0_add(Y, W, G, R, M, N, K);
}

void holo_matmul_batch_q4_0_multi(float *const *Y, const void *const *W, const int *N, int nmat, const float *X,
                                  int M, int K, void *scratch_q8)
{
    if (M <= 0) return;
    if (!Y || !W || !N || !X || !multi_fits(N, nmat)) {
        HOLO_REJECT("holo_matmul_batch_q4_0_multi: null array, or not 1..3 matrices whose N are multiples of 128");
        return;
    }
    const int T[3] = {HOLO_TYPE_Q4_0, HOLO_TYPE_Q4_0, HOLO_TYPE_Q4_0};
    if (M >= 64 && exact_mode() && exact_fits(W, T, nmat, X, nullptr, M, K)) {
        exact_product(Y, W, T, N, nmat, X, nullptr, nullptr, M, K);
        return;
    }
    if (M < 64 || exact_mode()) {
        for (int i = 0; i < nmat; i++) holo_matmul_batch_q4_0(Y[i], W[i], X, M, N[i], K, scratch_q8);
        return;
    }
    if (g_prefill_mode == HOLO_PREFILL_F16 && !((uintptr_t)X & 15u) && K % 32 == 0) {
        holo_gemm_q4_0_f16_multi(Y, W, N, nmat, X, M, K);
        return;
    }
    void *q = scratch_q8;
    if (!q) HOLO_CHECK(hipMallocAsync(&q, (size_t)M * (K / 32) * 34, stream()));
    if (!q) return;
    holo_quantize_act_q8_0(q, X, M, K);
    holo_gemm_q4_0_q8_0_multi(Y, W, N, nmat, q, M, K);
    if (!scratch_q8) HOLO_CHECK(hipFreeAsync(q, stream()));
}


}  // extern "C"

// ---- any weight format: dequantised to an f16 panel, then the f16 product -----------
//
// Q8_0, Q4_K, Q6_K, F16 and F32 weights are dequantised bit-exactly (the
// reference's dequantize_row_*, quant.c:118-311) and rounded to f16 into a
// stream-ordered workspace, w16 = f16_rne(w); the product over that panel is
// the f16 product above: Y = sum_k f16_rne(x) * w16, accumulated in fp32 on
// the matrix cores.  Q4_0 keeps its own kernels (its w16 = f16_rne(f16(dw) *
// (q - 8)) is the same value, unpacked in the GEMM).

// The formats the panel path takes, with K whole blocks.
static bool panel_ok(int type, int K)
{
    switch (type) {
    case HOLO_TYPE_Q4_0:
    case HOLO_TYPE_Q8_0:
    case HOLO_TYPE_F16:
    case HOLO_TYPE_F32: return K % 32 == 0;
    case HOLO_TYPE_Q4_K:
    case HOLO_TYPE_Q6_K: return K % 256 == 0;
    default: return false;
    }
}

static bool panel_src_aligned(const void *W, int type)
{
    const uintptr_t a = (uintptr_t)W;
    return type == HOLO_TYPE_F32 ? (a & 15u) == 0 : type == HOLO_TYPE_F16 ? (a & 1u) == 0 : (a & 3u) == 0;
}

// Matrix i of type types[i] (or all of `type` when types is null).
static void gemm_panel(float *const *Y, const void *const *W, const int *N, int nmat, const float *X, int M, int K,
                       int type, const float *U, const float *R, const int *types = nullptr)
{
    size_t total = 0;
    for (int i = 0; i < nmat; i++) total += (size_t)N[i] * K * 2;  // each a multiple of 64 bytes
    void *ws = workspace(0, total);
    const bool own = ws == nullptr;
    if (own) HOLO_CHECK(hipMallocAsync(&ws, total, stream()));
    if (!ws) return;
    const void *P[kPrefillMats];
    size_t off = 0;
    for (int i = 0; i < nmat; i++) {
        P[i] = (const uint8_t *)ws + off;
        holo_dequant_f16((void *)P[i], W[i], (int64_t)N[i] * K, types ? types[i] : type);
        off += (size_t)N[i] * K * 2;
    }
    gemm_multi(Y, P, N, nmat, nullptr, X, M, K, U, R, true);
    if (own) HOLO_CHECK(hipFreeAsync(ws, stream()));
}

namespace holo {
void panel_workspace_release()
{
    (void)hipDeviceSynchronize();
    for (int i = 0; i < 3; i++) {
        if (g_ws[i]) (void)hipFree(g_ws[i]);
        g_ws[i] = nullptr;
        g_ws_bytes[i] = 0;
    }
}
}  // namespace holo

extern "C" {

void holo_matmul_batch(float *Y, const void *W, const float *X, int M, int N, int K, int type)
{
    if (M <= 0 || N <= 0) return;
    if (type == HOLO_TYPE_Q4_0) {
        holo_matmul_batch_q4_0(Y, W, X, M, N, K, nullptr);
        return;
    }
    if (!Y || !W || !X) {
        HOLO_REJECT("holo_matmul_batch: null pointer");
        return;
    }
    if (M >= 64 && exact_mode() && exact_fits(&W, &type, 1, X, nullptr, M, K)) {
        exact_product(&Y, &W, &type, &N, 1, X, nullptr, nullptr, M, K);
        return;
    }
    if (M < 64 || exact_mode() || !panel_ok(type, K) || !panel_src_aligned(W, type) || ((uintptr_t)X & 15u)) {
        for (int m = 0; m < M; m++) holo_matmul(Y + (int64_t)m * N, W, X + (int64_t)m * K, N, K, type);
        return;
    }
    gemm_panel(&Y, &W, &N, 1, X, M, K, type, nullptr, nullptr);
}

void holo_matmul_batch_multi(float *const *Y, const void *const *W, const int *N, int nmat, const float *X, int M,
                             int K, int type)
{
    if (M <= 0) return;
    if (type == HOLO_TYPE_Q4_0) {
        holo_matmul_batch_q4_0_multi(Y, W, N, nmat, X, M, K, nullptr);
        return;
    }
    if (!Y || !W || !N || !X || !multi_fits(N, nmat)) {
        HOLO_REJECT("holo_matmul_batch_multi: null array, or not 1..3 matrices whose N are multiples of 128");
        return;
    }
    const int T[3] = {type, type, type};
    if (M >= 64 && exact_mode() && exact_fits(W, T, nmat, X, nullptr, M, K)) {
        exact_product(Y, W, T, N, nmat, X, nullptr, nullptr, M, K);
        return;
    }
    bool ok = M >= 64 && !exact_mode() && panel_ok(type, K) && !((uintptr_t)X & 15u);
    for (int i = 0; i < nmat; i++) ok = ok && Y[i] && W[i] && panel_src_aligned(W[i], type);
    if (!ok) {
        for (int i = 0; i < nmat; i++) holo_matmul_batch(Y[i], W[i], X, M, N[i], K, type);
        return;
    }
    gemm_panel(Y, W, N, nmat, X, M, K, type, nullptr, nullptr);
}

void holo_matmul_batch_multi_types(float *const *Y, const void *const *W, const int *types, const int *N, int nmat,
                                   const float *X, int M, int K)
{
    if (M <= 0) return;
    if (!Y || !W || !types || !N || !X || !multi_fits(N, nmat)) {
        HOLO_REJECT("holo_matmul_batch_multi_types: null array, or not 1..3 matrices whose N are multiples of 128");
        return;
    }
    bool same = true;
    for (int i = 1; i < nmat; i++) same = same && types[i] == types[0];
    if (same) {
        holo_matmul_batch_multi(Y, W, N, nmat, X, M, K, types[0]);
        return;
    }
    if (M >= 64 && exact_mode() && exact_fits(W, types, nmat, X, nullptr, M, K)) {
        exact_product(Y, W, types, N, nmat, X, nullptr, nullptr, M, K);
        return;
    }
    bool ok = M >= 64 && !exact_mode() && !((uintptr_t)X & 15u);
    for (int i = 0; i < nmat; i++)
        ok = ok && Y[i] && W[i] && panel_ok(types[i], K) && panel_src_aligned(W[i], types[i]);
    if (!ok) {
        for (int i = 0; i < nmat; i++) holo_matmul_batch(Y[i], W[i], X, M, N[i], K, types[i]);
        return;
    }
    gemm_panel(Y, W, N, nmat, X, M, K, 0, nullptr, nullptr, types);
}

void holo_matmul_batch_add(float *Y, const void *W, const float *X, const float *R, int M, int N, int K, int type)
{
    if (M <= 0 || N <= 0) return;
    if (type == HOLO_TYPE_Q4_0) {
        holo_matmul_batch_q4_0_add(Y, W, X, R, M, N, K);
        return;
    }
    if (!Y || !W || !X || !R) {
        HOLO_REJECT("holo_matmul_batch_add: null pointer");
        return;
    }
    if (M >= 64 && exact_mode() && exact_fits(&W, &type, 1, X, nullptr, M, K)) {
        exact_product(&Y, &W, &type, &N, 1, X, nullptr, R, M, K);  // the add in the GEMM's store
        return;
    }
    if (M >= 64 && !exact_mode() && panel_ok(type, K) && panel_src_aligned(W, type) && !((uintptr_t)X & 15u)) {
        gemm_panel(&Y, &W, &N, 1, X, M, K, type, nullptr, R);  // the add in the GEMM's store
        return;
    }
    // row by row; Y may alias R, so each row's product goes through a scratch row
    float *t = nullptr;
    HOLO_CHECK(hipMallocAsync((void **)&t, sizeof(float) * (size_t)N, stream()));
    if (!t) return;
    for (int m = 0; m < M; m++) {
        holo_matmul(t, W, X + (int64_t)m * K, N, K, type);
        cuda_vec_add(Y + (int64_t)m * N, R + (int64_t)m * N, t, N);
    }
    HOLO_CHECK(hipFreeAsync(t, stream()));
}

void holo_matmul_batch_swiglu_add(float *Y, const void *W, float *G, const float *U, const float *R, int M, int N,
                                  int K, int type)
{
    if (M <= 0 || N <= 0) return;
    if (type == HOLO_TYPE_Q4_0) {
        holo_matmul_batch_q4_0_swiglu_add(Y, W, G, U, R, M, N, K);
        return;
    }
    if (!Y || !W || !G || !U || !R) {
        HOLO_REJECT("holo_matmul_batch_swiglu_add: null pointer");
        return;
    }
    if (M >= 64 && exact_mode() && exact_fits(&W, &type, 1, G, U, M, K)) {
        exact_product(&Y, &W, &type, &N, 1, G, U, R, M, K);  // silu(G) * U in the activation halves
        return;
    }
    if (M >= 64 && !exact_mode() && panel_ok(type, K) && panel_src_aligned(W, type) &&
        !(((uintptr_t)G | (uintptr_t)U) & 15u)) {
        gemm_panel(&Y, &W, &N, 1, G, M, K, type, U, R);  // silu(G) * U in the activation panel
        return;
    }
    cuda_silu_mul(G, G, U, M * K);
    holo_matmul_batch_add(Y, W, G, R, M, N, K, type);
}

}  // extern "C"
