// prefill_exact.hip -- the batched product Y[M][N] = X[M][K] . W[N][K]^T at
// fp32 accuracy on the f16 matrix cores: the default of every batched
// matmul (holo_matmul_batch*, the prompt forward).
//
// The reference has no batched path: its prompt loop multiplies one token at
// a time in fp32 (src/ai/llm.c:1049, matmul_q llm.c:770-926).  The product
// here holds every operand exactly or to 22 bits:
//   activations  x = xh + xl, xh = f16(x), xl = f16(x - xh): |x - xh - xl|
//                <= 2^-22 |x| (xl rounds once more; both halves are f16)
//   weights      the block's integers, exact in f16, with the block's scales
//                in fp32 (every scale product of the formats is exact):
//                  Q4_0  q - 8                 scale d            (quant.c:136-153)
//                  Q8_0  q                     scale d            (quant.c:118-128)
//                  Q4_K  q (0..15), sub-block scale d*sc and min dmin*m
//                                                                 (quant.c:277-311)
//                  Q6_K  q - 32, 16-weight group scale d*sc       (quant.c:241-271)
//                  F16   the weight itself, no scale
// Per 32-block b, output (m, n), the matrix cores accumulate the block's
// integer-weight dot over both activation halves in fp32,
//   C = sum_k (xh[m,k] + xl[m,k]) * w[n,k]      (four v_mfma_f32_32x32x16_f16)
// and the fp32 epilogue folds it in, in block order:
//   acc = fmaf(scale[n,b], C, acc)          (Q6_K: once per 16-weight group)
//   acc = fmaf(-dmin*m[n,b], sum_k x[m,k], acc)    (Q4_K only)
// so the result carries fp32 accumulation error plus the 2^-22 split, not
// the 2^-11 of an f16 operand.  Each row of x is scaled by a power of two
// before the split (largest magnitude into [2^14, 2^15)) and the store
// scales back, so any finite x keeps both halves in f16 range.
//
// Workgroup: 4 waves in a 2 x 2 grid, each owning WM x WN 32 x 32 tiles; K
// advances S blocks per stage through a double-buffered LDS stage, the next
// stage's global loads in registers while the current one is multiplied.
#include "common.h"
#include "quant_blocks.h"
#include "block_reduce.h"

#include <hip/hip_ext.h>
#include <algorithm>
#include <limits.h>
#include <mutex>
#include <unordered_map>

#include <type_traits>

#pragma clang fp contract(off)

namespace holo {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v3u __attribute__((ext_vector_type(3)));

// Weight source of one launch (EW_Q6R: Q6_K repacked for the second tiling).
enum ExactW { EW_Q4_0 = 0, EW_Q8_0 = 1, EW_Q4_K = 2, EW_P16 = 3, EW_F16 = 4, EW_Q6_K = 5, EW_Q6R = 6 };

constexpr int kExactMats = 3;

struct ExactArgs {
    float *Y[kExactMats];
    const uint8_t *W[kExactMats];  // block stream, or f16 panel [N_i][K] (EW_P16, EW_F16)
    const float *WS[kExactMats];   // EW_P16: group scales [N_i][K/16]
    int n_end[kExactMats];         // prefix sums of N_i; unused entries INT_MAX
    const _Float16 *Ah, *Al;       // activation halves [M][K]
    const float *Sx;               // [M][nb] block sums of x (EW_Q4_K)
    const float *Rs;               // [M] row scales: the halves hold x / Rs
    int M, N, nb;
    int ntm, tiles;
    const float *R;                // one matrix only: Y = R + product (may alias Y)
};

struct ExactMat {
    const uint8_t *W;
    const float *WS;
    float *Y;
    int nbase, N;
    int64_t w_bytes;
};

// ---- integers of a block in f16 ----------------------------------------------------
// v_perm pairs a byte with 0x64, giving the f16 value 1024 + byte; one
// packed f16 add removes the bias, exactly.

__device__ __forceinline__ uint32_t f16_pair(uint32_t bytes, uint32_t sel, _Float16 bias)
{
    const h2 b2 = {bias, bias};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, bytes, sel)) + b2);
}

// Eight nibbles of x (four bytes): lo[0..1] = low nibbles (k = 4j..4j+3 of the
// block), hi[0..1] = high nibbles (k = 16+4j..), each as f16 (nibble + off).
__device__ __forceinline__ void nibbles_f16(uint32_t x, _Float16 off, uint32_t lo[2], uint32_t hi[2])
{
    const uint32_t t0 = x & 0x0F0F0F0Fu, t1 = (x >> 4) & 0x0F0F0F0Fu;
    const _Float16 bias = (_Float16)(-1024.0f) + off;
    lo[0] = f16_pair(t0, 0x04010400u, bias);
    lo[1] = f16_pair(t0, 0x04030402u, bias);
    hi[0] = f16_pair(t1, 0x04010400u, bias);
    hi[1] = f16_pair(t1, 0x04030402u, bias);
}

// Four signed bytes as f16: byte ^ 0x80 is q + 128 in 0..255.
__device__ __forceinline__ void int8s_f16(uint32_t x, uint32_t out[2])
{
    const uint32_t t = x ^ 0x80808080u;
    out[0] = f16_pair(t, 0x04010400u, (_Float16)-1152.0f);
    out[1] = f16_pair(t, 0x04030402u, (_Float16)-1152.0f);
}

template <int WM, int WN, int S>
struct XGeo {
    static constexpr int NT = 256;
    static constexpr int TM = 64 * WM, TN = 64 * WN;
    static constexpr int ROW = 32 * S + 8;  // f16 per LDS row; the 16-byte pad spreads rows over the banks
    static constexpr int AH = 0;
    static constexpr int AL = AH + TM * ROW * 2;
    static constexpr int B = AL + TM * ROW * 2;
    static constexpr int BS = B + TN * ROW * 2;   // fp32 [TN][2S]: scale of each 16-weight half-block
    static constexpr int BM = BS + TN * 2 * S * 4;  // fp32 [TN][S]: Q4_K mins
    static constexpr int AS = BM + TN * S * 4;    // fp32 [S][TM]: block sums of x
    static constexpr int STAGE = (AS + S * TM * 4 + 15) & ~15;
    static constexpr int LDS = 2 * STAGE;
    static constexpr int NA = TM * S * 4 / NT;           // 16-byte activation pieces per thread and half
    static constexpr int NAS = (TM * S + NT - 1) / NT;   // block sums per thread
    static constexpr int NB = (TN * S + NT - 1) / NT;    // weight blocks per thread
    static constexpr int NH = (TN * S * 2 + NT - 1) / NT;  // Q6_K: 16-weight half blocks per thread
    static constexpr int NWP = (TN * S * 4 + NT - 1) / NT;  // 16-byte weight-panel pieces per thread
    static constexpr int NWS = (TN * 2 * S + NT - 1) / NT;  // group scales per thread
    static_assert((TM * S * 4) % NT == 0, "activation pieces must split evenly over the threads");
};

template <int WF>
struct WRaw;
template <>
struct WRaw<EW_Q4_0> {
    Q4_0Raw r;
};
template <>
struct WRaw<EW_Q8_0> {
    Q8_0Raw r;
};
template <>
struct WRaw<EW_Q4_K> {
    v4u h, q;
    uint32_t j;
};
// Half p of a 32-weight sub-block of a Q6_K superblock (210 bytes: ql[128],
// qh[64], int8 scales[16], f16 d; quant.c:241-271): sub-block j of half hf
// holds, for l = 0..31, q = ((ql[64hf + 32(j&1) + l] >> 4(j>>1)) & 15) |
// (((qh[32hf + l] >> 2j) & 3) << 4), weight (d * sc[8hf + 2j + l/16]) * (q - 32);
// half p is l = 16p .. 16p + 15, one scale.  l and h are the dwords around its
// 16 ql and 16 qh bytes as loaded (the runs start s = 0 or 2 bytes into their
// first dword), sc its scale byte (bits 0-7 or 8-15 of the pair), d.  Half
// blocks rather than blocks, so that every thread of the workgroup unpacks
// (with whole blocks, half of the waves did and the others waited at the
// barrier).
template <>
struct WRaw<EW_Q6_K> {
    uint32_t l[5], h[5];
    uint32_t sc, d, s, j;
};

constexpr uint32_t kXBufWord3 = kRawBufWord3;

// The per-thread part of every stage load's address, computed once per
// workgroup: a stage then adds only its block index (a scalar multiple) to a
// 32-bit offset, where computing each 64-bit address per load and block cost
// about as many VALU instructions as the block's scale epilogue.  Rows and
// columns past the last one are clamped here, blocks past the last one per
// stage (they are re-read, in bounds, and never used).
template <int WF, int WM, int WN, int S>
struct XAddr {
    using G = XGeo<WM, WN, S>;
    static constexpr bool PANEL = WF == EW_P16 || WF == EW_F16;
    static constexpr int NWI = PANEL ? G::NWP : WF == EW_Q6_K ? G::NH : G::NB;
    __amdgpu_buffer_rsrc_t rah, ral;  // the activation halves (M*K f16 each, at most 2 GiB: exact_fits)
    uint32_t oa[G::NA];               // byte offset of A piece i at block 0
    int ka[G::NA];                    // its block within the stage
    int64_t ow[NWI];                  // weights: byte offset of the piece's row (at block 0)
    int kw[NWI];                      // its block within the stage

    __device__ __forceinline__ XAddr(const ExactArgs &a, const ExactMat &w, int tid, int m0, int n0)
    {
        const int nb = a.nb;
        const uint32_t abytes = (uint32_t)((int64_t)a.M * nb * 64);
        rah = __builtin_amdgcn_make_buffer_rsrc((void *)a.Ah, (short)0, (int)abytes, kXBufWord3);
        ral = __builtin_amdgcn_make_buffer_rsrc((void *)a.Al, (short)0, (int)abytes, kXBufWord3);
#pragma unroll
        for (int i = 0; i < G::NA; i++) {
            const int p = tid + G::NT * i, r = p / (4 * S), c = p % (4 * S);
            oa[i] = (uint32_t)min(m0 + r, a.M - 1) * (uint32_t)(nb * 64) + (uint32_t)(c % 4) * 16u;
            ka[i] = c / 4;
        }
#pragma unroll
        for (int i = 0; i < NWI; i++) {
            if constexpr (PANEL) {
                const int p = min(tid + G::NT * i, G::TN * S * 4 - 1), n = p / (4 * S), c = p % (4 * S);
                ow[i] = (int64_t)min(n0 + n, w.N - 1) * nb * 64 + (c % 4) * 16;
                kw[i] = c / 4;
            } else if constexpr (WF == EW_Q6_K) {
                // half block v: row v / 2S, block (v % 2S) / 2, half v % 2
                const int v = min(tid + G::NT * i, G::TN * S * 2 - 1);
                ow[i] = (int64_t)min(n0 + v / (2 * S), w.N - 1) * (nb / 8) * 210;
                kw[i] = v % (2 * S);
            } else {
                const int v = min(tid + G::NT * i, G::TN * S - 1), n = v / S;
                const int64_t row = min(n0 + n, w.N - 1);
                ow[i] = WF == EW_Q4_K ? row * (nb / 8) * 144 : row * nb * (WF == EW_Q4_0 ? 18 : 34);
                kw[i] = v % S;
            }
        }
    }
};

// Registers of one stage between its global loads and its LDS writes: blocks
// kb0 .. kb0+S-1 of the workgroup's rows and columns.  Indices past the last
// row, column or block re-read the last one (in bounds, never used).
template <int WF, int WM, int WN, int S>
struct XStage {
    using G = XGeo<WM, WN, S>;
    static constexpr bool PANEL = WF == EW_P16 || WF == EW_F16;
    v4u ah[G::NA], al[G::NA];
    float as[WF == EW_Q4_K ? G::NAS : 1];
    WRaw<WF == EW_Q4_0 || WF == EW_Q8_0 || WF == EW_Q4_K || WF == EW_Q6_K ? WF : EW_Q4_0>
        rb[PANEL ? 1 : WF == EW_Q6_K ? G::NH : G::NB];
    v4u rw[PANEL ? G::NWP : 1];
    float rs[WF == EW_P16 ? G::NWS : 1];

    __device__ __forceinline__ void fetch(const ExactArgs &a, const ExactMat &w, const XAddr<WF, WM, WN, S> &ad,
                                          int tid, int m0, int n0, int kb0)
    {
        const int nb = a.nb;
#pragma unroll
        for (int i = 0; i < G::NA; i++) {
            const uint32_t o = ad.oa[i] + (uint32_t)min(kb0 + ad.ka[i], nb - 1) * 64u;
            ah[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(ad.rah, (int)o, 0, 0));
            al[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(ad.ral, (int)o, 0, 0));
        }
        if constexpr (WF == EW_Q4_K) {
#pragma unroll
            for (int i = 0; i < G::NAS; i++) {
                const int v = min(tid + G::NT * i, G::TM * S - 1), sb = v / G::TM, r = v % G::TM;
                as[i] = a.Sx[(int64_t)min(m0 + r, a.M - 1) * nb + min(kb0 + sb, nb - 1)];
            }
        }
        if constexpr (PANEL) {
#pragma unroll
            for (int i = 0; i < G::NWP; i++)
                rw[i] = *(const v4u *)(w.W + ad.ow[i] + (int64_t)min(kb0 + ad.kw[i], nb - 1) * 64);
            if constexpr (WF == EW_P16) {
#pragma unroll
                for (int i = 0; i < G::NWS; i++) {
                    const int v = min(tid + G::NT * i, G::TN * 2 * S - 1), n = v / (2 * S), j = v % (2 * S);
                    rs[i] = w.WS[(int64_t)min(n0 + n, w.N - 1) * (2 * nb) + min(2 * kb0 + j, 2 * nb - 1)];
                }
            }
            return;
        }
        if constexpr (WF == EW_Q6_K) {
            // half p of sub-block b & 7 of superblock b / 8 (nb is a multiple
            // of 8); superblocks sit at even addresses, the runs at the
            // superblock's offset within a dword, and the fifth dword of a
            // run still lies inside the superblock
            typedef __attribute__((address_space(1))) const uint32_t g32;
            typedef __attribute__((address_space(1))) const uint16_t g16;
            typedef __attribute__((address_space(1))) const u32x4 g128;
#pragma unroll
            for (int i = 0; i < G::NH; i++) {
                const int b = min(kb0 + (ad.kw[i] >> 1), nb - 1), p = ad.kw[i] & 1;
                const uint8_t *sb = w.W + ad.ow[i] + (int64_t)(b >> 3) * 210;
                const uint32_t sub = (uint32_t)(b & 7), hf = sub >> 2, j = sub & 3;
                const uint32_t sh = (uint32_t)((uintptr_t)sb & 3u);
                const uintptr_t pl = (uintptr_t)(sb + 64 * hf + 32 * (j & 1) + 16 * p - sh);
                const uintptr_t ph = (uintptr_t)(sb + 128 + 32 * hf + 16 * p - sh);
                const u32x4 l4 = *(const g128 *)pl, h4 = *(const g128 *)ph;
                rb[i].l[0] = l4.x;
                rb[i].l[1] = l4.y;
                rb[i].l[2] = l4.z;
                rb[i].l[3] = l4.w;
                rb[i].l[4] = *(const g32 *)(pl + 16);
                rb[i].h[0] = h4.x;
                rb[i].h[1] = h4.y;
                rb[i].h[2] = h4.z;
                rb[i].h[3] = h4.w;
                rb[i].h[4] = *(const g32 *)(ph + 16);
                rb[i].sc = *(const g16 *)(sb + 192 + 8 * hf + 2 * j);
                rb[i].d = *(const g16 *)(sb + 208);
                rb[i].s = sh;
                rb[i].j = j;
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < G::NB; i++) {
            const int b = min(kb0 + ad.kw[i], nb - 1);
            if constexpr (WF == EW_Q4_0) {
                rb[i].r = load_q4_0_raw(w.W, ad.ow[i] + (int64_t)b * 18, w.w_bytes);
            } else if constexpr (WF == EW_Q8_0) {
                rb[i].r = load_q8_0_raw(w.W, ad.ow[i] + (int64_t)b * 34, w.w_bytes);
            } else if constexpr (WF == EW_Q4_K) {
                // block b of the row: superblock b / 8 (144 bytes, 16-byte
                // aligned; nb is a multiple of 8), sub-block b % 8
                const uint8_t *sb = w.W + ad.ow[i] + (int64_t)(b >> 3) * 144;
                rb[i].j = (uint32_t)(b & 7);
                rb[i].h = *(const v4u *)sb;
                rb[i].q = *(const v4u *)(sb + 16 + 16 * rb[i].j);
            }
        }
    }

    __device__ __forceinline__ void stash(uint8_t *base, int tid) const
    {
#pragma unroll
        for (int i = 0; i < G::NA; i++) {
            const int p = tid + G::NT * i, r = p / (4 * S), c = p % (4 * S);
            *(v4u *)(base + G::AH + (r * G::ROW + c * 8) * 2) = ah[i];
            *(v4u *)(base + G::AL + (r * G::ROW + c * 8) * 2) = al[i];
        }
        if constexpr (WF == EW_Q4_K) {
#pragma unroll
            for (int i = 0; i < G::NAS; i++) {
                const int v = tid + G::NT * i;
                if (v < G::TM * S) ((float *)(base + G::AS))[v] = as[i];  // [S][TM]
            }
        }
        if constexpr (PANEL) {
#pragma unroll
            for (int i = 0; i < G::NWP; i++) {
                const int p = tid + G::NT * i, n = p / (4 * S), c = p % (4 * S);
                if (p < G::TN * S * 4) *(v4u *)(base + G::B + (n * G::ROW + c * 8) * 2) = rw[i];
            }
            if constexpr (WF == EW_P16) {
#pragma unroll
                for (int i = 0; i < G::NWS; i++) {
                    const int v = tid + G::NT * i;
                    if (v < G::TN * 2 * S) ((float *)(base + G::BS))[v] = rs[i];
                }
            }
            return;
        }
        if constexpr (WF == EW_Q6_K) {
#pragma unroll
            for (int i = 0; i < G::NH; i++) {
                const int v = tid + G::NT * i, n = v / (2 * S), sb = (v % (2 * S)) >> 1, p = v & 1;
                if (v >= G::TN * S * 2) continue;
                const WRaw<EW_Q6_K> &r = rb[i];
                const uint32_t shq = 4 * (r.j >> 1), shh = 2 * r.j;
                uint32_t wv[8];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const uint32_t l = __builtin_amdgcn_alignbyte(r.l[c + 1], r.l[c], r.s);
                    const uint32_t hb = __builtin_amdgcn_alignbyte(r.h[c + 1], r.h[c], r.s);
                    const uint32_t q = ((l >> shq) & 0x0F0F0F0Fu) | (((hb >> shh) & 0x03030303u) << 4);
                    wv[2 * c] = f16_pair(q, 0x04010400u, (_Float16)-1056.0f);  // 1024 + q - 1056 = q - 32
                    wv[2 * c + 1] = f16_pair(q, 0x04030402u, (_Float16)-1056.0f);
                }
                v4u *dst = (v4u *)(base + G::B + (n * G::ROW + sb * 32 + 16 * p) * 2);
                dst[0] = v4u{wv[0], wv[1], wv[2], wv[3]};  // k = 16p .. 16p + 7
                dst[1] = v4u{wv[4], wv[5], wv[6], wv[7]};
                // exact: 11-bit x 8-bit
                ((float *)(base + G::BS))[n * 2 * S + 2 * sb + p] =
                    half_bits_to_float(r.d) * (float)(int8_t)((r.sc >> (8 * p)) & 0xFFu);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < G::NB; i++) {
            const int v = tid + G::NT * i, n = v / S, sb = v % S;
            if (v >= G::TN * S) continue;
            uint32_t lo[8], hi[8];
            float scale, mn = 0.f;
            if constexpr (WF == EW_Q4_0) {
                const Q4_0Unit u = q4_0_unit(rb[i].r);
#pragma unroll
                for (int j = 0; j < 4; j++) nibbles_f16(u.q[j], (_Float16)-8.0f, &lo[2 * j], &hi[2 * j]);
                scale = u.d;
            } else if constexpr (WF == EW_Q8_0) {
                const Q8_0Unit u = q8_0_unit(rb[i].r);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    int8s_f16(u.q[j], &lo[2 * j]);
                    int8s_f16(u.q[4 + j], &hi[2 * j]);
                }
                scale = u.d;
            } else if constexpr (WF == EW_Q4_K) {
                const v4u q = rb[i].q;
#pragma unroll
                for (int j = 0; j < 4; j++) nibbles_f16(q[j], (_Float16)0.0f, &lo[2 * j], &hi[2 * j]);
                uint32_t sc, m6;
                q4_k_scale_min(rb[i].h.y, rb[i].h.z, rb[i].h.w, rb[i].j, sc, m6);
                scale = half_bits_to_float(rb[i].h.x) * (float)sc;  // exact: 11-bit x 6-bit
                mn = half_bits_to_float(rb[i].h.x >> 16) * (float)m6;
            }
            v4u *dst = (v4u *)(base + G::B + (n * G::ROW + sb * 32) * 2);
            dst[0] = v4u{lo[0], lo[1], lo[2], lo[3]};  // k = 0..7
            dst[1] = v4u{lo[4], lo[5], lo[6], lo[7]};  // k = 8..15
            dst[2] = v4u{hi[0], hi[1], hi[2], hi[3]};  // k = 16..23
            dst[3] = v4u{hi[4], hi[5], hi[6], hi[7]};  // k = 24..31
            ((float *)(base + G::BS))[n * 2 * S + 2 * sb] = scale;
            if constexpr (WF == EW_Q4_K) ((float *)(base + G::BM))[n * S + sb] = mn;
        }
    }
};

__device__ __forceinline__ v16f mfma16(v8h a, v8h b, v16f c)
{
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_32x32x16_f16 (wave64): lane l supplies A[l%32][8*(l/32)+t] and
// B[8*(l/32)+t][l%32], t = 0..7; D[i][j] lands in lane j + 32*((i/4)%2),
// register (i%4) + 4*(i/8).  A lane's 16 outputs share one column n, so a
// block's scale is one value per lane.
// RD: stages of global loads in flight in registers (a ring), so each
// stage's loads have RD - 1 stages of products to land behind.
template <int WF, int WM, int WN, int S, int OCC, int RD>
__global__ __launch_bounds__(256, OCC) void gemm_exact_k(ExactArgs a)
{
    using G = XGeo<WM, WN, S>;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ __align__(16) float rs_l[G::TM];  // the tile's row scales
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, c32 = lane & 31;

    // Tile of this workgroup: XCD x (workgroups go to the 8 XCDs round
    // robin) takes a contiguous run of tiles when the count allows, so the
    // row tiles that share a weight tile share that XCD's L2.
    const int g = blockIdx.x;
    const int t = (a.tiles & 7) ? g : (g & 7) * (a.tiles >> 3) + (g >> 3);
    const int m0 = (t % a.ntm) * G::TM, ng = (t / a.ntm) * G::TN;
    // read in the epilogue, after the stage loop's barriers
    if (tid < G::TM) rs_l[tid] = a.Rs[min(m0 + tid, a.M - 1)];
    const int sel = (ng >= a.n_end[0]) + (ng >= a.n_end[1]);
    ExactMat w;
    w.W = sel == 2 ? a.W[2] : sel == 1 ? a.W[1] : a.W[0];
    w.WS = sel == 2 ? a.WS[2] : sel == 1 ? a.WS[1] : a.WS[0];
    w.Y = sel == 2 ? a.Y[2] : sel == 1 ? a.Y[1] : a.Y[0];
    w.nbase = sel == 2 ? a.n_end[1] : sel == 1 ? a.n_end[0] : 0;
    w.N = (sel == 2 ? a.n_end[2] : sel == 1 ? a.n_end[1] : a.n_end[0]) - w.nbase;
    w.w_bytes = (int64_t)w.N * a.nb * (WF == EW_Q4_0 ? 18 : 34);
    const int n0 = ng - w.nbase;
    const int wm0 = (wave >> 1) * 32 * WM, wn0 = (wave & 1) * 32 * WN;
    const int nb = a.nb;
    const int nst = (nb + S - 1) / S;
    v16f acc[WM][WN];
#pragma unroll
    for (int mi = 0; mi < WM; mi++)
#pragma unroll
        for (int ni = 0; ni < WN; ni++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;

    auto compute = [&](int buf, int kb0) {
        const uint8_t *base = lds + buf * G::STAGE;
        const _Float16 *lAh = (const _Float16 *)(base + G::AH);
        const _Float16 *lAl = (const _Float16 *)(base + G::AL);
        const _Float16 *lB = (const _Float16 *)(base + G::B);
        const float *lBs = (const float *)(base + G::BS);
        const float *lBm = (const float *)(base + G::BM);
        const float *lAs = (const float *)(base + G::AS);
        const v16f zero = {};
#pragma unroll
        for (int s = 0; s < S; s++) {
            if (kb0 + s >= nb) break;
            v8h ah0[WM], ah1[WM], al0[WM], al1[WM], b0[WN], b1[WN];
            float sc0[WN], sc1[WN], mn[WN];
            float4 sx[WM][4];
#pragma unroll
            for (int mi = 0; mi < WM; mi++) {
                const int r = wm0 + 32 * mi + c32;
                const int o = r * G::ROW + s * 32 + 8 * h;
                ah0[mi] = *(const v8h *)(lAh + o);
                ah1[mi] = *(const v8h *)(lAh + o + 16);
                al0[mi] = *(const v8h *)(lAl + o);
                al1[mi] = *(const v8h *)(lAl + o + 16);
                if constexpr (WF == EW_Q4_K) {
                    // rows (r & 3) + 4h + 8(r >> 2) of register r: four runs of four
#pragma unroll
                    for (int q = 0; q < 4; q++) sx[mi][q] = *(const float4 *)(lAs + s * G::TM + wm0 + 32 * mi + 8 * q + 4 * h);
                }
            }
#pragma unroll
            for (int ni = 0; ni < WN; ni++) {
                const int n = wn0 + 32 * ni + c32;
                const int o = n * G::ROW + s * 32 + 8 * h;
                b0[ni] = *(const v8h *)(lB + o);
                b1[ni] = *(const v8h *)(lB + o + 16);
                sc0[ni] = lBs[n * 2 * S + 2 * s];
                sc1[ni] = lBs[n * 2 * S + 2 * s + 1];
                mn[ni] = WF == EW_Q4_K ? lBm[n * S + s] : 0.f;
            }
#pragma unroll
            for (int mi = 0; mi < WM; mi++)
#pragma unroll
                for (int ni = 0; ni < WN; ni++) {
                    if constexpr (WF == EW_F16) {
                        acc[mi][ni] = mfma16(ah0[mi], b0[ni], acc[mi][ni]);
                        acc[mi][ni] = mfma16(ah1[mi], b1[ni], acc[mi][ni]);
                        acc[mi][ni] = mfma16(al0[mi], b0[ni], acc[mi][ni]);
                        acc[mi][ni] = mfma16(al1[mi], b1[ni], acc[mi][ni]);
                    } else if constexpr (WF == EW_P16 || WF == EW_Q6_K) {
                        v16f c = mfma16(al0[mi], b0[ni], mfma16(ah0[mi], b0[ni], zero));
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[mi][ni][r] = __builtin_fmaf(sc0[ni], c[r], acc[mi][ni][r]);
                        c = mfma16(al1[mi], b1[ni], mfma16(ah1[mi], b1[ni], zero));
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[mi][ni][r] = __builtin_fmaf(sc1[ni], c[r], acc[mi][ni][r]);
                    } else {
                        v16f c = mfma16(ah0[mi], b0[ni], zero);
                        c = mfma16(ah1[mi], b1[ni], c);
                        c = mfma16(al0[mi], b0[ni], c);
                        c = mfma16(al1[mi], b1[ni], c);
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[mi][ni][r] = __builtin_fmaf(sc0[ni], c[r], acc[mi][ni][r]);
                        if constexpr (WF == EW_Q4_K) {
#pragma unroll
                            for (int r = 0; r < 16; r++)
                                acc[mi][ni][r] = __builtin_fmaf(-mn[ni], sx[mi][r >> 2][r & 3], acc[mi][ni][r]);
                        }
                    }
                }
        }
    };

    // Ring of RD register stages: set d holds stage k with k % RD == d.
    // Stages past the last block re-read the last one (fetch clamps every
    // index), so every slot issues the same loads and the loop has one exit,
    // at its latch, with a trip count known up front: the compiler's wait
    // before each stash is then exactly that stage's own loads.
    const XAddr<WF, WM, WN, S> ad(a, w, tid, m0, n0);
    XStage<WF, WM, WN, S> st[RD];
#pragma unroll
    for (int d = 0; d < RD; d++) st[d].fetch(a, w, ad, tid, m0, n0, d * S);
    st[0].stash(lds, tid);
    st[0].fetch(a, w, ad, tid, m0, n0, RD * S);
    __syncthreads();
    const int rounds = (nst + RD - 1) / RD;
    for (int q = 0; q < rounds; q++) {
#pragma unroll
        for (int d = 0; d < RD; d++) {
            const int k = q * RD + d;  // compute(k) skips blocks past nb
            compute(k & 1, k * S);
            // stage k + 1 (register set (d + 1) % RD) into the other buffer,
            // then that set fetches stage k + 1 + RD
            st[(d + 1) % RD].stash(lds + ((k + 1) & 1) * G::STAGE, tid);
            st[(d + 1) % RD].fetch(a, w, ad, tid, m0, n0, (k + 1 + RD) * S);
            __syncthreads();
        }
    }

    // the residual of every output first, in one batch of loads: a load
    // between stores would wait for the stores issued before it as well
    float rv[WM][WN][16];
    if (a.R) {
#pragma unroll
        for (int mi = 0; mi < WM; mi++)
#pragma unroll
            for (int ni = 0; ni < WN; ni++) {
                const int n = min(n0 + wn0 + 32 * ni + c32, w.N - 1);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = min(m0 + wm0 + 32 * mi + (r & 3) + 4 * h + 8 * (r >> 2), a.M - 1);
                    rv[mi][ni][r] = a.R[(int64_t)m * w.N + n];
                }
            }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int mi = 0; mi < WM; mi++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            // rows wm0 + 32 mi + 8 q + 4 h + j, j = 0..3: one LDS read
            const float4 rs = *(const float4 *)(rs_l + wm0 + 32 * mi + 8 * q + 4 * h);
            const float rsj[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
            for (int ni = 0; ni < WN; ni++) {
                const int n = n0 + wn0 + 32 * ni + c32;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int r = 4 * q + j;
                    const int m = m0 + wm0 + 32 * mi + j + 4 * h + 8 * q;
                    if (m < a.M && n < w.N) {
                        const int64_t o = (int64_t)m * w.N + n;
                        const float y = acc[mi][ni][r] * rsj[j];  // a power of two: exact
                        w.Y[o] = a.R ? rv[mi][ni][r] + y : y;
                    }
                }
            }
        }
}

// ---- the activation halves: Ah, Al [M][K] f16, block sums Sx [M][K/32], row scales Rs [M] ----
// One workgroup per row.  The row's values y (x; silu(g) * u as
// cuda_silu_mul computes it, cuda_ops.cu:304-314; or the RMS-normed row,
// rms_norm_rows4_k's arithmetic: thread t sums the squares of float4s
// t + 256 j, the same workgroup reduction, x * scale * w, so the normed
// values are the bits the separate norm writes) are scaled by a power of two
// 2^e chosen from the row's largest magnitude a: a * 2^e lies in
// [2^14, 2^15).  The halves then never overflow f16 (|y| up to fp32's range
// is taken) and the low half is a normal f16 for every value above
// a * 2^-17, so x - xh - xl stays within 2^-22 |x| there and within
// a * 2^-40 below.  The product's store multiplies by Rs = 2^-e (exact).  A
// 32-block is the 8 float4 of 8 adjacent lanes (K % 32 == 0); Sx holds the
// block sums of the scaled values (for the Q4_K min term).
enum XSplitMode { XS_PLAIN = 0, XS_SWIGLU = 1, XS_NORM = 2 };

template <int NV, int MODE, int NT = 256>
__global__ __launch_bounds__(NT) void xsplit_row_k(uint2 *__restrict__ Ah, uint2 *__restrict__ Al,
                                                    float *__restrict__ Sx, float *__restrict__ Rs,
                                                    const float *__restrict__ X, const float *__restrict__ U,
                                                    const float *__restrict__ NW, int K, float eps)
{
    __shared__ float red[16];
    const int n4 = K >> 2;
    const int64_t r4 = (int64_t)blockIdx.x * n4;
    // every load of the row issued first, through buffer resources over the
    // row (and the norm weights): a float4 past K reads zeros, so no load
    // waits behind a branch or behind another's arithmetic
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void *)((const float4 *)X + r4), (short)0, K * 4, kXBufWord3);
    const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(MODE == XS_SWIGLU ? (const float4 *)U + r4 : (const float4 *)X + r4), (short)0, K * 4, kXBufWord3);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)(MODE == XS_NORM ? NW : X), (short)0, K * 4, kXBufWord3);
    float4 v[NV], wv[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int o = (int)(threadIdx.x + NT * j) * 16;
        v[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
        if constexpr (MODE == XS_SWIGLU)
            wv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ru, o, 0, 0));
        if constexpr (MODE == XS_NORM)
            wv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rw, o, 0, 0));
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        if constexpr (MODE == XS_SWIGLU) {
            const float4 u = wv[j];
            v[j].x = (v[j].x / (1.0f + expf(-v[j].x))) * u.x;
            v[j].y = (v[j].y / (1.0f + expf(-v[j].y))) * u.y;
            v[j].z = (v[j].z / (1.0f + expf(-v[j].z))) * u.z;
            v[j].w = (v[j].w / (1.0f + expf(-v[j].w))) * u.w;
        }
        if constexpr (MODE == XS_NORM)
            ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    }
    float scale = 1.f;
    if constexpr (MODE == XS_NORM) {
        ss = block_reduce<false>(ss, red);
        scale = 1.0f / sqrtf(ss / (float)K + eps);
    }
    float am = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        if constexpr (MODE == XS_NORM) {
            const float4 w4 = wv[j];
            v[j] = make_float4(v[j].x * scale * w4.x, v[j].y * scale * w4.y, v[j].z * scale * w4.z,
                               v[j].w * scale * w4.w);
        }
        am = fmaxf(am, fmaxf(fmaxf(fabsf(v[j].x), fabsf(v[j].y)), fmaxf(fabsf(v[j].z), fabsf(v[j].w))));
    }
    am = block_reduce<true>(am, red);
    // 2^e with a * 2^e in [2^14, 2^15); e = 0 for a zero or non-finite row
    int e = 0;
    if (am > 0.f && am <= 3.4028235e38f) {
        int ea;
        (void)frexpf(am, &ea);  // am = f * 2^ea, f in [0.5, 1)
        e = 15 - ea;
    }
    if (threadIdx.x == 0) Rs[blockIdx.x] = ldexpf(1.0f, -e);
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = threadIdx.x + NT * j;
        if (NT * j >= n4) break;  // uniform: no lane of this or a later j is live
        const float y[4] = {ldexpf(v[j].x, e), ldexpf(v[j].y, e), ldexpf(v[j].z, e), ldexpf(v[j].w, e)};
        _Float16 h[4], l[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            h[q] = (_Float16)y[q];
            l[q] = (_Float16)(y[q] - (float)h[q]);
        }
        // the block's sum over its 8 lanes (octets are wholly live or dead)
        float s = (y[0] + y[1]) + (y[2] + y[3]);
        s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
        s += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
        s += __shfl_xor(s, 4, 64);
        if (i < n4) {
            Ah[r4 + i] = make_uint2(__builtin_bit_cast(uint32_t, h2{h[0], h[1]}), __builtin_bit_cast(uint32_t, h2{h[2], h[3]}));
            Al[r4 + i] = make_uint2(__builtin_bit_cast(uint32_t, h2{l[0], l[1]}), __builtin_bit_cast(uint32_t, h2{l[2], l[3]}));
            if (Sx && (i & 7) == 0) Sx[r4 / 8 + (i >> 3)] = s;
        }
    }
}

// ---- Q6_K integer panel: (q - 32) in f16 [N][K] and the group scales d*sc [N][K/16] ----
// One thread per (superblock, half h, slice s): l = 16s .. 16s + 15 of the
// half, all four j, the values y[256b + 128h + 32j + l] of
// dequantize_row_q6_k (quant.c:252-268) without their scale, which goes to
// group (256b + 128h + 32j + 16s) / 16.

__global__ __launch_bounds__(256) void q6_k_int_panel_k(_Float16 *__restrict__ y, float *__restrict__ ys,
                                                        const uint8_t *__restrict__ W, int64_t ntask)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= ntask) return;
    const int64_t b = t >> 2;
    const int hf = (int)((t >> 1) & 1), sl = (int)(t & 1);
    const uint8_t *sb = W + b * 210;
    uint32_t qa[4], qb[4], qh[4];
    q6_run16(sb + 64 * hf + 16 * sl, qa);
    q6_run16(sb + 64 * hf + 32 + 16 * sl, qb);
    q6_run16(sb + 128 + 32 * hf + 16 * sl, qh);
    const int8_t *sc = (const int8_t *)(sb + 192) + 8 * hf;
    const float d = half_bits_to_float_exact((uint32_t)sb[208] | ((uint32_t)sb[209] << 8));
    _Float16 *o = y + b * 256 + 128 * hf + 16 * sl;
    float *os = ys + b * 16 + 8 * hf + sl;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t *ql = (j & 1) ? qb : qa;
        os[2 * j] = d * (float)sc[sl + 2 * j];  // exact: 11-bit x 8-bit
        uint32_t wv[8];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t q = ((ql[c] >> (4 * (j >> 1))) & 0x0F0F0F0Fu) | (((qh[c] >> (2 * j)) & 0x03030303u) << 4);
            wv[2 * c] = f16_pair(q, 0x04010400u, (_Float16)-1056.0f);      // 1024 + q - 1056 = q - 32
            wv[2 * c + 1] = f16_pair(q, 0x04030402u, (_Float16)-1056.0f);
        }
        uint4 *p = (uint4 *)(o + 32 * j);
        p[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
        p[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
    }
}

// ---- Q6_K repacked for the second tiling: 64 bytes per row and 64-weight stage ----
// Record (row n, stage t) holds blocks 2t and 2t + 1 of the row: sub-blocks
// sub = 2(t mod 4) + s (s = 0, 1) of superblock t / 4, so the stage's two
// sub-blocks share their half hf = (t mod 4) / 2, their nibble shift
// 4 (t mod 2) and their qh bytes.  Lane half h of the product reads the two
// 16-byte pieces at 16 h and 32 + 16 h:
//   dword 4h + 2s + j  (j = 0, 1): byte u holds the low nibble of weight
//                      8h + 4j + u of block s (its first k-step) in bits 0-3
//                      and that of weight 16 + 8h + 4j + u (second k-step)
//                      in bits 4-7 -- a Q4_0 qs word
//   dword 8 + 4h + s:  bits 8u + 4j + 2e .. + 1 hold bits 4-5 of weight
//                      16e + 8h + 4j + u of block s
//   dword 8 + 4h + 2:  the four int8 group scales, block s group g in byte 2s + g
//   dword 8 + 4h + 3:  d (f16 bits; the high half zero)
// with q as dequantize_row_q6_k (quant.c:252-268) takes it:
// q = ((ql[64hf + 32(j&1) + l] >> 4(j>>1)) & 15) | (((qh[32hf + l] >> 2j) & 3) << 4),
// j = sub mod 4, scale sc[8hf + 2j + l/16].  The bytes are the superblock's own
// bits rearranged: the product reads the same integers and scales.
// One thread per record; superblock k's records are 4k .. 4k + 3.
__global__ __launch_bounds__(256) void q6r_repack_k(uint4 *__restrict__ out, const uint8_t *__restrict__ W,
                                                    int64_t nrec)
{
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nrec) return;
    const int64_t k = t >> 2;
    const int q = (int)(t & 3), hf = q >> 1, j0 = 2 * (q & 1);
    const uint8_t *sb = W + k * 210;
    uint32_t l0[8], qh[8];  // ql[64hf .. 64hf + 31] (block 0), [.. + 63] (block 1); qh[32hf ..]
    q6_run16(sb + 64 * hf, *(uint32_t(*)[4])&l0[0]);
    q6_run16(sb + 64 * hf + 16, *(uint32_t(*)[4])&l0[4]);
    q6_run16(sb + 128 + 32 * hf, *(uint32_t(*)[4])&qh[0]);
    q6_run16(sb + 128 + 32 * hf + 16, *(uint32_t(*)[4])&qh[4]);
    uint32_t l1[8];
    q6_run16(sb + 64 * hf + 32, *(uint32_t(*)[4])&l1[0]);
    q6_run16(sb + 64 * hf + 48, *(uint32_t(*)[4])&l1[4]);
    const uint32_t shq = 4 * (uint32_t)(q & 1);  // nibble of both sub-blocks: j0 / 2
    const uint16_t *s16 = (const uint16_t *)(sb + 192 + 8 * hf + 2 * j0);
    const uint32_t sc4 = (uint32_t)s16[0] | ((uint32_t)s16[1] << 16);
    const uint32_t d = *(const uint16_t *)(sb + 208);
    uint32_t rec[16];
#pragma unroll
    for (int h = 0; h < 2; h++) {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint32_t *ql = s ? l1 : l0;
            const uint32_t shh = 2 * (uint32_t)(j0 + s);
            uint32_t hb = 0;
#pragma unroll
            for (int j = 0; j < 2; j++) {
                // dwords of weights 8h + 4j .. (first k-step) and 16 + 8h + 4j .. (second)
                const uint32_t a = ql[2 * h + j], b = ql[4 + 2 * h + j];
                rec[4 * h + 2 * s + j] = ((a >> shq) & 0x0F0F0F0Fu) | (((b >> shq) & 0x0F0F0F0Fu) << 4);
                hb |= ((qh[2 * h + j] >> shh) & 0x03030303u) << (4 * j);
                hb |= ((qh[4 + 2 * h + j] >> shh) & 0x03030303u) << (4 * j + 2);
            }
            rec[8 + 4 * h + s] = hb;
        }
        rec[8 + 4 * h + 2] = sc4;
        rec[8 + 4 * h + 3] = d;
    }
    uint4 *o = out + t * 4;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = make_uint4(rec[4 * i], rec[4 * i + 1], rec[4 * i + 2], rec[4 * i + 3]);
}

// ---- the second tiling: 64 x 256 workgroup tiles, weights straight into registers ----
//
// A workgroup takes 64 rows and 256 columns; wave w takes columns 64 w ..
// 64 w + 63 of them and all 64 rows (2 x 2 tiles of 32 x 32).  The four
// waves share one copy of the activation halves in LDS, staged S blocks at a
// time (registers -> LDS, one barrier per stage).  Each lane loads the weight
// words of its own columns straight into registers, one stage ahead (lane
// (c, h) of a 32 x 32 tile holds B[k][c] for k = 8h .. 8h + 7 of each
// 16-column step: Q4_0 / Q4_K the low nibbles of qs[8h .. 8h + 7] for the
// first step and their high nibbles for the second, Q8_0 qs[8h ..] and
// qs[16 + 8h ..], repacked Q6_K the same nibbles with their high bits beside
// them, F16 the row's own values), so the weights take no LDS traffic and no
// barrier.  The arithmetic is the first tiling's: per 32-block four MFMAs
// give C = sum_k (xh + xl) * w, folded in block order by
// acc = fmaf(scale, C, acc) (Q4_K: then acc = fmaf(-dmin*m, sum x, acc);
// Q6_K: a C and an fmaf per 16-k step, with its group's scale).
//
// Work is dealt by stages, not by tiles (a "stream-K" split), one row of
// tiles at a time: in row tile r, column tile c's stage s is item c * nst + s
// of the row's U = nct * nst, and of the row's Gr workgroups the i-th takes
// items [i U / Gr, (i + 1) U / Gr), so every workgroup runs the same number of
// stages to within one, whatever the tile count.  Workgroup w = i * ntm + r:
// the ntm workgroups with the same i walk the same column tiles and blocks in
// step on one XCD, so each weight word is fetched once for all of them, as in
// a tile-per-workgroup launch.  A range that covers a whole tile stores it
// directly.  Otherwise the range's share of the tile is a part: the workgroup
// stores its unscaled accumulators, device-scope, into its own slot (2 w for
// the first tile of its range, 2 w + 1 for the last), and counts itself on the
// tile's counter; the last of the tile's workgroups to arrive adds the parts
// in range order, scales and stores.  The result then depends on where the
// ranges cut the tiles (a different fp32 summation), which depends on Gr and
// the launch's shape.

constexpr int kX2MinStages = 8;      // the fewest stages of a part
constexpr int kX2MaxSplit = 4;       // workgroups per tile at most (on average)
constexpr int kX2DevScope = 16;      // sc1: device-scope store / device-coherent load
constexpr int kX2Counters = 16384;   // tile counters of the split form
constexpr uint32_t kX2OutOfRange = 0x80000000u;  // a buffer offset past any range: reads zeros

struct X2Args {
    float *Y[kExactMats];
    const uint8_t *W[kExactMats];    // block streams or f16 rows [N_i][K]
    int n_end[kExactMats];           // prefix sums of N_i; unused entries INT_MAX
    const _Float16 *Ah, *Al;         // activation halves [M][K]
    const float *Sx;                 // [M][K/32] block sums of the split rows (Q4_K)
    const float *Rs;                 // [M] row scales
    const float *R;                  // one matrix only: Y = R + product (may alias Y)
    float *part;                     // [2 G][64 x 256] part slots (split launches)
    uint32_t *cnt;                   // [tiles] arrival counters, zero between launches (split launches)
    int M, N, nb, ntm, tiles, nst;   // nst: stages per tile
    int gr;                          // workgroups per row of tiles
    int xi;                          // ranges are whole parts of tiles: part p's ranges share an XCD
};

// First item of the i-th range of a row, and the range that holds item x.
__device__ __forceinline__ int64_t x2_start(int i, int64_t U, int G) { return (int64_t)i * U / G; }
__device__ __forceinline__ int x2_owner(int64_t x, int64_t U, int G) { return (int)(((x + 1) * G - 1) / U); }

template <int S>
struct X2Geo {
    static constexpr int RB = S * 64 + 16;         // LDS bytes per row of one half (S blocks of 32 f16 + pad)
    static constexpr int HALF = 64 * RB;
    static constexpr int SX = 2 * HALF;            // fp32 [S][64]: the rows' block sums (Q4_K)
    static constexpr int STAGE = (SX + S * 64 * 4 + 255) & ~255;
    static constexpr int LDS = 2 * STAGE;
};

// Weight words of one block for one lane and one 32-column tile, as loaded.
// The weights are read through a buffer resource over the lane's matrix: the
// lane's row offset (plus 8 h) is the per-lane offset, fixed for the launch,
// and the block's offset is a wave-uniform scalar.  With an even number of
// blocks per row every Q4_0 / Q8_0 row starts 4-byte aligned, so block b sits
// 2 (b & 1) bytes into its first dword: the window starts there rounded down,
// and its realignment is a constant per unrolled block (none for odd b).
// The resource's size bounds the reads: a block past the last row's end
// reads zeros (its scale is then zero anyway).
template <int WF>
struct X2Raw;
template <>
struct X2Raw<EW_Q4_0> {
    v4u w;             // from the block's start rounded down, plus 8 h: qs[8h .. 8h + 7] at byte 2 + 2(b & 1);
                       // for h = 0 the window also holds d (bytes 0-1 or 2-3); the 16-byte load keeps each
                       // window in one aligned register quad
};
template <>
struct X2Raw<EW_Q8_0> {
    v4u w, v;          // the two 8-byte runs qs[8h ..] and qs[16 + 8h ..], same windows (h = 0: d too)
};

// The block scale d of lane (c, 0) in both lanes (c, 0) and (c, 1): the h = 1
// windows start 8 bytes into the block, so they take it from the h = 0 lane
// (v_permlane32_swap: lanes 32..63 of the first result are lanes 0..31 of x).
template <int P>
__device__ __forceinline__ uint32_t x2_scale_bits(uint32_t w0)
{
    const uint32_t x = P ? (w0 >> 16) : (w0 & 0xFFFFu);
    return __builtin_amdgcn_permlane32_swap(x, x, false, false)[0];
}
// Q4_K: a stage (sub-blocks j and j + 1, j even, of a superblock) in three
// loads: the superblock's 16-byte header (d, dmin, the 12 scale bytes) and,
// for each sub-block, the lane's 8 qs bytes 8h .. 8h + 7 of its 16 (weights
// k = 8h .. 8h + 7 in the low nibbles and 16 + 8h .. in the high ones,
// quant.c's layout, the same as a Q4_0 block's).
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
template <>
struct X2Raw<EW_Q4_K> {
    v4u hd;
    v2u q0, q1;
};
template <>
struct X2Raw<EW_F16> {
    v4u s0, s1;        // k = 8h .. 8h+7 and 16 + 8h .. 16 + 8h + 7
};
// Q6_K repacked (q6r_repack_k): a stage's record pieces of lane half h,
// the nibble words at 16h and {high bits of both blocks, scales, d} at 32 + 16h.
template <>
struct X2Raw<EW_Q6R> {
    v4u n, m;
};

// Block b of the lane's row (vo: the row's byte offset within the matrix,
// plus 8 h for the block formats, 16 h for F16).  P = b & 1 (block formats).
template <int WF, int P>
__device__ __forceinline__ X2Raw<WF> x2_fetch(__amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t vd, int b)
{
    X2Raw<WF> x;
    if constexpr (WF == EW_Q4_0) {
        const int so = 18 * b - 2 * P;
        x.w = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, so, 0));
    } else if constexpr (WF == EW_Q8_0) {
        const int so = 34 * b - 2 * P;
        x.w = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, so, 0));
        x.v = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, so + 16, 0));
    } else if constexpr (WF == EW_Q6R) {
        // b even: the stage's record; vo the row's records + 16 h
        const int so = 32 * b;
        x.n = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, so, 0));
        x.m = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, so + 32, 0));
    } else if constexpr (WF == EW_Q4_K) {
        // b even: the stage's first sub-block; vd the row, vo the row + 16 h
        const int sb = 144 * (b >> 3), qo = sb + 16 + 16 * (b & 7);
        x.hd = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vd, sb, 0));
        x.q0 = __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(r, (int)vo, qo, 0));
        x.q1 = __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(r, (int)vo, qo + 16, 0));
    } else {
        x.s0 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, 64 * b, 0));
        x.s1 = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, 64 * b + 32, 0));
    }
    return x;
}

// Sub-block j (the stage's first when e = 0, second when e = 1) of the stage
// held in x: both 16-k steps' B operands (q, exact in f16), d * sc and
// dmin * m (exact in fp32: 11-bit times 6-bit), zero past the part.
__device__ __forceinline__ void x2_unpack_q4_k(const X2Raw<EW_Q4_K> &x, int e, uint32_t j, bool live, v8h &b0,
                                               v8h &b1, float &dsc, float &dmn)
{
    const v2u q = e ? x.q1 : x.q0;
    uint32_t lo[4], hi[4];
    nibbles_f16(q.x, (_Float16)0.0f, &lo[0], &hi[0]);
    nibbles_f16(q.y, (_Float16)0.0f, &lo[2], &hi[2]);
    b0 = __builtin_bit_cast(v8h, v4u{lo[0], lo[1], lo[2], lo[3]});
    b1 = __builtin_bit_cast(v8h, v4u{hi[0], hi[1], hi[2], hi[3]});
    uint32_t sc, mn;
    q4_k_scale_min(x.hd.y, x.hd.z, x.hd.w, j, sc, mn);
    const uint32_t dd = x.hd.x & (0u - (uint32_t)live);
    dsc = half_bits_to_float(dd) * (float)sc;
    dmn = half_bits_to_float(dd >> 16) * (float)mn;
}

// Block s (0, 1) of the Q6_K stage held in x: both 16-k steps' B operands
// (q - 32, exact in f16) and their group scales d * sc (exact in fp32:
// 11-bit times 8-bit, as the first tiling forms them), zero past the part.
__device__ __forceinline__ void x2_unpack_q6r(const X2Raw<EW_Q6R> &x, int s, bool live, v8h &b0, v8h &b1,
                                              float &sc0, float &sc1)
{
    const uint32_t hb = s ? x.m.y : x.m.x;
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const uint32_t w = x.n[2 * s + j], hj = hb >> (4 * j);
        const uint32_t t0 = (w & 0x0F0F0F0Fu) | ((hj & 0x03030303u) << 4);
        const uint32_t t1 = ((w >> 4) & 0x0F0F0F0Fu) | (((hj >> 2) & 0x03030303u) << 4);
        lo[2 * j] = f16_pair(t0, 0x04010400u, (_Float16)-1056.0f);  // 1024 + q - 1056 = q - 32
        lo[2 * j + 1] = f16_pair(t0, 0x04030402u, (_Float16)-1056.0f);
        hi[2 * j] = f16_pair(t1, 0x04010400u, (_Float16)-1056.0f);
        hi[2 * j + 1] = f16_pair(t1, 0x04030402u, (_Float16)-1056.0f);
    }
    b0 = __builtin_bit_cast(v8h, v4u{lo[0], lo[1], lo[2], lo[3]});
    b1 = __builtin_bit_cast(v8h, v4u{hi[0], hi[1], hi[2], hi[3]});
    const float d = half_bits_to_float(x.m.w & (0u - (uint32_t)live));
    const uint32_t sc = x.m.z >> (16 * s);
    sc0 = d * (float)(int8_t)(sc & 0xFFu);
    sc1 = d * (float)(int8_t)((sc >> 8) & 0xFFu);
}

// The B operands of both 16-k steps and the block's scale; live: the block
// is inside the part (else the scale is zero).
template <int WF, int P>
__device__ __forceinline__ void x2_unpack(const X2Raw<WF> &x, bool live, v8h &b0, v8h &b1, float &sc)
{
    uint32_t lo[4], hi[4];
    // the loads' unused last dwords count as read here: otherwise their
    // registers look free at once and the next write to one of them waits
    // for the load in flight
    if constexpr (WF == EW_Q4_0) asm volatile("" ::"v"(x.w[3]));
    if constexpr (WF == EW_Q8_0) asm volatile("" ::"v"(x.w[3]), "v"(x.v[3]));
    if constexpr (WF == EW_Q4_0) {
        // qs[8h ..] at byte 2 of the window (even b) or 4 (odd b)
        const uint32_t q0 = P ? x.w[1] : __builtin_amdgcn_alignbyte(x.w[1], x.w[0], 2);
        const uint32_t q1 = P ? x.w[2] : __builtin_amdgcn_alignbyte(x.w[2], x.w[1], 2);
        nibbles_f16(q0, (_Float16)-8.0f, &lo[0], &hi[0]);
        nibbles_f16(q1, (_Float16)-8.0f, &lo[2], &hi[2]);
        // a mask, not a select: the swap stays outside any branch
        sc = half_bits_to_float(x2_scale_bits<P>(x.w[0]) & (0u - (uint32_t)live));
    } else if constexpr (WF == EW_Q8_0) {
        const uint32_t q0 = P ? x.w[1] : __builtin_amdgcn_alignbyte(x.w[1], x.w[0], 2);
        const uint32_t q1 = P ? x.w[2] : __builtin_amdgcn_alignbyte(x.w[2], x.w[1], 2);
        const uint32_t q4 = P ? x.v[1] : __builtin_amdgcn_alignbyte(x.v[1], x.v[0], 2);
        const uint32_t q5 = P ? x.v[2] : __builtin_amdgcn_alignbyte(x.v[2], x.v[1], 2);
        int8s_f16(q0, &lo[0]);
        int8s_f16(q1, &lo[2]);
        int8s_f16(q4, &hi[0]);
        int8s_f16(q5, &hi[2]);
        // a mask, not a select: the swap stays outside any branch
        sc = half_bits_to_float(x2_scale_bits<P>(x.w[0]) & (0u - (uint32_t)live));
    } else {
        b0 = __builtin_bit_cast(v8h, x.s0);
        b1 = __builtin_bit_cast(v8h, x.s1);
        sc = 1.f;
        return;
    }
    b0 = __builtin_bit_cast(v8h, v4u{lo[0], lo[1], lo[2], lo[3]});
    b1 = __builtin_bit_cast(v8h, v4u{hi[0], hi[1], hi[2], hi[3]});
}

template <int WF, int S>
__global__ __launch_bounds__(256, 2) void gemm_exact2_k(X2Args a)
{
    static_assert(S % 2 == 0, "blocks of a stage alternate in parity: S even");
    using G = X2Geo<S>;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t last;
    __shared__ __align__(16) float rs_l[64];  // the tile's row scales
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);  // uniform: the weight resource stays scalar
    const int nb = a.nb;

    // workgroup g -> w = i * ntm + r.  The ntm row tiles of one range i
    // (which walk the same weights in step) run on one XCD (g mod 8 under
    // round-robin dispatch).  The XCD takes a contiguous run of ranges, or,
    // when every tile splits into the same whole parts, the ranges i = x
    // (mod 8): then with a part count dividing 8 an XCD holds one part of
    // each of its tiles, and reads that part of the activations only.
    const int NG = (int)gridDim.x, g = blockIdx.x;
    const int nst = a.nst, ntm = a.ntm, Gr = a.gr;
    const int w = (NG & 7) ? g
                  : a.xi   ? ((g & 7) + 8 * ((g >> 3) / ntm)) * ntm + (g >> 3) % ntm
                           : (g & 7) * (NG >> 3) + (g >> 3);
    const int ri = w / ntm, rt = w - ri * ntm;  // range i of row tile r
    const int64_t U = (int64_t)(a.tiles / ntm) * nst;
    const int64_t ibeg = x2_start(ri, U, Gr), iend = x2_start(ri + 1, U, Gr);
    const int cfirst = (int)(ibeg / nst);  // the first column tile of the range

    // one pass per tile the range touches (uniform)
    for (int64_t i0 = ibeg; i0 < iend;) {
    // the thread index as an opaque value of the pass: per-lane addresses are
    // then computed in each pass, not kept live through every pass's loop
    int tid_v = (int)threadIdx.x;
    asm volatile("" : "+v"(tid_v));
    const int tid = tid_v, lane = tid & 63, h = lane >> 5, c32 = lane & 31;
    const int ct = (int)(i0 / nst);
    const int s0 = (int)(i0 - (int64_t)ct * nst);
    const int s1 = (int)min((int64_t)nst, (int64_t)s0 + (iend - i0));
    i0 += s1 - s0;
    const int t = ct * ntm + rt;
    const int m0 = (t % a.ntm) * 64, n0 = (t / a.ntm) * 256 + 64 * wave;
    const int kb0 = s0 * S;  // even
    const int kb1 = min(nb, s1 * S);

    // this wave's 64 columns lie in one matrix (n_end multiples of 64); in
    // the last column tile a wave may start at or past N: it loads in-bounds
    // rows of the last matrix and stores nothing
    const bool live = n0 < a.N;
    const int nc = min(n0, a.N - 1);
    const int sel = (nc >= a.n_end[0]) + (nc >= a.n_end[1]);
    const uint8_t *Wm = sel == 2 ? a.W[2] : sel == 1 ? a.W[1] : a.W[0];
    float *Ym = sel == 2 ? a.Y[2] : sel == 1 ? a.Y[1] : a.Y[0];
    const int nbase = sel == 2 ? a.n_end[1] : sel == 1 ? a.n_end[0] : 0;
    const int Nm = (sel == 2 ? a.n_end[2] : sel == 1 ? a.n_end[1] : a.n_end[0]) - nbase;
    const int nl = nc - nbase;  // the wave's first column in its matrix (clamped)
    // bytes of a row: 18 / 34 per Q4_0 / Q8_0 block, 144 per 8 Q4_K sub-blocks, 64 per F16 block,
    // 64 per repacked Q6_K stage
    const uint32_t rowb = WF == EW_Q4_K ? (uint32_t)(nb >> 3) * 144u
                                        : (uint32_t)nb * (WF == EW_Q4_0   ? 18u
                                                          : WF == EW_Q8_0 ? 34u
                                                          : WF == EW_Q6R  ? 32u
                                                                          : 64u);
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)Wm, (short)0, (int)((uint32_t)Nm * rowb), kXBufWord3);
    uint32_t vo[2], vd[2];
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
        vd[ni] = (uint32_t)min(nl + 32 * ni + c32, Nm - 1) * rowb;
        vo[ni] = vd[ni] + (WF == EW_F16 || WF == EW_Q6R ? 16u : 8u) * (uint32_t)h;
    }

    // activation staging: thread tid moves piece tid + 256 i of each half,
    // row (tid + 256 i) / 4S, 16-byte piece (tid + 256 i) % 4S
    constexpr int NP = 4 * S;  // pieces per row and half in a stage
    const uint32_t abytes = (uint32_t)((int64_t)a.M * nb * 64);
    const __amdgpu_buffer_rsrc_t rah = __builtin_amdgcn_make_buffer_rsrc((void *)a.Ah, (short)0, (int)abytes, kXBufWord3);
    const __amdgpu_buffer_rsrc_t ral = __builtin_amdgcn_make_buffer_rsrc((void *)a.Al, (short)0, (int)abytes, kXBufWord3);
    uint32_t aoff[S];
    int ablk[S];
    uint32_t lw[S];
#pragma unroll
    for (int i = 0; i < S; i++) {
        const int pc = tid + 256 * i, r = pc / NP, c = pc % NP;
        aoff[i] = (uint32_t)min(m0 + r, a.M - 1) * (uint32_t)(nb * 64) + (uint32_t)(c & 3) * 16u;
        ablk[i] = c >> 2;
        lw[i] = (uint32_t)(r * G::RB + c * 16);
    }
    // Q4_K: the rows' block sums, thread tid < 64 S: row tid % 64, block tid / 64
    const __amdgpu_buffer_rsrc_t rsx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)a.Sx, (short)0, WF == EW_Q4_K ? (int)((uint32_t)a.M * (uint32_t)nb * 4u) : 0, kXBufWord3);
    const uint32_t sxo = (uint32_t)min(m0 + (tid & 63), a.M - 1) * (uint32_t)nb;
    const int sxb = (tid >> 6) & (S - 1);
    v4u sah[S], sal[S];
    float sxv = 0.f;
    auto fetch_a = [&](int st) {
        const int kb = kb0 + st * S;
#pragma unroll
        for (int i = 0; i < S; i++) {
            const uint32_t o = aoff[i] + (uint32_t)min(kb + ablk[i], kb1 - 1) * 64u;
            sah[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rah, (int)o, 0, 0));
            sal[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(ral, (int)o, 0, 0));
        }
        if constexpr (WF == EW_Q4_K)
            sxv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                rsx, (int)((sxo + (uint32_t)min(kb + sxb, kb1 - 1)) * 4u), 0, 0));
    };
    auto stash_a = [&](int buf) {
        uint8_t *base = lds + buf * G::STAGE;
#pragma unroll
        for (int i = 0; i < S; i++) {
            *(v4u *)(base + lw[i]) = sah[i];
            *(v4u *)(base + G::HALF + lw[i]) = sal[i];
        }
        if constexpr (WF == EW_Q4_K)
            if (tid < 64 * S) ((float *)(base + G::SX))[tid] = sxv;  // [block][row]
    };

    v16f acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;

    // F16 has no scale to zero a block past the part with: its block index
    // is clamped instead (no alignment depends on it)
    auto wblk = [&](int b) { return WF == EW_F16 ? min(b, kb1 - 1) : b; };
    const int nsg = (kb1 - kb0 + S - 1) / S;  // stages of this pass
    // the weight words of a stage's S blocks, fetched one stage ahead
    // (Q4_K, Q6R: one slot per stage, ring[0])
    constexpr bool kStageSlot = WF == EW_Q4_K || WF == EW_Q6R;
    X2Raw<WF> ring[S][2];
#pragma unroll
    for (int s = 0; s < (kStageSlot ? 1 : S); s++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
            if (s & 1) ring[s][ni] = x2_fetch<WF, 1>(rw, vo[ni], vd[ni], wblk(kb0 + s));
            else ring[s][ni] = x2_fetch<WF, 0>(rw, vo[ni], vd[ni], wblk(kb0 + s));
        }
    __syncthreads();  // the previous pass's readers of rs_l are done
    if (tid < 64) rs_l[tid] = a.Rs[min(m0 + tid, a.M - 1)];
    fetch_a(0);
    stash_a(0);
    fetch_a(1);
    __syncthreads();
    float mneg[2] = {0.f, 0.f};  // Q4_K: -dmin * m of the lane's column and sub-block (stage start + h)
    for (int st = 0; st < nsg; st++) {
        const uint8_t *base = lds + (st & 1) * G::STAGE;
        // stage st + 1 into the other buffer (free: every wave passed the
        // barrier after stage st - 1), then fetch stage st + 2: both a whole
        // stage before their use
        stash_a((st + 1) & 1);
        fetch_a(st + 2);
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int b = kb0 + st * S + s;
            // this block's weight operands, then its ring slot fetches block b + S
            v8h b0[2], b1[2];
            float sc[2], sc1[2];
            if constexpr (WF == EW_Q6R) {
                // block s of the stage's record in ring[0]: a scale per 16-k step
#pragma unroll
                for (int ni = 0; ni < 2; ni++) {
                    x2_unpack_q6r(ring[0][ni], s, b < kb1, b0[ni], b1[ni], sc[ni], sc1[ni]);
                    if (s == S - 1) ring[0][ni] = x2_fetch<WF, 0>(rw, vo[ni], vd[ni], b + 1);
                }
            } else if constexpr (WF == EW_Q4_K) {
                // sub-block b of the stage in ring[0]; its min term goes to
                // the stage's fp32 MFMA below (lane h: sub-block b - s + h)
#pragma unroll
                for (int ni = 0; ni < 2; ni++) {
                    float dmn;
                    x2_unpack_q4_k(ring[0][ni], s, (uint32_t)(b & 7), b < kb1, b0[ni], b1[ni], sc[ni], dmn);
                    if (s == h) mneg[ni] = -dmn;  // a select: h is the lane's half
                    if (s == S - 1) ring[0][ni] = x2_fetch<WF, 0>(rw, vo[ni], vd[ni], b + 1);
                }
            } else {
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                if (s & 1) {
                    x2_unpack<WF, 1>(ring[s][ni], b < kb1, b0[ni], b1[ni], sc[ni]);
                    ring[s][ni] = x2_fetch<WF, 1>(rw, vo[ni], vd[ni], wblk(b + S));
                } else {
                    x2_unpack<WF, 0>(ring[s][ni], b < kb1, b0[ni], b1[ni], sc[ni]);
                    ring[s][ni] = x2_fetch<WF, 0>(rw, vo[ni], vd[ni], wblk(b + S));
                }
            }
            }
            const bool bl = b < kb1;  // F16: a block past the part adds nothing
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                const uint8_t *ra = base + (32 * mi + c32) * G::RB + s * 64 + 16 * h;
                const v8h ah0 = *(const v8h *)ra, ah1 = *(const v8h *)(ra + 32);
                const v8h al0 = *(const v8h *)(ra + G::HALF), al1 = *(const v8h *)(ra + G::HALF + 32);
#pragma unroll
                for (int ni = 0; ni < 2; ni++) {
                    if constexpr (WF == EW_F16) {
                        if (bl) {
                            acc[mi][ni] = mfma16(ah0, b0[ni], acc[mi][ni]);
                            acc[mi][ni] = mfma16(ah1, b1[ni], acc[mi][ni]);
                            acc[mi][ni] = mfma16(al0, b0[ni], acc[mi][ni]);
                            acc[mi][ni] = mfma16(al1, b1[ni], acc[mi][ni]);
                        }
                    } else if constexpr (WF == EW_Q6R) {
                        // the first tiling's Q6_K order: each 16-k step's C, then its group scale
                        const v16f zero = {};
                        v16f c = mfma16(al0, b0[ni], mfma16(ah0, b0[ni], zero));
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[mi][ni][r] = __builtin_fmaf(sc[ni], c[r], acc[mi][ni][r]);
                        c = mfma16(al1, b1[ni], mfma16(ah1, b1[ni], zero));
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[mi][ni][r] = __builtin_fmaf(sc1[ni], c[r], acc[mi][ni][r]);
                    } else {
                        const v16f zero = {};
                        v16f c = mfma16(ah0, b0[ni], zero);
                        c = mfma16(ah1, b1[ni], c);
                        c = mfma16(al0, b0[ni], c);
                        c = mfma16(al1, b1[ni], c);
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[mi][ni][r] = __builtin_fmaf(sc[ni], c[r], acc[mi][ni][r]);
                    }
                }
            }
        }
        if constexpr (WF == EW_Q4_K) {
            // the stage's min terms, sum over its two sub-blocks j of
            // (-dmin m_j)[n] * (sum x)[m][j], on one fp32 MFMA per tile:
            // A[m][j] = the row's block sum (lane (c, h): row c, sub-block h),
            // B[j][n] = -dmin m_j of column n (lane (c, h): column c, sub-block h)
            const float *sxl = (const float *)(base + G::SX);
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                const float av = sxl[64 * h + 32 * mi + c32];
#pragma unroll
                for (int ni = 0; ni < 2; ni++)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, mneg[ni], acc[mi][ni], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // lane (c, h) holds rows 4h + 8q + j (register 4q + j) of column c of each tile
    bool store = s0 == 0 && s1 == nst;
    if (!store) {
        // a part: store it in this range's slot, count, and the last of the
        // tile's ranges to arrive adds the parts in range order.  The slots
        // (2 G of 64 KB, far below 2^31 bytes) bound the resource, so an
        // offset of kX2OutOfRange reads zeros.
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
            (void *)a.part, (short)0, (int)((uint32_t)NG * 131072u), kXBufWord3);
        auto word = [&](int sl, int mi, int ni, int q) {
            return (uint32_t)sl * 65536u + (uint32_t)((((wave * 4 + 2 * mi + ni) * 4 + q) * 1024) + 16 * lane);
        };
        const int mine = 2 * w + (ct == cfirst ? 0 : 1);
        const int64_t it = (int64_t)ct * nst;
        const int jf = x2_owner(it, U, Gr), jl = x2_owner(it + nst - 1, U, Gr);
        const int nparts = jl - jf + 1;
        // every other range of the tile has already counted itself (at the
        // end of a range the tile's other parts were usually computed first,
        // at the start of the next ranges): this one is the last, and adds
        // its own part from registers instead of storing and reloading it.
        // Exactly one workgroup can see nparts - 1 before counting itself.
        if (tid == 0)
            last = nparts <= 4 &&
                   __hip_atomic_load(a.cnt + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(nparts - 1);
        __syncthreads();
        const bool early = last;
        if (!early) {
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int ni = 0; ni < 2; ni++)
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float4 v = {acc[mi][ni][4 * q], acc[mi][ni][4 * q + 1], acc[mi][ni][4 * q + 2],
                                          acc[mi][ni][4 * q + 3]};
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), rp,
                                                               (int)word(mine, mi, ni, q), 0, kX2DevScope);
                    }
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the stores have completed (device scope)
            __syncthreads();
            if (tid == 0) {
                const uint32_t old = __hip_atomic_fetch_add(a.cnt + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last = old == (uint32_t)(nparts - 1);
            }
            __syncthreads();
        }
        store = last;
        if (store) {
            if (tid == 0) __hip_atomic_store(a.cnt + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // up to four parts' words of one 32 x 32 tile in one batch of
            // loads (parts past the last read as zeros and are not added):
            // one round trip per batch, not one per part and word
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int ni = 0; ni < 2; ni++)
#pragma unroll 1
                    for (int jb = 0; jb < nparts; jb += 4) {
                        v4u wv[4][4];
#pragma unroll
                        for (int jj = 0; jj < 4; jj++) {
                            const int j = jf + jb + jj;
                            const int sl = 2 * (j * ntm + rt) + ((int)(x2_start(j, U, Gr) / nst) == ct ? 0 : 1);
                            // early: this range's own part (j == ri) is in acc, not in its slot
                            const bool ld = j <= jl && !(early && j == ri);
#pragma unroll
                            for (int q = 0; q < 4; q++)
                                wv[jj][q] = __builtin_bit_cast(
                                    v4u, __builtin_amdgcn_raw_buffer_load_b128(
                                             rp, ld ? (int)word(sl, mi, ni, q) : (int)kX2OutOfRange, 0, kX2DevScope));
                        }
#pragma unroll
                        for (int q = 0; q < 4; q++)
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                // the parts in range order (an early last's own part from
                                // its accumulators: nparts <= 4, a single batch)
                                const float own = acc[mi][ni][4 * q + e];
                                auto part = [&](int jj) {
                                    return early && jf + jb + jj == ri ? own : __uint_as_float(wv[jj][q][e]);
                                };
                                const float p0 = part(0);
                                float v = jb == 0 ? p0 : own + p0;
#pragma unroll
                                for (int jj = 1; jj < 4; jj++)
                                    if (jb + jj < nparts) v = v + part(jj);
                                acc[mi][ni][4 * q + e] = v;
                            }
                    }
        }
    }
    if (store) {
        // the residual of every output first, in one batch of loads (a load
        // between stores would wait for the stores issued before it as
        // well), then the stores.  Outputs of under 2^31 bytes go through
        // buffer resources: the lane's offset for row m0 + 4h (out of range
        // past the matrix's columns or for a wave without columns) plus a
        // wave-uniform row offset, no per-element address registers; rows
        // past M fall outside the resource.
        float rv[2][2][16];
        if ((int64_t)a.M * Nm < (1LL << 29)) {
            const int bytes = a.M * Nm * 4;
            const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc((void *)Ym, (short)0, bytes, kXBufWord3);
            const __amdgpu_buffer_rsrc_t rr =
                __builtin_amdgcn_make_buffer_rsrc((void *)(a.R ? a.R : Ym), (short)0, bytes, kXBufWord3);
            uint32_t vb[2];
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                const int n = nl + 32 * ni + c32;
                vb[ni] = live && n < Nm ? (uint32_t)(((m0 + 4 * h) * Nm + n) * 4) : kX2OutOfRange;
            }
            auto roff = [&](int mi, int q, int j) { return (32 * mi + 8 * q + j) * Nm * 4; };
            if (a.R) {
#pragma unroll
                for (int mi = 0; mi < 2; mi++)
#pragma unroll
                    for (int ni = 0; ni < 2; ni++)
#pragma unroll
                        for (int q = 0; q < 4; q++)
#pragma unroll
                            for (int j = 0; j < 4; j++)
                                rv[mi][ni][4 * q + j] = __builtin_bit_cast(
                                    float, __builtin_amdgcn_raw_buffer_load_b32(rr, (int)vb[ni], roff(mi, q, j), 0));
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    // rows 32 mi + 8 q + 4 h + j, j = 0..3: one LDS read
                    const float4 rs = *(const float4 *)(rs_l + 32 * mi + 8 * q + 4 * h);
                    const float rsj[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                    for (int ni = 0; ni < 2; ni++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int r = 4 * q + j;
                            const float y = acc[mi][ni][r] * rsj[j];  // a power of two: exact
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, a.R ? rv[mi][ni][r] + y : y),
                                                                  ry, (int)vb[ni], roff(mi, q, j), 0);
                        }
                }
        } else {
            if (a.R) {
#pragma unroll
                for (int mi = 0; mi < 2; mi++)
#pragma unroll
                    for (int ni = 0; ni < 2; ni++) {
                        const int n = min(nl + 32 * ni + c32, Nm - 1);
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int m = min(m0 + 32 * mi + (r & 3) + 4 * h + 8 * (r >> 2), a.M - 1);
                            rv[mi][ni][r] = a.R[(int64_t)m * Nm + n];
                        }
                    }
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 rs = *(const float4 *)(rs_l + 32 * mi + 8 * q + 4 * h);
                    const float rsj[4] = {rs.x, rs.y, rs.z, rs.w};
#pragma unroll
                    for (int ni = 0; ni < 2; ni++) {
                        const int n = nl + 32 * ni + c32;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int r = 4 * q + j;
                            const int m = m0 + 32 * mi + j + 4 * h + 8 * q;
                            if (live && m < a.M && n < Nm) {
                                const int64_t o = (int64_t)m * Nm + n;
                                const float y = acc[mi][ni][r] * rsj[j];  // a power of two: exact
                                Ym[o] = a.R ? rv[mi][ni][r] + y : y;
                            }
                        }
                    }
                }
        }
    }
    }  // passes
}

template <int WF, int WM, int WN, int S, int OCC, int RD>
void launch_exact(ExactArgs a)
{
    using G = XGeo<WM, WN, S>;
    a.ntm = (a.M + G::TM - 1) / G::TM;
    a.tiles = a.ntm * ((a.N + G::TN - 1) / G::TN);
    auto kern = gemm_exact_k<WF, WM, WN, S, OCC, RD>;
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

// Register stages in flight: two take 512x11008x4096 from 191 to 167 us and
// 512x4096x11008 from 228 to 182 us; three or four measured the same, and at
// four the Q8_0, Q4_K and panel variants of the 128 x 128 tile spill.
constexpr int kExactRing = 2;

// 128 x 128 workgroup tiles (64 x 64 per wave, one block per stage) when there
// are at least as many as CUs; otherwise 64 x 64 (32 x 32 per wave, two
// blocks per stage) for four times the workgroups.
template <int WF>
void launch_exact_for(const ExactArgs &a)
{
    const long tiles128 = (long)((a.M + 127) / 128) * ((a.N + 127) / 128);
    if (tiles128 >= num_cus()) launch_exact<WF, 2, 2, 1, 2, kExactRing>(a);
    else launch_exact<WF, 1, 1, 2, 2, kExactRing>(a);
}

uint32_t *g_x2_cnt = nullptr;  // tile counters of the split form, zero between launches

// The second tiling: about 2 workgroups per CU (both resident), the same
// number per row of tiles, share the stages evenly, with ranges of at least
// kX2MinStages stages and at most about kX2MaxSplit workgroups per tile; a
// launch whose ranges all fall on tile boundaries needs no part slots or
// counters.
template <int WF, int S>
void launch_exact2(X2Args a)
{
    using G = X2Geo<S>;
    a.ntm = (a.M + 63) / 64;
    a.tiles = a.ntm * ((a.N + 255) / 256);
    a.nst = (a.nb + S - 1) / S;
    const int nct = a.tiles / a.ntm;
    const int64_t U = (int64_t)nct * a.nst;  // items of a row of tiles
    int64_t gr = std::max(1, 2 * num_cus() / a.ntm);
    gr = std::min(gr, U / kX2MinStages);
    gr = std::max<int64_t>(1, std::min(gr, (int64_t)kX2MaxSplit * nct));
    if (!g_x2_cnt || a.tiles > kX2Counters) gr = nct;  // whole tiles only
    a.gr = (int)gr;
    const int64_t NG = (int64_t)a.ntm * gr;
    a.xi = gr % 8 == 0 && U % gr == 0 && a.nst % (U / gr) == 0;
    void *pws = nullptr;
    bool own = false;
    if (U % gr != 0 || (U / gr) % a.nst != 0) {
        // some range cuts a tile: part slots (two a workgroup) and counters
        const size_t bytes = (size_t)NG * 2 * 64 * 256 * 4;
        pws = workspace(2, bytes);
        own = pws == nullptr;
        if (own) HOLO_CHECK(hipMallocAsync(&pws, bytes, stream()));
        if (!pws) return;
        a.part = (float *)pws;
        a.cnt = g_x2_cnt;
    }
    auto kern = gemm_exact2_k<WF, S>;
    static bool attr = false;
    if (!attr) {
        HOLO_CHECK(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS));
        attr = true;
    }
    launch_timed(kern, dim3((unsigned)NG), dim3(256), G::LDS, a);
    HOLO_LAUNCH_CHECK();
    if (own) HOLO_CHECK(hipFreeAsync(pws, stream()));
}

// The first tiling only (HOLO_EXACT_V1=1): for same-box comparisons
static bool exact_v1()
{
    static const bool on = getenv("HOLO_EXACT_V1") != nullptr;
    return on;
}

// Q6_K through the integer panel instead of unpacked in the staging
// (HOLO_EXACT_Q6K_PANEL=1)
static bool q6_panel()
{
    static const bool on = getenv("HOLO_EXACT_Q6K_PANEL") != nullptr;
    return on;
}

int exact_kind(int type)
{
    switch (type) {
    case HOLO_TYPE_Q4_0: return EW_Q4_0;
    case HOLO_TYPE_Q8_0: return EW_Q8_0;
    case HOLO_TYPE_Q4_K: return EW_Q4_K;
    case HOLO_TYPE_Q6_K: return q6_panel() ? EW_P16 : exact_v1() ? EW_Q6_K : EW_Q6R;
    case HOLO_TYPE_F16: return EW_F16;
    default: return -1;
    }
}

}  // namespace

bool exact_init()
{
    if (g_x2_cnt) return true;
    if (hipMalloc((void **)&g_x2_cnt, kX2Counters * sizeof(uint32_t)) != hipSuccess) {
        (void)hipGetLastError();
        g_x2_cnt = nullptr;
        return false;
    }
    return hipMemset(g_x2_cnt, 0, kX2Counters * sizeof(uint32_t)) == hipSuccess &&
           hipDeviceSynchronize() == hipSuccess;
}

// ---- Q6_K matrices repacked once (holo_prefill_prepare) ----
// The repacked copy of each registered matrix, keyed by its device address;
// the caller keeps the matrix unchanged until it releases it.
namespace {
struct PreparedQ6 {
    int N, K;
    void *rec;
};
std::mutex g_prep_mu;
std::unordered_map<const void *, PreparedQ6> g_prep;

const void *prepared_q6r(const void *W, int N, int K)
{
    std::lock_guard<std::mutex> lk(g_prep_mu);
    const auto it = g_prep.find(W);
    return it != g_prep.end() && it->second.N == N && it->second.K == K ? it->second.rec : nullptr;
}

// Frees every registered copy (cuda_cleanup).
void prepared_release_all()
{
    std::lock_guard<std::mutex> lk(g_prep_mu);
    for (auto &e : g_prep) (void)hipFree(e.second.rec);
    g_prep.clear();
}

// W [N][K] Q6_K (K a multiple of 256, W 2-byte aligned) into records [N][K/64][64 B] at out
void q6r_repack(void *out, const void *W, int N, int K)
{
    const int64_t nrec = (int64_t)N * (K / 256) * 4;
    hipLaunchKernelGGL(q6r_repack_k, dim3((unsigned)((nrec + 255) / 256)), dim3(256), 0, stream(), (uint4 *)out,
                       (const uint8_t *)W, nrec);
    HOLO_LAUNCH_CHECK();
}
}  // namespace

void exact_release()
{
    if (g_x2_cnt) (void)hipFree(g_x2_cnt);
    g_x2_cnt = nullptr;
    prepared_release_all();
}

// Takes the exact product: M >= 1, K whole blocks of the type (Q4_K, Q6_K: a
// multiple of 256) up to 16384, activations 16-byte aligned; the weight stream
// aligned as its loads need (Q4_0/Q8_0: 4 bytes, Q4_K: 16, Q6_K: 2, F16:
// 16).
bool exact_ok(int type, int K, const void *W)
{
    const uintptr_t w = (uintptr_t)W;
    if (K > 16384) return false;  // the activation split keeps a row in registers
    switch (type) {
    case HOLO_TYPE_Q4_0:
    case HOLO_TYPE_Q8_0: return K % 32 == 0 && K > 0 && (w & 3u) == 0;
    case HOLO_TYPE_Q4_K: return K % 256 == 0 && K > 0 && (w & 15u) == 0;
    case HOLO_TYPE_Q6_K: return K % 256 == 0 && K > 0 && (w & 1u) == 0;
    case HOLO_TYPE_F16: return K % 32 == 0 && K > 0 && (w & 15u) == 0;
    default: return false;
    }
}

// Y[i] = X . W[i]^T (or (silu(X) * U) . W[i]^T, plus R for one matrix) for
// nmat matrices sharing the activations; every type must pass exact_ok, and
// with several matrices of one type every N[i] must be a multiple of 128.
// Matrices of one type share a launch; the activation halves are built once.
void exact_product(float *const *Y, const void *const *W, const int *types, const int *N, int nmat, const float *X,
                   const float *U, const float *R, int M, int K, const float *NW, float eps)
{
    const int nb = K / 32;
    const size_t half = ((size_t)M * K * 2 + 255) & ~(size_t)255;
    const size_t sxb = ((size_t)M * nb * 4 + 255) & ~(size_t)255;
    const size_t abytes = 2 * half + sxb + (size_t)M * 4;
    void *aws = workspace(1, abytes);
    const bool own_a = aws == nullptr;
    if (own_a) HOLO_CHECK(hipMallocAsync(&aws, abytes, stream()));
    if (!aws) return;
    _Float16 *Ah = (_Float16 *)aws, *Al = (_Float16 *)((uint8_t *)aws + half);
    float *Sx = (float *)((uint8_t *)aws + 2 * half);
    float *Rs = (float *)((uint8_t *)aws + 2 * half + sxb);
    bool need_sx = false;
    size_t pbytes = 0;
    // each matrix's launch kind: Q6_K repacked for the second tiling unless
    // a mode asks for another form or the repacked matrix (N*K bytes) would
    // pass the 32-bit offsets
    int kinds[kExactMats];
    const void *PW[kExactMats] = {nullptr, nullptr, nullptr};
    const float *PS[kExactMats] = {nullptr, nullptr, nullptr};
    for (int i = 0; i < nmat; i++) {
        need_sx = need_sx || types[i] == HOLO_TYPE_Q4_K;
        kinds[i] = exact_kind(types[i]);
        if (kinds[i] == EW_Q6R && (int64_t)N[i] * K >= (1LL << 31)) kinds[i] = EW_Q6_K;
        if (kinds[i] == EW_P16) pbytes += (size_t)N[i] * K * 2 + (size_t)N[i] * (K / 16) * 4;
        if (kinds[i] == EW_Q6R) {
            PW[i] = prepared_q6r(W[i], N[i], K);  // repacked once by the caller's request
            if (!PW[i]) pbytes += ((size_t)N[i] * K + 255) & ~(size_t)255;
        }
    }
    // one workgroup per row, K <= 16384 (exact_ok): the row in registers
    auto split = [&](auto kern, int nt) {
        hipLaunchKernelGGL(kern, dim3(M), dim3(nt), 0, stream(), (uint2 *)Ah, (uint2 *)Al, need_sx ? Sx : nullptr,
                           Rs, X, U, NW, K, eps);
    };
    // the normed form keeps rms_norm_rows4_k's 256 threads (its sum of squares
    // in the same order); the others reduce only a maximum, so their threads
    // per row change no bit.  The long SwiGLU rows (g and u in registers) take
    // 512: 14.9 against 15.8 us at 512 x 11008; 512 or 1024 threads measured
    // level on the plain 4096-wide rows.
    const bool small = K <= 1024 * 4;
    if (NW) small ? split(xsplit_row_k<4, XS_NORM>, 256) : split(xsplit_row_k<16, XS_NORM>, 256);
    else if (U) small ? split(xsplit_row_k<2, XS_SWIGLU, 512>, 512) : split(xsplit_row_k<8, XS_SWIGLU, 512>, 512);
    else small ? split(xsplit_row_k<4, XS_PLAIN>, 256) : split(xsplit_row_k<16, XS_PLAIN>, 256);
    HOLO_LAUNCH_CHECK();
    // Q6_K matrices: repacked, or their integer panels and group scales
    void *pws = nullptr;
    bool own_p = false;
    if (pbytes) {
        pws = workspace(0, pbytes);
        own_p = pws == nullptr;
        if (own_p) HOLO_CHECK(hipMallocAsync(&pws, pbytes, stream()));
        if (!pws) return;
        size_t off = 0;
        for (int i = 0; i < nmat; i++) {
            if (kinds[i] == EW_Q6R) {
                if (PW[i]) continue;  // prepared
                void *p = (uint8_t *)pws + off;
                off += ((size_t)N[i] * K + 255) & ~(size_t)255;
                q6r_repack(p, W[i], N[i], K);
                PW[i] = p;
                continue;
            }
            if (kinds[i] != EW_P16) continue;
            _Float16 *p = (_Float16 *)((uint8_t *)pws + off);
            off += (size_t)N[i] * K * 2;
            float *ps = (float *)((uint8_t *)pws + off);
            off += (size_t)N[i] * (K / 16) * 4;
            const int64_t ntask = (int64_t)N[i] * (K / 256) * 4;
            hipLaunchKernelGGL(q6_k_int_panel_k, dim3((unsigned)((ntask + 255) / 256)), dim3(256), 0, stream(), p, ps,
                               (const uint8_t *)W[i], ntask);
            HOLO_LAUNCH_CHECK();
            PW[i] = p;
            PS[i] = ps;
        }
    }
    // one launch per weight kind, over that kind's matrices in order
    bool done[kExactMats] = {false, false, false};
    for (int i = 0; i < nmat; i++) {
        if (done[i]) continue;
        const int kind = kinds[i];
        ExactArgs a = {};
        int cnt = 0, acc = 0;
        const void *raw[kExactMats] = {W[i], W[i], W[i]};  // the matrices as given (EW_Q6R's fallback)
        for (int j = i; j < nmat; j++) {
            if (done[j] || kinds[j] != kind) continue;
            done[j] = true;
            acc += N[j];
            a.Y[cnt] = Y[j];
            raw[cnt] = W[j];
            a.W[cnt] = (const uint8_t *)(PW[j] ? PW[j] : W[j]);
            a.WS[cnt] = PS[j];
            a.n_end[cnt] = acc;
            cnt++;
        }
        for (int j = cnt; j < kExactMats; j++) {
            a.Y[j] = a.Y[0];
            a.W[j] = a.W[0];
            a.WS[j] = a.WS[0];
            a.n_end[j] = INT_MAX;
        }
        a.Ah = Ah;
        a.Al = Al;
        a.Sx = Sx;
        a.Rs = Rs;
        a.M = M;
        a.N = acc;
        a.nb = nb;
        a.R = (nmat == 1) ? R : nullptr;
        // the second tiling: Q4_0 and Q8_0 rows of an even block count (every
        // row 4-byte aligned), Q4_K, repacked Q6_K and F16 rows; with several
        // matrices every N but the last a multiple of 64 (a wave's 64 columns
        // in one matrix); each matrix under 2 GiB (32-bit offsets)
        bool x2 = !exact_v1() && (((kind == EW_Q4_0 || kind == EW_Q8_0) && nb % 2 == 0) || kind == EW_F16 ||
                                  kind == EW_Q4_K || kind == EW_Q6R);
        for (int j = 0; j < cnt - 1 && x2; j++) x2 = a.n_end[j] % 64 == 0;
        for (int j = 0; j < cnt && x2; j++) {
            const int64_t rows = a.n_end[j] - (j ? a.n_end[j - 1] : 0);
            // bytes per 32-weight block: Q4_0 18, Q4_K 144 / 8, repacked Q6_K 32, Q8_0 34, F16 64
            x2 = rows * (int64_t)nb *
                     (kind == EW_Q4_0 || kind == EW_Q4_K ? 18 : kind == EW_Q6R ? 32 : kind == EW_Q8_0 ? 34 : 64) <
                 (1LL << 31);
        }
        if (x2) {
            X2Args b = {};
            for (int j = 0; j < kExactMats; j++) {
                b.Y[j] = a.Y[j];
                b.W[j] = a.W[j];
                b.n_end[j] = a.n_end[j];
            }
            b.Ah = Ah;
            b.Al = Al;
            b.Sx = Sx;
            b.Rs = Rs;
            b.R = a.R;
            b.M = M;
            b.N = acc;
            b.nb = nb;
            switch (kind) {
            case EW_Q4_0: launch_exact2<EW_Q4_0, 2>(b); break;
            case EW_Q8_0: launch_exact2<EW_Q8_0, 2>(b); break;
            case EW_Q4_K: launch_exact2<EW_Q4_K, 2>(b); break;
            case EW_Q6R: launch_exact2<EW_Q6R, 2>(b); break;
            default: launch_exact2<EW_F16, 2>(b); break;
            }
            continue;
        }
        if (kind == EW_Q6R) {
            // no second tiling for this group: the first, on the matrices as given
            for (int j = 0; j < kExactMats; j++) a.W[j] = (const uint8_t *)raw[j < cnt ? j : 0];
            launch_exact_for<EW_Q6_K>(a);
            continue;
        }
        switch (kind) {
        case EW_Q4_0: launch_exact_for<EW_Q4_0>(a); break;
        case EW_Q8_0: launch_exact_for<EW_Q8_0>(a); break;
        case EW_Q4_K: launch_exact_for<EW_Q4_K>(a); break;
        case EW_P16: launch_exact_for<EW_P16>(a); break;
        case EW_Q6_K: launch_exact_for<EW_Q6_K>(a); break;
        default: launch_exact_for<EW_F16>(a); break;
        }
    }
    if (own_p) HOLO_CHECK(hipFreeAsync(pws, stream()));
    if (own_a) HOLO_CHECK(hipFreeAsync(aws, stream()));
}

}  // namespace holo

extern "C" {

int holo_prefill_prepare(const void *W, int N, int K, int type)
{
    if (!W || N <= 0 || type != HOLO_TYPE_Q6_K || K <= 0 || K % 256 != 0 || K > 16384 || ((uintptr_t)W & 1u) ||
        (int64_t)N * K >= (1LL << 31)) {
        HOLO_REJECT("holo_prefill_prepare: not a Q6_K matrix the exact product repacks (K a multiple of 256 up "
                    "to 16384, 2-byte aligned, N*K under 2^31)");
        return HOLO_EINVAL;
    }
    if (holo::stream_capturing()) {
        HOLO_REJECT("holo_prefill_prepare: called under graph capture");
        return HOLO_EINVAL;
    }
    {
        std::lock_guard<std::mutex> lk(holo::g_prep_mu);
        const auto it = holo::g_prep.find(W);
        if (it != holo::g_prep.end()) {
            if (it->second.N == N && it->second.K == K) return 0;
            HOLO_REJECT("holo_prefill_prepare: W is registered with another shape");
            return HOLO_EINVAL;
        }
    }
    void *rec = nullptr;
    const hipError_t e = hipMalloc(&rec, (size_t)N * K);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        HOLO_CHECK(e);
        return (int)e;
    }
    holo::q6r_repack(rec, W, N, K);
    const hipError_t es = hipStreamSynchronize(holo::stream());
    if (es != hipSuccess) {
        HOLO_CHECK(es);
        (void)hipFree(rec);
        return (int)es;
    }
    std::lock_guard<std::mutex> lk(holo::g_prep_mu);
    holo::g_prep[W] = holo::PreparedQ6{N, K, rec};
    return 0;
}

void holo_prefill_release(const void *W)
{
    void *rec = nullptr;
    {
        std::lock_guard<std::mutex> lk(holo::g_prep_mu);
        const auto it = holo::g_prep.find(W);
        if (it == holo::g_prep.end()) return;
        rec = it->second.rec;
        holo::g_prep.erase(it);
    }
    HOLO_CHECK(hipStreamSynchronize(holo::stream()));  // no product in flight still reads it
    HOLO_CHECK(hipFree(rec));
}

}  // extern "C"
