// gemv.hip -- fused dequant + matrix-vector product over GGUF Q8_0, Q4_0 and
// Q4_K blocks (decode path, batch 1).
//
// Replaces cuda_matmul_q8_0 / q4_0 / q4_k and the two fused Q8_0 multi-GEMVs
// of the reference (src/ai/cuda_ops.cu:1132-1175, 1184-1395).  The reference
// CPU path (src/ai/llm.c:770-926, src/ai/quant.c:541-633) defines the result.
//
// Work mapping (wave64, workgroup of 8 waves):
//   * lane <-> one 32-weight unit of a row (Q8_0/Q4_0 block, Q4_K sub-block);
//     the 64 lanes of a wave read 64 consecutive units of one row, so one
//     load instruction covers one contiguous run of the row (1152 B for
//     Q4_0, 2176 B for Q8_0, 8 superblocks for Q4_K);
//   * an item is R rows x one 64-unit segment of the row.  A workgroup owns a
//     tile of G*R rows x all nsegs segments (G*nsegs items) and deals the
//     items round-robin to its 8 waves (at most P per wave), so long rows
//     are split across waves and every wave has P independent items;
//   * tiles are double-buffered in registers: the raw block loads of the
//     workgroup's next tile are issued before the current tile is decoded,
//     and the first tile's loads are issued before x is staged;
//   * x is staged once per workgroup in LDS with coalesced 16-byte loads
//     (one float4 per lane; per-unit max and sum reduced across the unit's 8
//     lanes with DPP);
//   * each item's R row partials are reduced across the wave with DPP and
//     written to LDS; after the tile's barrier the row sums are finished and
//     stored (the partial buffers alternate between tiles).
//
// Two activation modes (same weights, same decode):
//   XM_F32   exact fp32 activations: unpack nibbles/bytes, v_cvt_f32_ubyte,
//            one FMA per weight; quant offsets folded per unit
//              Q4_0  d*(sum q*x - 8*sum x)      Q8_0  d*(sum (q+128)*x - 128*sum x)
//              Q4_K  (d*sc)*sum q*x - (dmin*m)*sum x
//   XM_I24   activations as 24-bit fixed point per 32-block, held as three
//            int8 planes: xi = rint(x * Q/amax), Q = 127*65536,
//            xi = 65536*h + 256*m + l with h in [-127,127], m, l in
//            [-128,127]; the unit's integer dots sum q*h, sum q*m, sum q*l
//            run on v_dot4_i32_i8 (4 weights per op) and are exact; the
//            rest is fp32:  S = 65536*Sh + 256*Sm + Sl,
//              Q4_0  d_w * (d_x*S - 8*sum x)      Q8_0  d_w * d_x * S
//              Q4_K  (d*sc) * d_x*S - (dmin*m) * sum x
//            |x - d_x*xi| <= d_x = amax * 2^-23 per activation: the
//            activation error is at the level of an fp32 rounding of the
//            block's largest term.
// Accumulation across units is fp32 in both modes.
#include "gemv_mfma.h"

#include <hip/hip_ext.h>
#include <limits.h>
#include <stdlib.h>

#include <type_traits>

namespace holo {

// ---- raw block loads (issued early) and decode (at compute time) ----------------

template <int FMT>
struct Raw;

template <>
struct Raw<FMT_Q4_0> {
    u32x4 a;
    uint32_t e, s;
};
template <>
struct Raw<FMT_Q8_0> {
    u32x4 a, b;
    uint32_t e, s;
};
template <>
struct Raw<FMT_Q4_K> {
    u32x4 h, q;
    uint32_t j;
};

// Loads the raw dwords of one unit.  `ba` is the row's first byte rounded
// down to 4 (wave uniform), `mis` the rounding (0 or 2), `off` the unit's
// byte offset in the row (unit_offset).  Q4_0/Q8_0 load the dword-aligned
// window of the block (block_window); Q4_K loads the superblock header and
// the sub-block's 16 quant bytes.
// Weight loads go through address-space-1 pointers so they compile to
// global_load (vmcnt only).  A flat load would also count against lgkmcnt,
// and every LDS wait would then wait for the weight stream as well.

template <int FMT>
__device__ __forceinline__ void load_raw(Raw<FMT> &r, gbyte *ba, uint32_t mis, uint32_t off, uint32_t u)
{
    if constexpr (FMT == FMT_Q4_0 || FMT == FMT_Q8_0) {
        Window w = block_window(mis, off);
        gbyte *p = ba + w.start;
        r.a = *(gu32x4 *)p;
        if constexpr (FMT == FMT_Q4_0) {
            r.e = *(gu32 *)(p + 16);
        } else {
            r.b = *(gu32x4 *)(p + 16);
            r.e = *(gu32 *)(p + 32);
        }
        r.s = w.s;
    } else {
        gbyte *sb = ba + mis + off;
        r.j = u & 7u;
        r.h = *(gu32x4 *)sb;
        r.q = *(gu32x4 *)(sb + 16 + 16 * r.j);
    }
}

template <int XM>
struct XVals;

template <>
struct XVals<XM_F32> {
    float4 x[8];
    float sx;
    __device__ __forceinline__ void load(const void *lds, int units, int u)
    {
        const float4 *lx = (const float4 *)lds;
        const float4 *p = lx + u * 8;
        const int sw = u & 7;
#pragma unroll
        for (int c = 0; c < 8; c++) x[c] = p[c ^ sw];
        sx = ((const float *)(lx + units * 8))[u];
    }
};

template <>
struct XVals<XM_I24> {
    uint32_t h[8], m[8], l[8];
    float dx, sx;
    __device__ __forceinline__ void load(const void *lds, int units, int u)
    {
        const uint4 *p = (const uint4 *)lds + u * 6;
        uint4 c0 = p[0], c1 = p[1], c2 = p[2], c3 = p[3], c4 = p[4], c5 = p[5];
        h[0] = c0.x; h[1] = c0.y; h[2] = c0.z; h[3] = c0.w;
        h[4] = c1.x; h[5] = c1.y; h[6] = c1.z; h[7] = c1.w;
        m[0] = c2.x; m[1] = c2.y; m[2] = c2.z; m[3] = c2.w;
        m[4] = c3.x; m[5] = c3.y; m[6] = c3.z; m[7] = c3.w;
        l[0] = c4.x; l[1] = c4.y; l[2] = c4.z; l[3] = c4.w;
        l[4] = c5.x; l[5] = c5.y; l[6] = c5.z; l[7] = c5.w;
        float2 s = ((const float2 *)((const uint4 *)lds + units * 6))[u];
        dx = s.x;
        sx = s.y;
    }
};

// Rows too long for LDS staging: each lane reads its unit's 32 activations
// from global memory (L1/L2 resident) and sums them itself.
template <>
struct XVals<XM_GF32> {
    float4 x[8];
    float sx;
    __device__ __forceinline__ void load(const float *__restrict__ gx, int u)
    {
        const float *p = gx + (int64_t)u * 32;
#pragma unroll
        for (int c = 0; c < 8; c++) x[c] = make_float4(p[4 * c], p[4 * c + 1], p[4 * c + 2], p[4 * c + 3]);
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < 8; c++) s += (x[c].x + x[c].y) + (x[c].z + x[c].w);
        sx = s;
    }
};

// ---- per-unit dot products --------------------------------------------------------

// sum q*x over 32 nibbles (q in 0..15), fp32
__device__ __forceinline__ float nib_dot_f32(const uint32_t (&q)[4], const float4 (&x)[8])
{
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t lo = q[i] & 0x0F0F0F0Fu;
        uint32_t hi = (q[i] >> 4) & 0x0F0F0F0Fu;
        opaque(lo);
        opaque(hi);
        const float4 xl = x[i];      // columns 4i..4i+3
        const float4 xh = x[4 + i];  // columns 16+4i..16+4i+3
        a0 = fmaf((float)(lo & 0xFFu), xl.x, a0);
        a1 = fmaf((float)((lo >> 8) & 0xFFu), xl.y, a1);
        a0 = fmaf((float)((lo >> 16) & 0xFFu), xl.z, a0);
        a1 = fmaf((float)(lo >> 24), xl.w, a1);
        a2 = fmaf((float)(hi & 0xFFu), xh.x, a2);
        a3 = fmaf((float)((hi >> 8) & 0xFFu), xh.y, a3);
        a2 = fmaf((float)((hi >> 16) & 0xFFu), xh.z, a2);
        a3 = fmaf((float)(hi >> 24), xh.w, a3);
    }
    return (a0 + a1) + (a2 + a3);
}

// sum (q+128)*x over 32 int8 q, fp32
__device__ __forceinline__ float byte_dot_f32(const uint32_t (&q)[8], const float4 (&x)[8])
{
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t b = q[i] ^ 0x80808080u;
        opaque(b);
        const float4 xv = x[i];
        a0 = fmaf((float)(b & 0xFFu), xv.x, a0);
        a1 = fmaf((float)((b >> 8) & 0xFFu), xv.y, a1);
        a2 = fmaf((float)((b >> 16) & 0xFFu), xv.z, a2);
        a3 = fmaf((float)(b >> 24), xv.w, a3);
    }
    return (a0 + a1) + (a2 + a3);
}

// S = 65536*sum q*h + 256*sum q*m + sum q*l over 32 nibbles (q in 0..15);
// the three integer dots are exact, S rounds once per fma.
__device__ __forceinline__ float nib_dot_i24(const uint32_t (&q)[4], const XVals<XM_I24> &x)
{
    int ah = 0, am = 0, al = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t ln = q[i] & 0x0F0F0F0Fu;
        uint32_t hn = (q[i] >> 4) & 0x0F0F0F0Fu;
        ah = sdot4(ln, x.h[i], ah);
        ah = sdot4(hn, x.h[4 + i], ah);
        am = sdot4(ln, x.m[i], am);
        am = sdot4(hn, x.m[4 + i], am);
        al = sdot4(ln, x.l[i], al);
        al = sdot4(hn, x.l[4 + i], al);
    }
    return fmaf(65536.0f, (float)ah, fmaf(256.0f, (float)am, (float)al));
}

// The same over 32 int8 q.
__device__ __forceinline__ float byte_dot_i24(const uint32_t (&q)[8], const XVals<XM_I24> &x)
{
    int ah = 0, am = 0, al = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        ah = sdot4(q[i], x.h[i], ah);
        am = sdot4(q[i], x.m[i], am);
        al = sdot4(q[i], x.l[i], al);
    }
    return fmaf(65536.0f, (float)ah, fmaf(256.0f, (float)am, (float)al));
}

template <int FMT, int XM>
__device__ __forceinline__ float unit_dot(const Raw<FMT> &r, const XVals<XM> &x)
{
    if constexpr (FMT == FMT_Q4_0) {
        uint32_t sel = realign_sel(r.s);
        uint32_t q[4] = {perm(r.a.y, r.a.x, sel), perm(r.a.z, r.a.y, sel), perm(r.a.w, r.a.z, sel),
                         perm(r.e, r.a.w, sel)};
        float d = half_bits_to_float(__builtin_amdgcn_alignbyte(r.a.y, r.a.x, r.s));
        if constexpr (XM != XM_I24) {
            return d * fmaf(-8.0f, x.sx, nib_dot_f32(q, x.x));
        } else {
            return d * fmaf(-8.0f, x.sx, x.dx * nib_dot_i24(q, x));
        }
    } else if constexpr (FMT == FMT_Q8_0) {
        uint32_t sel = realign_sel(r.s);
        uint32_t q[8] = {perm(r.a.y, r.a.x, sel), perm(r.a.z, r.a.y, sel), perm(r.a.w, r.a.z, sel),
                         perm(r.b.x, r.a.w, sel), perm(r.b.y, r.b.x, sel), perm(r.b.z, r.b.y, sel),
                         perm(r.b.w, r.b.z, sel), perm(r.e, r.b.w, sel)};
        float d = half_bits_to_float(__builtin_amdgcn_alignbyte(r.a.y, r.a.x, r.s));
        if constexpr (XM != XM_I24) {
            return d * fmaf(-128.0f, x.sx, byte_dot_f32(q, x.x));
        } else {
            return d * (x.dx * byte_dot_i24(q, x));
        }
    } else {
        uint32_t sc, mn;
        q4_k_scale_min(r.h.y, r.h.z, r.h.w, r.j, sc, mn);
        float dsc = half_bits_to_float(r.h.x) * (float)sc;
        float dmn = half_bits_to_float(r.h.x >> 16) * (float)mn;
        uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        if constexpr (XM != XM_I24) {
            return fmaf(dsc, nib_dot_f32(q, x.x), -dmn * x.sx);
        } else {
            return fmaf(dsc, x.dx * nib_dot_i24(q, x), -dmn * x.sx);
        }
    }
}


// ---- the kernel -------------------------------------------------------------------

struct GemvArgs {
    const uint8_t *W[kMaxSeg];
    float *y[kMaxSeg];
    int rows[kMaxSeg];
    int tile_end[kMaxSeg];  // inclusive prefix sums of tiles per matrix
    int nseg;               // matrices in this launch (PLAIN) or 2 (GATEUP)
    int ntiles;
    const float *x;
    int units;              // 32-weight units per row
    int nsegs;              // 64-unit segments per row
    int groups;             // G: R-row groups per tile
    int x_lds_bytes;        // staged x, then the partial-sum buffers
    int64_t row_bytes;
    const float *r;         // residual: y = r + W.x (one matrix, PLAIN); may alias y
};

template <int FMT, int XM, int R, int P, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs args)
{
    extern __shared__ uint4 lds[];
    constexpr int NM = MODE == MODE_GATEUP ? 2 : 1;
    const int lane = threadIdx.x & 63;
    // readfirstlane: the wave index is uniform, so tiles, rows and row base
    // pointers live in SGPRs and the loads use a 32-bit per-lane offset
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int units = args.units;
    const int nsegs = args.nsegs;
    const int G = args.groups;
    const int ipt = G * nsegs;  // items per tile, <= kWaves * P
    const int TR = G * R;       // rows per tile
    float *part = (float *)((char *)lds + args.x_lds_bytes);  // [2][NM][TR][nsegs]

    // tile -> (matrix, first row)
    auto locate = [&](int t, int &mseg, int &row0) {
        int s = 0, base = 0;
        if constexpr (MODE == MODE_PLAIN) {
            while (s + 1 < args.nseg && t >= args.tile_end[s]) {
                base = args.tile_end[s];
                s++;
            }
        }
        mseg = s;
        row0 = (t - base) * TR;
    };

    // item slot p of this wave in tile t: item j = wave + 4p -> (group j / nsegs, segment j % nsegs)
    auto issue_tile = [&](Raw<FMT>(&buf)[P][NM][R], int t) {
        int mseg, row0;
        locate(t, mseg, row0);
        const int rows = args.rows[mseg];
        // Every slot loads (an idle slot re-reads the tile's last item), so the
        // number of loads per call is fixed and the wait counts stay exact.
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int j = min(wave + kWaves * p, ipt - 1);
            const int g = j / nsegs, sgm = j - g * nsegs;
            int u = sgm * 64 + lane;
            u = u < units ? u : units - 1;
            const uint32_t off = unit_offset(FMT, (uint32_t)u);
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int mi = MODE == MODE_GATEUP ? m : mseg;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int row = min(row0 + g * R + r, rows - 1);
                    gbyte *rowp = (gbyte *)args.W[mi] + (int64_t)row * args.row_bytes;
                    const uint32_t mis = (uint32_t)((uintptr_t)rowp & 3u);
                    load_raw<FMT>(buf[p][m][r], rowp - mis, mis, off, (uint32_t)u);
                }
            }
        }
    };

    // One tile = the workgroup's work between two barriers.
    auto process_tile = [&](const Raw<FMT>(&buf)[P][NM][R], int t, int pb) {
        float *pt = part + pb * (NM * TR * nsegs);
#pragma unroll
        for (int p = 0; p < P; p++) {
            const int j = wave + kWaves * p;
            if (j < ipt) {
                const int g = j / nsegs, sgm = j - g * nsegs;
                const int u = sgm * 64 + lane;
                const bool active = u < units;
                XVals<XM> xv;
                if constexpr (XM == XM_GF32) xv.load(args.x, active ? u : units - 1);
                else xv.load(lds, units, active ? u : units - 1);
#pragma unroll
                for (int m = 0; m < NM; m++)
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        float v = unit_dot<FMT, XM>(buf[p][m][r], xv);
                        float s0 = wave_sum(active ? v : 0.f);
                        if (lane == 0) pt[(m * TR + g * R + r) * nsegs + sgm] = s0;
                    }
            }
        }
        __syncthreads();

        // finish the tile's rows: sum the nsegs partials in segment order
        int mseg, row0;
        locate(t, mseg, row0);
        const int rows = args.rows[mseg];
        for (int rr = threadIdx.x; rr < TR; rr += kThreads) {
            float s0 = 0.f;
            for (int k = 0; k < nsegs; k++) s0 += pt[rr * nsegs + k];
            if (row0 + rr < rows) {
                if constexpr (MODE == MODE_GATEUP) {
                    float s1 = 0.f;
                    for (int k = 0; k < nsegs; k++) s1 += pt[(TR + rr) * nsegs + k];
                    ((gfloat *)args.y[0])[row0 + rr] = silu(s0) * s1;
                } else {
                    ((gfloat *)args.y[mseg])[row0 + rr] = args.r ? ((gcfloat *)args.r)[row0 + rr] + s0 : s0;
                }
            }
        }
    };

    // The grid never exceeds the tile count, so every workgroup has a tile.
    int t = blockIdx.x;
    const int my_tiles = (args.ntiles - 1 - t) / (int)gridDim.x + 1;

    Raw<FMT> cur[P][NM][R], nxt[P][NM][R];
    float4 pre[kPreX];
    if constexpr (XM != XM_GF32) x_preload(args.x, units, pre);
    issue_tile(cur, t);
    if constexpr (XM != XM_GF32) x_stage<FMT, XM>(args.x, units, lds, pre);
    __syncthreads();

    // All tiles but the last: the next tile's loads are issued (always) before
    // the current one is decoded.  The partial buffers alternate.
    int pb = 0;
    for (int k = 1; k < my_tiles; k++) {
        issue_tile(nxt, t + gridDim.x);
        process_tile(cur, t, pb);
        pb ^= 1;
        t += gridDim.x;
#pragma unroll
        for (int p = 0; p < P; p++)
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
                for (int r = 0; r < R; r++) cur[p][m][r] = nxt[p][m][r];
    }
    process_tile(cur, t, pb);
}

struct MfmaArgs {
    const uint8_t *W[kMaxSeg];
    float *y[kMaxSeg];
    int row_end[kMaxSeg];  // prefix sums of the matrices' rows (PLAIN); unused entries INT_MAX
    int total_rows;        // rows of all matrices (PLAIN) or of one (GATEUP)
    int max_tiles;         // tiles of the longest workgroup range
    int full_tiles;        // F: full tiles per workgroup (dealt round-robin)
    int rem_start;         // first row after the full tiles: F * grid * TR
    const float *x;
    int units;             // 32-weight units per row
    int nsegs;             // G: 16-unit segments per row
    int x_lds_bytes;       // staged activations (planes, then {dx, c} pairs)
    int64_t row_bytes;
    const float *nw;       // RMS-norm weights: x is staged as rms_norm(x) * nw (P <= 2 kernels)
    float eps;
    const float *r;        // residual: y = r + W.x (one matrix, PLAIN); may alias y
};

// One GEMV launch's work for this workgroup: the per-workgroup constants
// derived from MfmaArgs and the item pipeline (gemv_mfma_kernel).
template <int FMT, int P, int MODE>
struct MfmaStage {
    using GE = Geo<FMT>;
    static constexpr int TR = MODE == MODE_GATEUP ? 8 : 16;  // rows per matrix per tile

    const MfmaArgs &args;
    uint8_t *ldsb;
    int lane, wave, n, g, units, G;
    uint32_t zero_off, plane_off, ls_off;
    bool plane_lane;
    uint8_t *stage;
    float *tpart;
    uint32_t *tcnt;
    // This workgroup's rows: F full tiles of TR rows dealt round-robin over
    // the grid (at any moment the grid reads one contiguous stretch of the
    // matrices), then an even share of the remaining rows as one short tile
    // (its spare rows re-read the tile's last row and are not stored).  F and
    // the remainder's start come from the host: a division here would delay
    // every workgroup's first load.
    uint32_t W, wg;
    int F, ex0, ex1, my_tiles, Q;
    // Kernel-argument arrays are read only with constant indices: a per-lane
    // index would turn each access into a memory load ahead of every weight
    // load.  Row v of all matrices -> (matrix, row) by selects.
    int re0, re1;
    uint64_t w0, dw1, dw2, y0, dy1, dy2;
    // Loads of an item of a full tile: the item starts at a wave-uniform
    // address and piece i of this lane lies loff[i] bytes past it (for GATEUP
    // the offset also picks the gate or up matrix, counted from the lower of
    // the two bases, wlo), so an item costs no per-lane address arithmetic.
    // fast: every such offset fits 32 bits.
    static constexpr bool kFastIssue = true;
    uint32_t loff[kFastIssue ? GE::NL : 1];
    uint64_t wlo;
    bool fast;

    __device__ __forceinline__ MfmaStage(const MfmaArgs &a, uint8_t *l) : args(a), ldsb(l)
    {
        lane = threadIdx.x & 63;
        wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        n = lane & 15;
        g = lane >> 4;
        units = a.units;
        G = a.nsegs;
        zero_off = zero_region_off((uint32_t)a.x_lds_bytes);
        stage = ldsb + zero_off + kZeroBytes + wave * GE::STAGE;
        tpart = (float *)(ldsb + zero_off + kZeroBytes + kWaves * GE::STAGE);  // [max_tiles][kWaves][16]
        tcnt = (uint32_t *)(tpart + a.max_tiles * kWaves * 16);               // [max_tiles]
        plane_lane = (n >> 2) == g && (n & 3) < 3;
        plane_off = (uint32_t)(n & 3) * 32u;
        ls_off = (uint32_t)units * 96u;
        W = gridDim.x;
        wg = blockIdx.x;
        F = a.full_tiles;
        const uint32_t rem = (uint32_t)(a.total_rows - a.rem_start);  // < W * TR: wg * rem fits 32 bits
        ex0 = a.rem_start + (int)((wg * rem) / W);
        ex1 = a.rem_start + (int)(((wg + 1) * rem) / W);
        my_tiles = F + (ex1 > ex0 ? 1 : 0);
        Q = my_tiles * P;  // item slots of this wave: P per tile
        re0 = a.row_end[0];
        re1 = a.row_end[1];
        w0 = (uint64_t)a.W[0];
        dw1 = (uint64_t)a.W[1] - w0;
        dw2 = (uint64_t)a.W[2] - w0;
        y0 = (uint64_t)a.y[0];
        dy1 = (uint64_t)a.y[1] - y0;
        dy2 = (uint64_t)a.y[2] - y0;
        const uint64_t rb = (uint64_t)a.row_bytes;
        fast = false;
        wlo = w0;
        if constexpr (!kFastIssue) {
        } else if constexpr (MODE == MODE_GATEUP) {
            const bool up_low = (int64_t)dw1 < 0;
            wlo = up_low ? w0 + dw1 : w0;
            const uint64_t dg = up_low ? 0 - dw1 : 0, du = up_low ? 0 : dw1;  // gate and up past wlo
            fast = (dg > du ? dg : du) + TR * rb < (1ull << 32);
#pragma unroll
            for (int i = 0; i < GE::NL; i++) {
                const Piece pc = item_piece(FMT, 64 * i + lane, false);
                loff[i] = (uint32_t)((pc.row >> 3 ? du : dg) + (uint64_t)(pc.row & 7) * rb + 16u * pc.col);
            }
        } else {
            fast = TR * rb < (1ull << 32);
#pragma unroll
            for (int i = 0; i < GE::NL; i++) {
                const Piece pc = item_piece(FMT, 64 * i + lane, false);
                loff[i] = (uint32_t)((uint64_t)pc.row * rb + 16u * pc.col);
            }
        }
    }

    // rows [row0, rend) of local tile k
    __device__ __forceinline__ void tile_rows(int k, int &row0, int &rend) const
    {
        if (k < F) {
            row0 = (k * (int)W + (int)wg) * TR;
            rend = row0 + TR;
        } else {
            row0 = ex0;
            rend = ex1;
        }
    }
    __device__ __forceinline__ void split_row(int v, int &m, int &r) const
    {
        const int a1 = v >= re0, a2 = v >= re1;
        m = a1 + a2;
        r = v - (a2 ? re1 : a1 ? re0 : 0);
    }
    __device__ __forceinline__ static void store_y(gfloat *p, float v) { *p = v; }
    __device__ __forceinline__ gbyte *wbase(int m) const { return (gbyte *)(w0 + (m == 2 ? dw2 : m == 1 ? dw1 : 0)); }
    __device__ __forceinline__ gfloat *ybase(int m) const { return (gfloat *)(y0 + (m == 2 ? dy2 : m == 1 ? dy1 : 0)); }

    // Slot q: local tile q / P, item (segment) wave + 8 * (q % P).  Slots
    // past the end issue nothing (a wave cannot end before its loads return),
    // except with ALWAYS, where such a slot re-reads row 0 of the first
    // matrix (in bounds, never used).  ALWAYS is the first slot, issued while
    // the activations are staged: with a path that issues no loads, or two
    // load paths, the compiler could not count the loads in flight and waited
    // for all of them, this slot's too, before converting the activations.
    // Weights are read once per launch: the loads are non-temporal, so they
    // do not push the activations and other reused lines out of the caches.
    template <bool ALWAYS = false>
    __device__ __forceinline__ void issue(Raw2<FMT> &b, int q) const
    {
        if (!ALWAYS && q >= Q) return;
        const bool none = ALWAYS && q >= Q;
        const int k = none ? F : q / P, p = none ? 0 : q - k * P;
        int row0, rend;
        tile_rows(k, row0, rend);
        if (none) {
            row0 = 0;
            rend = 1;
        }
        const int seg = min(wave + kWaves * p, G - 1);
        const bool half = 16 * seg + 16 > units;
        // ALWAYS takes the general path alone: one load site, so the loads
        // in flight can be counted wherever they merge
        if (!ALWAYS && kFastIssue && fast && k < F && !half) {
            // a full tile in one matrix (GATEUP: 8 rows of each): the
            // uniform item base plus the lane's fixed offsets
            uint64_t base;
            bool one = true;
            if constexpr (MODE == MODE_GATEUP) {
                base = wlo + (uint64_t)row0 * (uint64_t)args.row_bytes;
            } else {
                int m, r, m1, r1;
                split_row(row0, m, r);
                split_row(row0 + TR - 1, m1, r1);
                one = m == m1;
                base = (uint64_t)wbase(m) + (uint64_t)r * (uint64_t)args.row_bytes;
            }
            if (one) {
                // raw buffer loads: scalar base (uniform by construction),
                // 32-bit lane offset, no range limit
                base += (uint64_t)seg * GE::SEGB;
                const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)base);
                const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
                const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
                    (void *)(((uint64_t)hi << 32) | lo), (short)0, -1, kBufferWord3);
#pragma unroll
                for (int i = 0; i < GE::NL; i++)
                    b.v[i] = __builtin_bit_cast(u32x4a, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)loff[i], 0,
                                                                                              kNonTemporal));
                return;
            }
        }
#pragma unroll
        for (int i = 0; i < GE::NL; i++) {
            const Piece pc = item_piece(FMT, 64 * i + lane, half);
            int m, row;
            if constexpr (MODE == MODE_GATEUP) {
                m = pc.row >> 3;
                row = min(row0 + (pc.row & 7), rend - 1);
            } else {
                split_row(min(row0 + pc.row, rend - 1), m, row);
            }
            gbyte *ap = wbase(m) + (int64_t)row * args.row_bytes + seg * GE::SEGB + 16 * pc.col;
            b.v[i] = __builtin_nontemporal_load((gu32x4a *)ap);
        }
    }

    // the item into the wave's stage (16-byte piece p of row p / PR)
    __device__ __forceinline__ void stage_write(const Raw2<FMT> &b) const
    {
#pragma unroll
        for (int i = 0; i < GE::NL; i++) {
            const int pc = 64 * i + lane;
            // piece pc = row * PR + col goes to row * RS + 16 col = 16 (pc + row)
            if (GE::NP % 64 == 0 || pc < GE::NP) {
                uint8_t *p = stage + 16 * pc + (GE::RS - GE::SEGB) * (pc / GE::PR);
                *(u32x2a *)p = (u32x2a){b.v[i].x, b.v[i].y};
                *(u32x2a *)(p + 8) = (u32x2a){b.v[i].z, b.v[i].w};
            }
        }
    }

    __device__ __forceinline__ void process(int q, float &acc) const
    {
        const int k = q / P, p = q - k * P;
        const int j = wave + kWaves * p;
        if (j < G) {
            Chunk<FMT> c;
            read_chunk<FMT>(c, stage, n, g);
            const int cs0 = 16 * j + 4 * g;
            const bool valid = cs0 < units;  // false only in an 8-unit last segment
            const int cs = valid ? cs0 : units - 4;
            const uint32_t abase = plane_lane ? (uint32_t)cs * 96u + plane_off : zero_off;
            acc += item_dot<FMT>(c, ldsb, abase, ls_off + (uint32_t)cs * 8u, (uint32_t)cs, valid ? 0 : 4,
                                 j == G - 1);
        }
        if (p == P - 1) {
            // Tile end without a barrier: the wave's 16 row partials (the four
            // lane groups summed) go to the tile's own slot, and the wave that
            // completes the tile's count sums the 8 waves' partials and stores.
            float r = acc;
            r += __shfl_xor(r, 16);
            r += __shfl_xor(r, 32);
            acc = 0.f;
            float *pt = tpart + k * (kWaves * 16);
            if (lane < 16) pt[wave * 16 + lane] = r;
            uint32_t arrived = 0;
            if (lane == 0)
                arrived = __hip_atomic_fetch_add(tcnt + k, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
            arrived = __builtin_amdgcn_readfirstlane(arrived);
            if (arrived == kWaves - 1 && lane < TR) {
                int row0, rend;
                tile_rows(k, row0, rend);
                const int v = row0 + lane;
                float s0 = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; w++) s0 += pt[w * 16 + lane];
                if constexpr (MODE == MODE_GATEUP) {
                    float s1 = 0.f;
#pragma unroll
                    for (int w = 0; w < kWaves; w++) s1 += pt[w * 16 + 8 + lane];
                    if (v < rend) store_y(ybase(0) + v, silu(s0) * s1);
                } else if (v < rend) {
                    int m, row;
                    split_row(v, m, row);
                    if (args.r) s0 = ((gcfloat *)args.r)[row] + s0;
                    store_y(ybase(m) + row, s0);
                }
            }
        }
    }

    // x into LDS (planes, {dx, c} pairs, the zero region) and the tile
    // counters cleared; the caller's barrier follows.  x preload: 2P float4
    // per thread cover rows of up to 128 P units, which is every row with P
    // items per wave (G = units/16 <= 8 P); each load instruction costs issue
    // time, so no more are issued.  `first` (loads of slot 0) is issued after
    // the x loads, so the conversion does not wait for it.
    __device__ __forceinline__ void stage_x(Raw2<FMT> &first, bool issue_first) const
    {
        constexpr int NPX = 2 * P;
        constexpr int CPOL = 0;
        constexpr bool NORM = P <= 2;
        float4 pre[NPX], w4[NORM ? NPX : 1];
        x_preload<NPX, CPOL>(args.x, units, pre);
        // the norm weights before the first slot's loads, and every load
        // unconditional (a null weight reads as zeros through an empty buffer
        // range): the conversion then waits for the activations and the
        // weights only, while the first slot's weights are still in flight
        if constexpr (NORM) nw_preload(w4);
        if (issue_first) issue<true>(first, 0);
        if constexpr (NORM) {
            if (args.nw) rms_norm_pre(pre, w4);
        }
        x_stage<FMT, XM_MFMA, NPX, CPOL>(args.x, units, (void *)ldsb, pre);
        if (threadIdx.x < kZeroBytes / 16) ((uint4 *)(ldsb + zero_off))[threadIdx.x] = make_uint4(0, 0, 0, 0);
        for (int i = threadIdx.x; i < args.max_tiles; i += kThreads) tcnt[i] = 0;
    }

    // The norm weights of this thread's x chunks (zeros past the row, and all
    // zeros without a norm).
    template <int NPX>
    __device__ __forceinline__ void nw_preload(float4 (&w4)[NPX]) const
    {
        const __amdgpu_buffer_rsrc_t rs =
            args.nw ? x_rsrc((const float *)args.nw, units) : x_rsrc((const float *)args.x, 0);
#pragma unroll
        for (int k = 0; k < NPX; k++) {
            const int i = threadIdx.x + kThreads * k;
            w4[k] = load_x4<0>(rs, i < units * 8 ? (uint32_t)i * 16u : kOutOfRange);
        }
    }
    // x <- x * (1/sqrt(mean(x^2) + eps)) * nw, in registers before staging, as
    // rms_norm_k computes it (cuda_ops.cu:1479-1504): every chunk of x is in
    // pre[] (the host checks in_dim), so each workgroup reduces the whole
    // vector itself; the 8 wave sums meet in the first wave's stage, which is
    // not written before the staging barrier.
    template <int NPX>
    __device__ __forceinline__ void rms_norm_pre(float4 (&pre)[NPX], const float4 (&w4)[NPX]) const
    {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < NPX; k++)  // chunks past the end were loaded as zeros
            ss += pre[k].x * pre[k].x + pre[k].y * pre[k].y + pre[k].z * pre[k].z + pre[k].w * pre[k].w;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        float *red = (float *)(ldsb + zero_off + kZeroBytes);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) tot += red[w];
        const float scale = 1.0f / sqrtf(tot / (float)(units * 32) + args.eps);
#pragma unroll
        for (int k = 0; k < NPX; k++)
            pre[k] = make_float4(pre[k].x * scale * w4[k].x, pre[k].y * scale * w4[k].y, pre[k].z * scale * w4[k].z,
                                 pre[k].w * scale * w4[k].w);
    }

    // All item slots, slot 0 already issued into b0.  One item in flight per
    // wave: the next item is issued once the current one has arrived (more
    // outstanding loads measured slower on MI355X).
    __device__ __forceinline__ void run(Raw2<FMT> &b0, Raw2<FMT> &b1) const
    {
        float acc = 0.f;
        for (int q = 0; q < Q; q += 2) {
            stage_write(b0);
            issue(b1, q + 1);
            process(q, acc);
            if (q + 1 < Q) {
                stage_write(b1);
                issue(b0, q + 2);
                process(q + 1, acc);
            }
        }
    }
};

template <int FMT, int P, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_mfma_kernel(MfmaArgs args)
{
    extern __shared__ uint4 lds[];
    MfmaStage<FMT, P, MODE> st(args, (uint8_t *)lds);
    Raw2<FMT> b0, b1;
    st.stage_x(b0, true);
    __syncthreads();
    st.run(b0, b1);
}

// ---- host side ---------------------------------------------------------------------

// Activation mode and launch shape; environment overrides are read once:
// HOLO_GEMV_XMODE=f32|i24|mfma, HOLO_GEMV_WG_PER_CU, HOLO_GEMV_ROWS=1|2|4.
struct Tuning {
    int xmode = XM_MFMA;
    bool mfma_q8 = true;  // MFMA path for Q8_0 as well (4096x4096: 5.9 against 6.2 us on F32)
    int wg_per_cu = 0;  // 0 = by grid size
    int rows = 0;       // 0 = by shape
    bool read = false;
};
static Tuning g_tune;

static const Tuning &tuning()
{
    if (!g_tune.read) {
        if (const char *e = getenv("HOLO_GEMV_XMODE")) {
            g_tune.xmode = (e[0] == 'f') ? XM_F32 : (e[0] == 'i') ? XM_I24 : XM_MFMA;
            g_tune.mfma_q8 = g_tune.xmode == XM_MFMA;
        }
        if (const char *e = getenv("HOLO_GEMV_WG_PER_CU")) g_tune.wg_per_cu = atoi(e) > 0 ? atoi(e) : 0;
        if (const char *e = getenv("HOLO_GEMV_ROWS")) g_tune.rows = atoi(e);
        g_tune.read = true;
    }
    return g_tune;
}

constexpr int kMaxLdsBytes = 64 * 1024;
constexpr size_t kMaxMfmaLds = 160 * 1024;  // MI355X: 160 KB of LDS per workgroup

template <int FMT, int XM, int R, int P, int MODE>
static void launch_t(GemvArgs &a)
{
    constexpr int NM = MODE == MODE_GATEUP ? 2 : 1;
    size_t lds = (size_t)a.x_lds_bytes + sizeof(float) * 2 * NM * a.groups * R * a.nsegs;
    // One workgroup per CU for small grids (fewer redundant x stagings), two
    // once there are more than two tiles per CU (measured on MI355X).
    int wpc = tuning().wg_per_cu;
    if (wpc <= 0) wpc = a.ntiles <= 2 * num_cus() ? 1 : 2;
    int blocks = a.ntiles;
    int cap = num_cus() * wpc;
    if (blocks > cap) blocks = cap;
    launch_timed(gemv_kernel<FMT, XM, R, P, MODE>, dim3(blocks), dim3(kThreads), lds, a);
    HOLO_LAUNCH_CHECK();
}

template <int FMT, int XM, int R, int MODE>
static void launch_p(GemvArgs &a, int P)
{
    if (P <= 2) launch_t<FMT, XM, R, 2, MODE>(a);
    else if (P == 3) launch_t<FMT, XM, R, 3, MODE>(a);
    else launch_t<FMT, XM, R, 4, MODE>(a);
}

template <int FMT, int XM, int MODE>
static void launch_r(GemvArgs &a, int R, int P)
{
    if (R <= 1) {
        launch_p<FMT, XM, 1, MODE>(a, P);
    } else if constexpr (MODE == MODE_GATEUP) {
        launch_p<FMT, XM, 2, MODE>(a, P);  // two matrices per item: at most 2 rows
    } else {
        if (R == 2) launch_p<FMT, XM, 2, MODE>(a, P);
        else launch_p<FMT, XM, 4, MODE>(a, P);
    }
}

// holo_time_next_launch: events for the next timed launch (MFMA GEMV or
// prefill GEMM)
static void *g_time_start = nullptr, *g_time_stop = nullptr;

bool take_launch_events(hipEvent_t *start, hipEvent_t *stop)
{
    if (!g_time_start) return false;
    *start = (hipEvent_t)g_time_start;
    *stop = (hipEvent_t)g_time_stop;
    g_time_start = g_time_stop = nullptr;
    return true;
}

template <int FMT>
static size_t mfma_lds_bytes(int units, int max_tiles)
{
    const size_t x_lds = ((size_t)units * lds_bytes_per_unit<XM_I24>() + 15) & ~(size_t)15;
    return zero_region_off((uint32_t)x_lds) + kZeroBytes + (size_t)kWaves * Geo<FMT>::STAGE +
           (size_t)max_tiles * (kWaves * 16 * 4 + 4);
}

static int mfma_max_tiles(int total_rows, int tr, int grid)
{
    return total_rows / (grid * tr) + 1;  // full tiles plus the short one
}

// Workgroups for an MFMA launch: one or two per CU (HOLO_GEMV_WG_PER_CU
// forces it), at most one per tile of rows.  Two per CU give each CU 16
// waves; they are used when both fit in LDS and the rows fill the tiles as
// well as with one per CU (the short last tile costs about a full tile).
template <int FMT>
static int mfma_grid(int total_rows, int tr, int units)
{
    const int tiles = (total_rows + tr - 1) / tr;
    auto clamp = [&](int w) { return w < tiles ? w : tiles; };
    const int forced = tuning().wg_per_cu;
    if (forced > 0) return clamp(num_cus() * forced);
    auto fill = [&](int w) {
        const int t = total_rows / (w * tr) + (total_rows % (w * tr) ? 1 : 0);
        return (double)total_rows / ((double)w * tr * t);
    };
    const int w1 = clamp(num_cus()), w2 = clamp(2 * num_cus());
    const size_t lds2 = mfma_lds_bytes<FMT>(units, mfma_max_tiles(total_rows, tr, w2));
    if (w2 > w1 && 2 * lds2 <= kMaxMfmaLds && fill(w2) >= fill(w1) - 0.02) return w2;
    return w1;
}

template <int FMT, int MODE>
static void launch_mfma(MfmaArgs &a, int P)
{
    constexpr int TR = MODE == MODE_GATEUP ? 8 : 16;
    const int blocks = mfma_grid<FMT>(a.total_rows, TR, a.units);
    a.max_tiles = mfma_max_tiles(a.total_rows, TR, blocks);
    a.full_tiles = a.total_rows / (blocks * TR);
    a.rem_start = a.full_tiles * blocks * TR;
    const size_t lds = mfma_lds_bytes<FMT>(a.units, a.max_tiles);
    auto go = [&](auto kern) {
        // more than 64 KB of LDS must be enabled per kernel (once)
        static bool attr = false;
        if (!attr) {
            HOLO_CHECK(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)kMaxMfmaLds));
            attr = true;
        }
        hipEvent_t e0, e1;
        if (take_launch_events(&e0, &e1)) {
            // events at the kernel's own start and end (holo_time_next_launch)
            hipExtLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, stream(), e0, e1, 0, a);
        } else {
            hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), lds, stream(), a);
        }
        HOLO_LAUNCH_CHECK();
    };
    switch (P) {
    case 1: go(gemv_mfma_kernel<FMT, 1, MODE>); break;
    case 2: go(gemv_mfma_kernel<FMT, 2, MODE>); break;
    case 3: go(gemv_mfma_kernel<FMT, 3, MODE>); break;
    default: go(gemv_mfma_kernel<FMT, 4, MODE>); break;
    }
}

// The MFMA path takes rows whose unit count is a multiple of 8 (row bytes a
// multiple of 16; in_dim a multiple of 256), at most 4 items per wave per
// tile, and LDS within kMaxMfmaLds (checked for the largest tile count,
// every row in its own tile).
static bool mfma_fits(int fmt, int units, int total_rows, int tr)
{
    if (units < 8 || (units & 7) || (units + 15) / 16 > 4 * kWaves) return false;
    auto lds_for = [&](auto fmtc) {
        constexpr int F = decltype(fmtc)::value;
        const int grid = mfma_grid<F>(total_rows, tr, units);
        return mfma_lds_bytes<F>(units, mfma_max_tiles(total_rows, tr, grid > 0 ? grid : 1));
    };
    const size_t lds = fmt == FMT_Q4_0   ? lds_for(std::integral_constant<int, FMT_Q4_0>{})
                       : fmt == FMT_Q8_0 ? lds_for(std::integral_constant<int, FMT_Q8_0>{})
                                         : lds_for(std::integral_constant<int, FMT_Q4_K>{});
    return lds <= kMaxMfmaLds;
}

static bool check_ptr(const void *p, const char *what)
{
    if (((uintptr_t)p & 3u) != 0) {
        HOLO_REJECT(what);
        return false;
    }
    return true;
}

// Items per wave P and row groups per tile G for nsegs segments per row:
// the tile holds G*nsegs <= 4P items; pick the fullest P in 2..4.
static void tile_shape(int nsegs, int &P, int &G)
{
    P = 2;
    G = 1;
    double best = -1.0;
    for (int p = 2; p <= 4; p++) {
        int g = (kWaves * p) / nsegs;
        if (g < 1) continue;
        double util = (double)(g * nsegs) / (kWaves * p);
        if (util > best + 1e-9) {
            best = util;
            P = p;
            G = g;
        }
    }
}

static void gemv_mfma(int fmt, int mode, int nseg, const void *const *W, float *const *y, const int *rows,
                      const float *x, int units, int64_t row_bytes, const float *nw = nullptr, float eps = 0.f,
                      const float *r = nullptr)
{
    MfmaArgs a = {};
    a.nw = nw;
    a.eps = eps;
    a.r = r;
    a.units = units;
    a.row_bytes = row_bytes;
    a.x = x;
    a.nsegs = (units + 15) / 16;
    a.x_lds_bytes = (units * lds_bytes_per_unit<XM_I24>() + 15) & ~15;
    const int P = (a.nsegs + kWaves - 1) / kWaves;
    int total = 0;
    for (int s = 0; s < kMaxSeg; s++) {
        if (s < nseg) {
            a.W[s] = (const uint8_t *)W[s];
            a.y[s] = y[s];
            total += rows[s];
            a.row_end[s] = total;
        } else {
            a.W[s] = a.W[0];
            a.y[s] = a.y[0];
            a.row_end[s] = INT_MAX;
        }
    }
    a.total_rows = mode == MODE_GATEUP ? rows[0] : total;
    if (a.total_rows == 0) return;
    if (fmt == FMT_Q4_0) {
        if (mode == MODE_PLAIN) launch_mfma<FMT_Q4_0, MODE_PLAIN>(a, P);
        else launch_mfma<FMT_Q4_0, MODE_GATEUP>(a, P);
    } else if (fmt == FMT_Q8_0) {
        if (mode == MODE_PLAIN) launch_mfma<FMT_Q8_0, MODE_PLAIN>(a, P);
        else launch_mfma<FMT_Q8_0, MODE_GATEUP>(a, P);
    } else {
        if (mode == MODE_PLAIN) launch_mfma<FMT_Q4_K, MODE_PLAIN>(a, P);
        else launch_mfma<FMT_Q4_K, MODE_GATEUP>(a, P);
    }
}


// One launch over up to three matrices sharing x and in_dim.  nw: stage
// rms_norm(x) * nw instead of x (the MFMA path with in_dim <= 8192 only;
// false, with nothing launched, otherwise).  r: y = r + W.x (one matrix).
static bool gemv_multi(int fmt, int mode, int nseg, const void *const *W, float *const *y, const int *rows,
                       const float *x, int in_dim, const float *nw = nullptr, float eps = 0.f,
                       const float *r = nullptr)
{
    const Tuning &tn = tuning();
    GemvArgs a = {};
    a.units = units_per_row(fmt, in_dim);
    a.row_bytes = row_bytes_of(fmt, in_dim);
    a.nsegs = (a.units + 63) / 64;
    a.x = x;
    a.nseg = nseg;
    a.r = r;
    if (a.nsegs > 4 * kWaves) {
        HOLO_REJECT("gemv: in_dim too large (at most 32 segments of 64 units per row)");
        return true;
    }
    if (a.units == 0) {
        // No complete block per row: every dot product is empty (gate/up:
        // silu(0) * 0 = 0).
        if (r) {
            if (r != y[0])
                HOLO_CHECK(hipMemcpyAsync(y[0], r, sizeof(float) * rows[0], hipMemcpyDeviceToDevice, stream()));
            return true;
        }
        for (int s = 0; s < (mode == MODE_GATEUP ? 1 : nseg); s++)
            if (rows[s] > 0) fill_bytes(y[s], 0, sizeof(float) * rows[s]);
        return true;
    }
    // Q8_0 rows carry twice the bytes per weight, so the F32 path streams
    // them well at in_dim 4096: on MI355X it is faster at 32000x4096 (26.9
    // against 31.3 us) and level or faster at 4096x4096 and 11008x4096.  At
    // 4096x11008 the MFMA path is faster (12.8 against 15.1 us).  Q8_0
    // therefore takes the MFMA path when in_dim > 8192 (always with
    // HOLO_GEMV_XMODE=mfma); Q4_0 and Q4_K always.
    int total = 0;
    for (int s = 0; s < nseg; s++) total += rows[s];
    if (mode == MODE_GATEUP) total = rows[0];
    if (tn.xmode == XM_MFMA && (fmt != FMT_Q8_0 || tn.mfma_q8 || a.units > 256)) {
        bool aligned16 = ((uintptr_t)x & 3u) == 0;
        for (int s = 0; s < nseg; s++) aligned16 = aligned16 && (((uintptr_t)W[s] & 15u) == 0);
        const bool norm_ok = !nw || (a.units % 8 == 0 && a.units <= 256 && ((uintptr_t)nw & 15u) == 0);
        if (aligned16 && norm_ok && mfma_fits(fmt, a.units, total, mode == MODE_GATEUP ? 8 : 16)) {
            gemv_mfma(fmt, mode, nseg, W, y, rows, x, a.units, a.row_bytes, nw, eps, r);
            return true;
        }
    }
    if (nw) return false;
    // x staged in LDS when it fits (F32 needs 132 B per unit, I24 104 B),
    // otherwise read by each lane from global memory.
    int xm = tn.xmode == XM_MFMA ? XM_F32 : tn.xmode;
    const size_t budget = (size_t)kMaxLdsBytes - 4096;
    if (xm == XM_F32 && (size_t)a.units * lds_bytes_per_unit<XM_F32>() > budget) xm = XM_I24;
    if (xm == XM_I24 && (size_t)a.units * lds_bytes_per_unit<XM_I24>() > budget) xm = XM_GF32;
    a.x_lds_bytes = xm == XM_F32   ? a.units * lds_bytes_per_unit<XM_F32>()
                    : xm == XM_I24 ? a.units * lds_bytes_per_unit<XM_I24>()
                                   : 0;
    a.x_lds_bytes = (a.x_lds_bytes + 15) & ~15;
    int P, G;
    tile_shape(a.nsegs, P, G);
    int total_rows = 0;
    for (int s = 0; s < nseg; s++) total_rows += rows[s];
    int R = tn.rows ? tn.rows : 1;
    R = R <= 1 ? 1 : R <= 2 ? 2 : 4;
    if (mode == MODE_GATEUP && R > 2) R = 2;
    a.groups = G;
    const int TR = G * R;
    if (!check_ptr(x, "activation vector must be 4-byte aligned")) return true;
    int tiles = 0;
    for (int s = 0; s < nseg; s++) {
        if (!check_ptr(W[s], "weight matrix must be 4-byte aligned")) return true;
        a.W[s] = (const uint8_t *)W[s];
        a.y[s] = y[s];
        a.rows[s] = rows[s];
        if (mode == MODE_PLAIN) tiles += (rows[s] + TR - 1) / TR;
        a.tile_end[s] = tiles;
    }
    if (mode == MODE_GATEUP) tiles = (rows[0] + TR - 1) / TR;
    a.ntiles = tiles;
    if (tiles == 0) return true;
#define HOLO_DISPATCH(F)                                                             \
    if (xm == XM_F32) {                                                              \
        if (mode == MODE_PLAIN) launch_r<F, XM_F32, MODE_PLAIN>(a, R, P);            \
        else launch_r<F, XM_F32, MODE_GATEUP>(a, R, P);                              \
    } else if (xm == XM_GF32) {                                                      \
        if (mode == MODE_PLAIN) launch_r<F, XM_GF32, MODE_PLAIN>(a, R, P);           \
        else launch_r<F, XM_GF32, MODE_GATEUP>(a, R, P);                             \
    } else {                                                                         \
        if (mode == MODE_PLAIN) launch_r<F, XM_I24, MODE_PLAIN>(a, R, P);            \
        else launch_r<F, XM_I24, MODE_GATEUP>(a, R, P);                              \
    }
    if (fmt == FMT_Q4_0) {
        HOLO_DISPATCH(FMT_Q4_0)
    } else if (fmt == FMT_Q8_0) {
        HOLO_DISPATCH(FMT_Q8_0)
    } else {
        HOLO_DISPATCH(FMT_Q4_K)
    }
#undef HOLO_DISPATCH
    (void)total_rows;
    return true;
}

static void gemv_one(int fmt, float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    if (out_dim <= 0) return;
    if (!M) {
        // matmul_q with a NULL matrix writes zeros (llm.c:772-775).
        fill_bytes(dst, 0, sizeof(float) * out_dim);
        return;
    }
    const void *W[1] = {M};
    float *y[1] = {dst};
    int rows[1] = {out_dim};
    gemv_multi(fmt, MODE_PLAIN, 1, W, y, rows, v, in_dim);
}

static int fmt_of_type(int type)
{
    switch (type) {
    case HOLO_TYPE_Q4_0: return FMT_Q4_0;
    case HOLO_TYPE_Q8_0: return FMT_Q8_0;
    case HOLO_TYPE_Q4_K: return FMT_Q4_K;
    default: return -1;
    }
}

}  // namespace holo

using namespace holo;

extern "C" {

void cuda_matmul_q8_0(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    gemv_one(FMT_Q8_0, dst, M, v, out_dim, in_dim);
}

void cuda_matmul_q4_0(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    gemv_one(FMT_Q4_0, dst, M, v, out_dim, in_dim);
}

void cuda_matmul_q4_k(float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    gemv_one(FMT_Q4_K, dst, M, v, out_dim, in_dim);
}

void holo_gemv_set_xmode(int xmode)
{
    tuning();
    g_tune.xmode = xmode == 1 ? XM_I24 : (xmode >= 2 && xmode <= 4) ? XM_MFMA : XM_F32;
    g_tune.mfma_q8 = xmode != 4;
}

void holo_time_next_launch(void *start_event, void *stop_event)
{
    g_time_start = start_event;
    g_time_stop = stop_event;
}

void holo_gemv_set_launch(int rows_per_item, int wg_per_cu)
{
    tuning();
    g_tune.rows = rows_per_item > 0 ? rows_per_item : 0;
    g_tune.wg_per_cu = wg_per_cu > 0 ? wg_per_cu : 0;
}

void holo_batched_qkv(float *q_out, float *k_out, float *v_out, const void *Wq, const void *Wk, const void *Wv,
                      const float *x, int q_dim, int kv_dim, int in_dim, int type)
{
    int fmt = fmt_of_type(type);
    if (fmt < 0 || !Wq || !Wk || !Wv || q_dim < 0 || kv_dim < 0) {
        HOLO_REJECT("holo_batched_qkv: unsupported type or missing matrix");
        return;
    }
    const void *W[3] = {Wq, Wk, Wv};
    float *y[3] = {q_out, k_out, v_out};
    int rows[3] = {q_dim, kv_dim, kv_dim};
    gemv_multi(fmt, MODE_PLAIN, 3, W, y, rows, x, in_dim);
}

void holo_batched_ffn_gate_up(float *out, const void *W1, const void *W3, const float *x, int ffn_dim, int in_dim,
                              int type)
{
    int fmt = fmt_of_type(type);
    if (fmt < 0 || !W1 || !W3 || ffn_dim < 0) {
        HOLO_REJECT("holo_batched_ffn_gate_up: unsupported type or missing matrix");
        return;
    }
    const void *W[2] = {W1, W3};
    float *y[2] = {out, out};
    int rows[2] = {ffn_dim, ffn_dim};
    gemv_multi(fmt, MODE_GATEUP, 2, W, y, rows, x, in_dim);
}

// ---- fused with the RMS norm before, or the residual add after ---------------------
// A decode layer is rms_norm -> q/k/v, o -> residual add, rms_norm -> gate/up,
// down -> residual add (llm_cuda.c:598-880).  These fold the norms into the
// GEMV's activation staging and the adds into its output stores, halving the
// launches of a decode step.  No reference counterpart (extensions).

void holo_batched_qkv_norm(float *q_out, float *k_out, float *v_out, const void *Wq, const void *Wk, const void *Wv,
                           const float *x, const float *norm_w, float eps, float *xb, int q_dim, int kv_dim, int in_dim,
                           int type)
{
    int fmt = fmt_of_type(type);
    if (fmt < 0 || !Wq || !Wk || !Wv || !x || q_dim < 0 || kv_dim < 0) {
        HOLO_REJECT("holo_batched_qkv_norm: unsupported type or missing matrix");
        return;
    }
    const void *W[3] = {Wq, Wk, Wv};
    float *y[3] = {q_out, k_out, v_out};
    int rows[3] = {q_dim, kv_dim, kv_dim};
    if (norm_w && gemv_multi(fmt, MODE_PLAIN, 3, W, y, rows, x, in_dim, norm_w, eps)) return;
    if (!xb) {
        HOLO_REJECT("holo_batched_qkv_norm: shape outside the fused path and no xb scratch");
        return;
    }
    cuda_rms_norm(xb, x, norm_w, in_dim, eps);
    gemv_multi(fmt, MODE_PLAIN, 3, W, y, rows, xb, in_dim);
}

void holo_batched_ffn_gate_up_norm(float *out, const void *W1, const void *W3, const float *x, const float *norm_w,
                                   float eps, float *xb, int ffn_dim, int in_dim, int type)
{
    int fmt = fmt_of_type(type);
    if (fmt < 0 || !W1 || !W3 || !x || ffn_dim < 0) {
        HOLO_REJECT("holo_batched_ffn_gate_up_norm: unsupported type or missing matrix");
        return;
    }
    const void *W[2] = {W1, W3};
    float *y[2] = {out, out};
    int rows[2] = {ffn_dim, ffn_dim};
    if (norm_w && gemv_multi(fmt, MODE_GATEUP, 2, W, y, rows, x, in_dim, norm_w, eps)) return;
    if (!xb) {
        HOLO_REJECT("holo_batched_ffn_gate_up_norm: shape outside the fused path and no xb scratch");
        return;
    }
    cuda_rms_norm(xb, x, norm_w, in_dim, eps);
    gemv_multi(fmt, MODE_GATEUP, 2, W, y, rows, xb, in_dim);
}

void holo_matmul_add(float *y, const void *M, const float *v, const float *r, int out_dim, int in_dim, int type)
{
    if (out_dim <= 0) return;
    if (!y || !r || !v) {
        HOLO_REJECT("holo_matmul_add: null pointer");
        return;
    }
    const int fmt = fmt_of_type(type);
    if (!M) {
        // a NULL matrix multiplies to zeros (llm.c:772-775): y = r
        if (y != r) HOLO_CHECK(hipMemcpyAsync(y, r, sizeof(float) * out_dim, hipMemcpyDeviceToDevice, stream()));
        return;
    }
    if (fmt >= 0) {
        const void *W[1] = {M};
        float *yy[1] = {y};
        int rows[1] = {out_dim};
        gemv_multi(fmt, MODE_PLAIN, 1, W, yy, rows, v, in_dim, nullptr, 0.f, r);
        return;
    }
    if (y == r) {
        HOLO_REJECT("holo_matmul_add: y may alias r only for Q8_0, Q4_0 and Q4_K");
        return;
    }
    holo_matmul(y, M, v, out_dim, in_dim, type);
    cuda_vec_add(y, y, r, out_dim);
}

// cuda_ops.cu:1282-1294
void cuda_batched_qkv_q8_0(float *q_out, float *k_out, float *v_out, const void *Wq, const void *Wk, const void *Wv,
                           const float *x, int q_dim, int kv_dim, int in_dim)
{
    holo_batched_qkv(q_out, k_out, v_out, Wq, Wk, Wv, x, q_dim, kv_dim, in_dim, HOLO_TYPE_Q8_0);
}

// cuda_ops.cu:1386-1395
void cuda_batched_ffn_gate_up_q8_0(float *out, const void *W1, const void *W3, const float *x, int ffn_dim,
                                   int in_dim)
{
    holo_batched_ffn_gate_up(out, W1, W3, x, ffn_dim, in_dim, HOLO_TYPE_Q8_0);
}

}  // extern "C"
