// gemv_mfma.h -- device helpers shared by the GEMV kernels (gemv.hip) and
// the persistent decode-step kernel (gemv_stream.hip): wave reductions, the
// activation staging (22-bit fixed point in three int8 planes) and the int8
// MFMA unit dots over Q4_0 / Q8_0 / Q4_K items.
#pragma once

#include "block_window.h"
#include "common.h"
#include "quant_blocks.h"

#include <type_traits>

namespace holo {

enum Mode { MODE_PLAIN = 0, MODE_GATEUP = 1 };
enum XMode { XM_F32 = 0, XM_I24 = 1, XM_GF32 = 2, XM_MFMA = 3 };

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxSeg = 3;
// Activations are held as xi = rint(x * kQmax / amax) per 32-value unit,
// |xi| <= kQmax (< 2^22), split exactly into three signed bytes
// xi = 65536 h + 256 m + l (x_convert); each plane's int8 dot is exact in int32.
constexpr int kQmax = 63 * 65536;

// ---- wave reduction ----------------------------------------------------------

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_shift_add(float v)
{
    int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
    return v + __int_as_float(t);
}

// Sum over the 64 lanes, returned in every lane.
__device__ __forceinline__ float wave_sum(float v)
{
    v = dpp_shift_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_shift_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_shift_add<0x141, 0xF>(v);  // row_half_mirror
    v = dpp_shift_add<0x140, 0xF>(v);  // row_mirror: each lane holds its row's sum
    v = dpp_shift_add<0x142, 0xA>(v);  // row_bcast:15 -> rows 1, 3
    v = dpp_shift_add<0x143, 0xC>(v);  // row_bcast:31 -> rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Hides a value's known bits from the optimiser, so (float)((v >> 8k) & 0xFF)
// selects v_cvt_f32_ubyte{k} instead of a 4-bit v_bfe_u32 + v_cvt_f32_ubyte0.
// Emits no instruction.
__device__ __forceinline__ void opaque(uint32_t &v) { asm volatile("" : "+v"(v)); }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c)
{
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

typedef __attribute__((address_space(1))) const uint8_t gbyte;
typedef __attribute__((address_space(1))) const u32x4 gu32x4;
typedef __attribute__((address_space(1))) const uint32_t gu32;
// Output pointers in the global address space: a store through a generic
// pointer becomes a flat store, which also counts against lgkmcnt, so every
// later LDS wait of the wave would wait for the store's round trip as well.
typedef __attribute__((address_space(1))) float gfloat;
typedef __attribute__((address_space(1))) const float gcfloat;

// ---- activations staged in LDS ------------------------------------------------
//
// XM_F32 : float4 lx[units*8] (chunk c of unit u at slot c ^ (u&7)), then
//          float sx[units] = sum of the unit's 32 activations
// XM_I24 : uint4 lq[units*6] (chunks 0/1 = h bytes of columns 0-15/16-31,
//          2/3 = m bytes, 4/5 = l bytes; the 96-byte unit stride already puts
//          8 neighbouring lanes on distinct banks), then
//          float2 ls[units] = { d_x, sum x }

template <int XM>
__host__ __device__ constexpr int lds_bytes_per_unit()
{
    return XM == XM_F32 ? 128 + 4 : 96 + 8;
}

// Reductions over the 8 lanes of an aligned lane octet (all 8 active).
template <int CTRL>
__device__ __forceinline__ float dpp_get(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float octet_sum(float v)
{
    v += dpp_get<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_get<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_get<0x141>(v);  // row_half_mirror: lane i <- lane 7-i of the octet
    return v;
}
// Maximum of non-negative floats over the octet, compared as their bit
// patterns (which order like the values): v_max_u32 takes the DPP operand
// directly, where fmaxf would first canonicalise it.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_get_u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float octet_max_nonneg(float f)
{
    uint32_t v = __float_as_uint(f);
    v = max(v, dpp_get_u<0xB1>(v));
    v = max(v, dpp_get_u<0x4E>(v));
    v = max(v, dpp_get_u<0x141>(v));
    return __uint_as_float(v);
}

// Packs byte 0 of four ints into one dword (little-endian order a, b, c, d).
__device__ __forceinline__ uint32_t pack4(int a, int b, int c, int d)
{
    uint32_t lo = __builtin_amdgcn_perm((uint32_t)b, (uint32_t)a, 0x0c0c0400u);
    uint32_t hi = __builtin_amdgcn_perm((uint32_t)d, (uint32_t)c, 0x0c0c0400u);
    return lo | (hi << 16);
}

// x staging is split in two so that the activation loads are issued before
// the first tile's weight loads: vector-memory loads complete in issue order
// (s_waitcnt vmcnt), so loads issued after the weight stream would make the
// staging arithmetic wait for the whole weight fetch.
//
// Every thread takes float4 chunks i = tid + 256*k of x (unit i>>3, chunk
// i&7), so the 8 chunks of a unit sit in one aligned lane octet.  The
// kPreX = 8 chunks per thread (in_dim <= 16384) are loaded up front with
// buffer loads: every instruction issues, so the compiler's wait counts stay
// exact, and a chunk past the end of x gets an out-of-range offset, which
// the buffer unit answers with zeros without touching memory.  Longer rows
// load their remaining chunks in x_stage.
constexpr int kPreX = 8;
constexpr uint32_t kBufferWord3 = kRawBufWord3;
constexpr uint32_t kOutOfRange = 0x80000000u;

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t x_rsrc(const float *x, int units)
{
    return __builtin_amdgcn_make_buffer_rsrc((void *)x, (short)0, units * 128, kBufferWord3);
}

// Cache policy of the activation loads: 0 = default; kDeviceScope (sc1) = a
// device-coherent read, which never returns a line this XCD's L2 holds from
// before another XCD wrote it (the multi-stage launch reads earlier stages'
// outputs this way, without invalidating the cache).
constexpr int kDeviceScope = 16;
// Cache policy of the weight loads: non-temporal (streamed once per launch).
constexpr int kNonTemporal = 2;

template <int CPOL = 0>
__device__ __forceinline__ float4 load_x4(__amdgpu_buffer_rsrc_t rs, uint32_t off)
{
    v4f v = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, CPOL));
    return make_float4(v.x, v.y, v.z, v.w);
}

template <int NPX = kPreX, int CPOL = 0>
__device__ __forceinline__ void x_preload(const float *__restrict__ x, int units, float4 (&pre)[NPX])
{
    const int tid = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rs = x_rsrc(x, units);
#pragma unroll
    for (int k = 0; k < NPX; k++) {
        const int i = tid + kThreads * k;
        pre[k] = load_x4<CPOL>(rs, i < units * 8 ? (uint32_t)i * 16u : kOutOfRange);
    }
}

template <int FMT, int XM>
__device__ __forceinline__ void x_convert(const float4 v, int i, int units, void *lds)
{
    const int u = i >> 3, c = i & 7;
    const float sx = octet_sum((v.x + v.y) + (v.z + v.w));
    if constexpr (XM == XM_F32) {
        float4 *lx = (float4 *)lds;
        lx[u * 8 + (c ^ (u & 7))] = v;
        if (c == 0) ((float *)(lx + units * 8))[u] = sx;
    } else {
        const float amax = octet_max_nonneg(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        const float dx = amax * (1.0f / (float)kQmax);
        // kQmax/amax to within an ulp (v_rcp_f32; a correctly rounded divide is
        // a dozen dependent instructions on the staging path): |x * inv| stays
        // within kQmax + 1 < 2^22, and |x - dx*xi| within dx/2 plus an fp32
        // rounding of amax
        const float inv = amax > 0.f ? (float)kQmax * __builtin_amdgcn_rcpf(amax) : 0.f;
        // xi = rint(x * inv) in one fma: 1.5 * 2^23 + x * inv lies in
        // [2^23, 2^24), where floats are the integers, so the fma rounds x * inv
        // to nearest even and the float's bits are 0x4B400000 + xi.  w = xi +
        // 0x808080 has bytes B0..B2 with xi = 65536 (B2-128) + 256 (B1-128) +
        // (B0-128): the signed planes are the bytes of w with the top bit
        // flipped.
        uint32_t w[4];
        const float xv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; k++)
            w[k] = __float_as_uint(__builtin_fmaf(xv[k], inv, 12582912.0f)) - (0x4B400000u - 0x808080u);
        const uint32_t p01 = __builtin_amdgcn_perm(w[1], w[0], 0x05010400u);  // w0.b0 w1.b0 w0.b1 w1.b1
        const uint32_t p23 = __builtin_amdgcn_perm(w[3], w[2], 0x05010400u);  // w2.b0 w3.b0 w2.b1 w3.b1
        const uint32_t r01 = __builtin_amdgcn_perm(w[1], w[0], 0x0c0c0602u);  // w0.b2 w1.b2 0 0
        const uint32_t r23 = __builtin_amdgcn_perm(w[3], w[2], 0x0c0c0602u);  // w2.b2 w3.b2 0 0
        uint32_t *lq = (uint32_t *)((uint4 *)lds + u * 6);
        lq[c] = __builtin_amdgcn_perm(r23, r01, 0x05040100u) ^ 0x80808080u;       // h plane
        lq[8 + c] = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;   // m plane
        lq[16 + c] = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;  // l plane
        // the MFMA path folds Q4_0's -8 into the stored sum
        const float s2 = (XM == XM_MFMA && FMT == FMT_Q4_0) ? -8.0f * sx : sx;
        if (c == 0) ((float2 *)((uint4 *)lds + units * 6))[u] = make_float2(dx, s2);
    }
}

template <int FMT, int XM, int NPX = kPreX, int CPOL = 0>
__device__ __forceinline__ void x_stage(const float *__restrict__ x, int units, void *lds, const float4 (&pre)[NPX])
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int k = 0; k < NPX; k++) {
        const int i = tid + kThreads * k;
        if (i < units * 8) x_convert<FMT, XM>(pre[k], i, units, lds);
    }
    // rows longer than the preload: the remaining chunks are loaded here
    // (after the weight loads, so their wait includes the first tile's weights)
    const __amdgpu_buffer_rsrc_t rs = x_rsrc(x, units);
    for (int i = tid + kThreads * NPX; i < units * 8; i += kThreads)
        x_convert<FMT, XM>(load_x4<CPOL>(rs, (uint32_t)i * 16u), i, units, lds);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// ---- int8 MFMA path -------------------------------------------------------------------
//
// The unit dots of the XM_I24 arithmetic (three exact int8 planes of the
// activations against the unit's weight bytes) run on
// v_mfma_i32_16x16x64_i8 instead of v_dot4, which takes the per-weight work
// off the VALU.  That instruction computes D[i][j] = sum_k A[i][k] B[k][j]
// (16 x 16, k < 64); lane l supplies 16 bytes of A row l%16 and of B column
// l%16 for the k-chunk l/16 and receives D[i][j], j = l%16, i = 4*(l/16) + r,
// in register r.
//
// Lane l = n + 16*g holds one unit of row n: its weights are B column n in
// chunk g (first 16 weights in one MFMA, last 16 in a second one).  A row
// 4*g + p carries activation plane p (h, m, l) of lane group g's unit in
// chunk g and zeros elsewhere, so D[4g + p][n] is the plane-p dot of exactly
// that unit and arrives in lane n + 16 g, register p: every lane receives the
// three integer sums of its own unit.  Only the 12 lanes 20*g + p (p < 3)
// read plane data from LDS; the others read a zero region, so each A operand
// is one LDS read with no lane arithmetic.  The MFMA computes 16x more
// products than are used; on CDNA4 that costs 32 cycles of the matrix core
// per 1024 weights, far below the time to stream those weights from HBM.
//
// Work mapping: an item is 16 rows x one 16-unit segment.  A wave loads it
// with coalesced 16-byte loads (each load instruction reads whole runs of
// rows, item_piece), writes it to its own LDS stage, and each lane (n, g)
// reads back the 4-unit chunk 4g..4g+3 of row n and runs 4 MFMA pairs over
// it (one per unit).  Loading the chunks directly from HBM would make each
// load instruction touch 16 rows x 4 scattered pieces; the staged form runs
// the weight stream at close to the plain-copy rate.  A tile is 16 rows
// (PLAIN) or 8 gate + 8 up rows (GATEUP: B columns 0-7 gate, 8-15 up)
// across all G segments; wave w takes items w, w+8, ... (P slots per tile),
// with two items' loads in flight ahead of the one being computed.
//
// Per unit (d = block scale, {dx, c} = the unit's activation scale and sum
// term staged with the planes, S = 65536*Sh + 256*Sm + Sl):
//   Q4_0  d * (dx*S + c),  c = -8 * sum x
//   Q8_0  d * (dx*S)
//   Q4_K  (d*sc) * (dx*S) - (dmin*m) * c,  c = sum x

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));
typedef __attribute__((address_space(1))) const u32x2 gu32x2;

constexpr int kZeroBytes = 384;  // >= 3*96 + 32: the A reads of non-plane lanes

// Byte offset of the zero region after x_lds bytes of staged activations.  A
// plane lane (g, p) reads its unit-T operand at dword 384j + 96g + 8p + 24T
// (banks 32g + 24T + [0, 24) mod 64); the zero lanes of its 8-lane group read
// dword zero/4 + 24T + [0, 8).  With zero = 96 mod 128 those start at bank
// 24 + 24T, outside the plane lanes' window for either parity of g, so a
// broadcast read and a plane read never wait on one bank.
__host__ __device__ constexpr uint32_t zero_region_off(uint32_t x_lds) { return ((x_lds + 127u) & ~127u) + 96u; }

template <int FMT>
struct Chunk;
template <>
struct Chunk<FMT_Q4_0> {
    u32x4 q[4];
    u32x2 e;
};
template <>
struct Chunk<FMT_Q8_0> {
    u32x4 q[8];
    u32x2 e;
};
template <>
struct Chunk<FMT_Q4_K> {
    u32x4 h;
    u32x4 q[4];
};

// Dword I of a Q4_0 / Q8_0 chunk (a compile-time index, so the chunk stays in
// registers).
template <int I, int FMT>
__device__ __forceinline__ uint32_t cw(const Chunk<FMT> &c)
{
    constexpr int NQ = FMT == FMT_Q4_0 ? 16 : 32;
    if constexpr (I < NQ) return c.q[I / 4][I % 4];
    else return c.e[I - NQ];
}

// ---- coalesced item loads and the per-wave LDS stage ----------------------------

template <int FMT>
struct Geo {
    static constexpr int SEGB = FMT == FMT_Q8_0 ? 544 : 288;  // bytes per row per item
    static constexpr int PR = SEGB / 16;                       // 16-byte pieces per row
    static constexpr int NP = 16 * PR;                         // pieces per item
    static constexpr int NL = (NP + 63) / 64;                  // load instructions per item
    // Stage rows sit RS = SEGB + 16 bytes apart.  At the unpadded stride the
    // lanes n = 0..15 of a chunk read rows at dword offsets 72n or 136n, both
    // 8n mod 64, so rows n and n + 8 hit the same LDS banks; at SEGB + 16
    // (76n or 140n, both 12n mod 64) the 16 rows start in distinct banks, and
    // pieces stay 16-byte aligned.
    static constexpr int RS = SEGB + 24;
    static constexpr int STAGE = 16 * RS;                      // LDS stage bytes per wave
};

typedef uint32_t u32x4a __attribute__((ext_vector_type(4)));   // 16-byte aligned
typedef uint32_t u32x2a __attribute__((ext_vector_type(2)));   // 8-byte aligned
typedef __attribute__((address_space(1))) const u32x4a gu32x4a;

template <int FMT>
struct Raw2 {
    u32x4a v[Geo<FMT>::NL];
};

// Lane (n, g)'s chunk from the wave's stage (row n of the item at n * RS):
// Q4_0 / Q8_0 units 4g..4g+3 = bytes [72g, +72) / [136g, +136) of the row
// (8-byte aligned); Q4_K the header of superblock g/2 and the 64 quant bytes
// of its half g&1 (16-byte aligned).
template <int FMT>
__device__ __forceinline__ void read_chunk(Chunk<FMT> &c, const uint8_t *stage, int n, int g)
{
    if constexpr (FMT == FMT_Q4_K) {
        const uint8_t *b = stage + n * Geo<FMT>::RS + 144 * (g >> 1);
        const u32x2a h0 = *(const u32x2a *)b, h1 = *(const u32x2a *)(b + 8);
        c.h = (u32x4){h0.x, h0.y, h1.x, h1.y};
        const uint8_t *q = b + 16 + 64 * (g & 1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u32x2a lo = *(const u32x2a *)(q + 16 * i), hi = *(const u32x2a *)(q + 16 * i + 8);
            c.q[i] = (u32x4){lo.x, lo.y, hi.x, hi.y};
        }
    } else {
        constexpr int NQ = FMT == FMT_Q4_0 ? 4 : 8;
        const uint8_t *b = stage + n * Geo<FMT>::RS + (FMT == FMT_Q4_0 ? 72 : 136) * g;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const u32x2a lo = *(const u32x2a *)(b + 16 * i);
            const u32x2a hi = *(const u32x2a *)(b + 16 * i + 8);
            c.q[i] = (u32x4){lo.x, lo.y, hi.x, hi.y};
        }
        const u32x2a e = *(const u32x2a *)(b + 16 * NQ);
        c.e = (u32x2){e.x, e.y};
    }
}

__device__ __forceinline__ v4i mfma_i8(v4i a, v4i b, v4i c)
{
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Unit T (0..3) of the chunk: the weight dwords as two MFMA B operands
// (weights 0-15, 16-31) and the block scale bits.  Q4_0 block T sits at byte
// 18T, Q8_0 block T at byte 34T: for even T the scale is the low half of a
// dword and the quants start 2 bytes into it; for odd T the scale is the
// high half of a dword and the quants are dword-aligned.
template <int T, int FMT>
__device__ __forceinline__ void chunk_unit(const Chunk<FMT> &c, v4i &lo, v4i &hi, uint32_t &dbits)
{
    if constexpr (FMT == FMT_Q4_K) {
        const u32x4 q = c.q[T];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = (int)(q[i] & 0x0F0F0F0Fu);
            hi[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
        }
        dbits = 0;
    } else {
        constexpr int W0 = ((FMT == FMT_Q4_0 ? 18 : 34) * T) >> 2;
        constexpr bool EVEN = (T & 1) == 0;
        auto qd = [&](auto I) -> uint32_t {
            constexpr int i = decltype(I)::value;
            if constexpr (EVEN) return __builtin_amdgcn_alignbyte(cw<W0 + i + 1>(c), cw<W0 + i>(c), 2);
            else return cw<W0 + 1 + i>(c);
        };
        dbits = EVEN ? cw<W0>(c) : (cw<W0>(c) >> 16);
        uint32_t q[8];
        q[0] = qd(std::integral_constant<int, 0>{});
        q[1] = qd(std::integral_constant<int, 1>{});
        q[2] = qd(std::integral_constant<int, 2>{});
        q[3] = qd(std::integral_constant<int, 3>{});
        if constexpr (FMT == FMT_Q8_0) {
            q[4] = qd(std::integral_constant<int, 4>{});
            q[5] = qd(std::integral_constant<int, 5>{});
            q[6] = qd(std::integral_constant<int, 6>{});
            q[7] = qd(std::integral_constant<int, 7>{});
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = (int)q[i];
                hi[i] = (int)q[4 + i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = (int)(q[i] & 0x0F0F0F0Fu);
                hi[i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
            }
        }
    }
}

// The 4 sub-block scales and mins of a Q4_K half superblock, one per byte
// (quant.c:290-297): half 0 (j < 4)  sc = s[j] & 63, m = s[j+4] & 63;
// half 1 (j = 4+t)  sc = (s[8+t] & 15) << 2 | s[t] >> 6,
//                   m  = (s[8+t] >> 4) << 2 | s[4+t] >> 6.
__device__ __forceinline__ void q4_k_half_scales(const u32x4 h, bool half1, uint32_t &sc, uint32_t &mn)
{
    const uint32_t s0 = h.y, s1 = h.z, s2 = h.w;
    const uint32_t sc1 = ((s2 & 0x0F0F0F0Fu) << 2) | ((s0 >> 6) & 0x03030303u);
    const uint32_t mn1 = (((s2 >> 4) & 0x0F0F0F0Fu) << 2) | ((s1 >> 6) & 0x03030303u);
    sc = half1 ? sc1 : (s0 & 0x3F3F3F3Fu);
    mn = half1 ? mn1 : (s1 & 0x3F3F3F3Fu);
}

// Unit T of an item: adds its contribution to acc.
template <int T, int FMT>
__device__ __forceinline__ void item_unit(float &acc, const Chunk<FMT> &c, const uint8_t *ldsb, uint32_t abase,
                                          uint32_t sbase, int skip, bool tail, float dk, float mk, uint32_t sc,
                                          uint32_t mn)
{
    const v4i a0 = *(const v4i *)(ldsb + abase + 96 * T);
    const v4i a1 = *(const v4i *)(ldsb + abase + 96 * T + 16);
    const float2 xs = *(const float2 *)(ldsb + sbase + 8 * T);
    v4i lo, hi;
    uint32_t dbits;
    chunk_unit<T, FMT>(c, lo, hi, dbits);
    const v4i zero = {0, 0, 0, 0};
    const v4i s = mfma_i8(a1, hi, mfma_i8(a0, lo, zero));
    // |Sh| <= 32*128*127, so 256*Sh + Sm is exact in int32
    const int t1 = (s[0] << 8) + s[1];
    const float S = fmaf(256.0f, (float)t1, (float)s[2]);
    if constexpr (FMT == FMT_Q4_K) {
        float dsc = dk * (float)((sc >> (8 * T)) & 0xFFu);
        float dmn = mk * (float)((mn >> (8 * T)) & 0xFFu);
        if (tail && T < skip) dsc = dmn = 0.f;
        acc = fmaf(dsc, xs.x * S, fmaf(-dmn, xs.y, acc));
    } else {
        float d = half_bits_to_float(dbits);
        if (tail && T < skip) d = 0.f;
        if constexpr (FMT == FMT_Q4_0) acc = fmaf(d, fmaf(xs.x, S, xs.y), acc);
        else acc = fmaf(d, xs.x * S, acc);
    }
}

// One item: this lane's 4 units.  abase = LDS byte address of the lane's A
// operand for unit 0 (plane data or the zero region), sbase = address of the
// {dx, c} pair of the chunk's first unit.  Slots t < skip repeat units of the
// previous chunk (clamped tail chunk) and get weight 0; `tail` is wave
// uniform and true only for the row's last segment.
template <int FMT>
__device__ __forceinline__ float item_dot(const Chunk<FMT> &c, const uint8_t *ldsb, uint32_t abase, uint32_t sbase,
                                          uint32_t cs, int skip, bool tail)
{
    float acc = 0.f;
    float dk = 0.f, mk = 0.f;
    uint32_t sc = 0, mn = 0;
    if constexpr (FMT == FMT_Q4_K) {
        dk = half_bits_to_float(c.h.x);
        mk = half_bits_to_float(c.h.x >> 16);
        q4_k_half_scales(c.h, (cs >> 2) & 1u, sc, mn);
    }
    item_unit<0, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    item_unit<1, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    item_unit<2, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    item_unit<3, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    return acc;
}

}  // namespace holo
