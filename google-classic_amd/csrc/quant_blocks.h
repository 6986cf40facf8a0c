// quant_blocks.h -- device-side decoding of GGUF blocks (gfx950).
//
// Block formats (reference src/ai/quant.h:43-120; sizes gguf.c:29-37):
//   Q8_0  34 B  { f16 d; int8 qs[32] }                 w[j] = d*qs[j]
//   Q4_0  18 B  { f16 d; u8 qs[16] }                   w[j] = d*((qs[j]&15)-8),
//                                                      w[j+16] = d*((qs[j]>>4)-8)
//   Q4_K 144 B  { f16 d, dmin; u8 scales[12]; u8 qs[128] }, 8 sub-blocks of 32:
//               sub-block j reads qs[16j..16j+15], low nibble -> 32j+l,
//               high nibble -> 32j+l+16, w = (d*sc_j)*q - dmin*m_j
//   Q6_K 210 B  { u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d }
//
// A "unit" is 32 consecutive weights of a row: one Q8_0/Q4_0 block or one
// Q4_K sub-block.  Unit u of a row covers columns 32u..32u+31 in every format.
//
// Q8_0 and Q4_0 blocks are 34/18 bytes, so a block starts at a 4-byte or a
// 2-byte boundary (s = offset & 3 is 0 or 2).  A lane loads the dword-aligned
// window that holds its block and realigns the quant bytes in registers with
// v_perm_b32: qs dword i = bytes [s+2+4i, s+5+4i] of the window.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace holo {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ float half_bits_to_float(uint32_t bits)
{
    // v_cvt_f32_f16: exact for zeros, subnormals, normals and Inf.
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
    return (float)h;
}

// Bit-level f16 -> f32 following the reference table (quant.c:44-82), which
// keeps a NaN's payload unchanged; used where results must match bit for bit.
__device__ __forceinline__ float half_bits_to_float_exact(uint32_t h)
{
    uint32_t sign = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 31u) return __uint_as_float(sign | 0x7F800000u | (m << 13));
    if (e == 0u) {
        float v = (float)m * 0x1.0p-24f;  // exact: m < 2^10
        return __uint_as_float(__float_as_uint(v) | sign);
    }
    return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

// Selector for v_perm_b32(hi, lo, sel): 4 bytes starting at byte s+2 of the
// 8-byte pair {hi:lo}, for s in {0, 2}.
__device__ __forceinline__ uint32_t realign_sel(uint32_t s) { return s ? 0x07060504u : 0x05040302u; }

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel)
{
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// ---- Q4_0 ------------------------------------------------------------------
struct Q4_0Unit {
    uint32_t q[4];  // 32 nibbles: byte k of q[i] = qs[4i+k]
    float d;
    uint32_t dh;    // d as raw f16 bits
};

// The words of one Q4_0 block as loaded, before realignment.  A staging
// pipeline keeps these in its registers and builds the unit (q4_0_unit) only
// where it uses it: realigning right after the loads would make the wave wait
// for them there, one stage early.
struct Q4_0Raw {
    u32x4 a;     // the 16 bytes from the block's 4-byte-aligned start
    uint32_t e;  // the next 4 (2 at the end of the matrix)
    uint32_t s;  // the block's offset within a (0 or 2)
};

// W: matrix base (4-byte aligned); o: the block's byte offset (18 g for block
// g); total: matrix bytes.
__device__ __forceinline__ Q4_0Raw load_q4_0_raw(const uint8_t *__restrict__ W, int64_t o, int64_t total)
{
    Q4_0Raw r;
    r.s = (uint32_t)(o & 3);
    const uint8_t *p = W + (o - r.s);
    r.a = *(const u32x4 *)p;
    // The 5th dword reaches 2 bytes past the block when s == 0; for the last
    // block of the matrix read only its own 2 bytes.
    if (o - r.s + 20 <= total)
        r.e = *(const uint32_t *)(p + 16);
    else
        r.e = *(const uint16_t *)(p + 16);
    return r;
}

__device__ __forceinline__ Q4_0Unit q4_0_unit(const Q4_0Raw &r)
{
    const uint32_t sel = realign_sel(r.s);
    Q4_0Unit u;
    u.q[0] = perm(r.a.y, r.a.x, sel);
    u.q[1] = perm(r.a.z, r.a.y, sel);
    u.q[2] = perm(r.a.w, r.a.z, sel);
    u.q[3] = perm(r.e, r.a.w, sel);
    u.dh = __builtin_amdgcn_alignbyte(r.a.y, r.a.x, r.s) & 0xFFFFu;
    u.d = half_bits_to_float(u.dh);
    return u;
}

__device__ __forceinline__ Q4_0Unit load_q4_0_at(const uint8_t *__restrict__ W, int64_t o, int64_t total)
{
    return q4_0_unit(load_q4_0_raw(W, o, total));
}
// g: block index
__device__ __forceinline__ Q4_0Unit load_q4_0(const uint8_t *__restrict__ W, int64_t g, int64_t total)
{
    return load_q4_0_at(W, g * 18, total);
}

// ---- Q8_0 ------------------------------------------------------------------
struct Q8_0Unit {
    uint32_t q[8];  // byte k of q[i] = qs[4i+k] (int8)
    float d;
    uint32_t dh;    // d as raw f16 bits
};

// The words of one Q8_0 block as loaded (as Q4_0Raw).
struct Q8_0Raw {
    u32x4 a, b;  // the 32 bytes from the block's 4-byte-aligned start
    uint32_t e;  // the next 4 (2 at the end of the matrix)
    uint32_t s;  // the block's offset within a (0 or 2)
};

__device__ __forceinline__ Q8_0Raw load_q8_0_raw(const uint8_t *__restrict__ W, int64_t o, int64_t total)
{
    Q8_0Raw r;
    r.s = (uint32_t)(o & 3);
    const uint8_t *p = W + (o - r.s);
    r.a = *(const u32x4 *)p;
    r.b = *(const u32x4 *)(p + 16);
    if (o - r.s + 36 <= total)
        r.e = *(const uint32_t *)(p + 32);
    else
        r.e = *(const uint16_t *)(p + 32);
    return r;
}

__device__ __forceinline__ Q8_0Unit q8_0_unit(const Q8_0Raw &r)
{
    const uint32_t sel = realign_sel(r.s);
    Q8_0Unit u;
    u.q[0] = perm(r.a.y, r.a.x, sel);
    u.q[1] = perm(r.a.z, r.a.y, sel);
    u.q[2] = perm(r.a.w, r.a.z, sel);
    u.q[3] = perm(r.b.x, r.a.w, sel);
    u.q[4] = perm(r.b.y, r.b.x, sel);
    u.q[5] = perm(r.b.z, r.b.y, sel);
    u.q[6] = perm(r.b.w, r.b.z, sel);
    u.q[7] = perm(r.e, r.b.w, sel);
    u.dh = __builtin_amdgcn_alignbyte(r.a.y, r.a.x, r.s) & 0xFFFFu;
    u.d = half_bits_to_float(u.dh);
    return u;
}

__device__ __forceinline__ Q8_0Unit load_q8_0_at(const uint8_t *__restrict__ W, int64_t o, int64_t total)
{
    return q8_0_unit(load_q8_0_raw(W, o, total));
}
__device__ __forceinline__ Q8_0Unit load_q8_0(const uint8_t *__restrict__ W, int64_t g, int64_t total)
{
    return load_q8_0_at(W, g * 34, total);
}

// ---- Q4_K ------------------------------------------------------------------
// 6-bit scale and min of sub-block j from the 12 packed bytes, in the layout
// of the reference CPU path (quant.c:290-297):
//   j < 4 : sc = s[j] & 63,                       m = s[j+4] & 63
//   j >= 4: sc = ((s[j+4] & 15) << 2) | (s[j-4] >> 6),
//           m  = ((s[j+4] >> 4) << 2) | (s[j] >> 6)
// h1 = scales[0..3], h2 = scales[4..7], h3 = scales[8..11] as little-endian dwords.
__device__ __forceinline__ void q4_k_scale_min(uint32_t h1, uint32_t h2, uint32_t h3, uint32_t j,
                                               uint32_t &sc, uint32_t &mn)
{
    uint32_t sh = (j & 3u) * 8u;
    uint32_t a = (h1 >> sh) & 0xFFu;  // s[j&3]
    uint32_t b = (h2 >> sh) & 0xFFu;  // s[(j&3)+4]
    uint32_t c = (h3 >> sh) & 0xFFu;  // s[(j&3)+8]
    if (j < 4u) {
        sc = a & 63u;
        mn = b & 63u;
    } else {
        sc = ((c & 15u) << 2) | (a >> 6);
        mn = ((c >> 4) << 2) | (b >> 6);
    }
}

struct Q4_KUnit {
    uint32_t q[4];  // qs[16j..16j+15] of the superblock
    float dsc;      // d * sc   (exact in fp32: 11-bit x 6-bit)
    float dmn;      // dmin * m (exact)
};

// u: flat unit index (superblock = u >> 3, sub-block j = u & 7).
__device__ __forceinline__ Q4_KUnit load_q4_k(const uint8_t *__restrict__ W, int64_t u)
{
    const uint8_t *sb = W + (u >> 3) * 144;
    uint32_t j = (uint32_t)(u & 7);
    u32x4 h = *(const u32x4 *)sb;
    u32x4 q = *(const u32x4 *)(sb + 16 + 16 * j);
    uint32_t sc, mn;
    q4_k_scale_min(h.y, h.z, h.w, j, sc, mn);
    Q4_KUnit r;
    r.q[0] = q.x;
    r.q[1] = q.y;
    r.q[2] = q.z;
    r.q[3] = q.w;
    r.dsc = half_bits_to_float(h.x) * (float)sc;
    r.dmn = half_bits_to_float(h.x >> 16) * (float)mn;
    return r;
}

// ---- Q6_K ------------------------------------------------------------------
// 4 dwords of bytes [p, p + 16) for a 2-byte-aligned p inside a 210-byte
// superblock that starts 4-byte aligned or 2 past it: one aligned 16-byte load
// from p rounded down to 4 bytes and one dword after it, realigned.  For the
// runs of a Q6_K superblock read here (ql, qh at offsets up to 176) both loads
// stay inside the superblock or the one before it.
__device__ __forceinline__ void q6_run16(const uint8_t *p, uint32_t (&w)[4])
{
    const uintptr_t a = (uintptr_t)p;
    const uint32_t sh = (uint32_t)(a & 3u);
    const uint32_t *b = (const uint32_t *)(a - sh);
    const uint4 v = *(const uint4 *)b;
    const uint32_t e = b[4];
    w[0] = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    w[1] = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    w[2] = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    w[3] = __builtin_amdgcn_alignbyte(e, v.w, sh);
}

}  // namespace holo
