/*
 * synth.c -- deterministic synthetic GGUF blocks and activations (host C).
 *
 * The reference ships no model files or fixtures, so every input of the
 * tests and of bench.py comes from this generator.  It is language-neutral:
 *
 *   mix64(z)         the SplitMix64 finaliser
 *                    z ^= z>>30; z *= 0xBF58476D1CE4E5B9;
 *                    z ^= z>>27; z *= 0x94D049BB133111EB; z ^= z>>31
 *   stream(seed, i)  state s = mix64(seed ^ mix64(i + 1)); next() is one
 *                    SplitMix64 step: s += 0x9E3779B97F4A7C15; return mix64(s)
 *                    Block i of a tensor (or element i of a vector) draws
 *                    only from stream(seed, i), so generation is parallel
 *                    and any block can be regenerated alone.
 *   uniform byte     bytes of next(), least significant first
 *   int in [-127,127] bytes 0..254 accepted as byte-127, 255 rejected
 *   N(0,1)           Box-Muller in double: u1 = 1 - (next()>>11)*2^-53,
 *                    u2 = (next()>>11)*2^-53, z = sqrt(-2 ln u1) cos(2 pi u2)
 *   f16 scale        f16_rne((float)(|z| * c)), c = 0.01 or 0.02
 *
 * Block contents follow the configurations of the benchmark:
 *   Q8_0  d = f16(|N|*0.01), qs[32] uniform in [-127,127]
 *   Q4_0  d = f16(|N|*0.02), qs[16] uniform bytes (two uniform nibbles)
 *   Q4_K  d, dmin = f16(|N|*0.01) (d first), scales[12] uniform bytes,
 *         qs[128] uniform bytes
 *   Q6_K  d = f16(|N|*0.01), ql/qh uniform bytes, scales[16] uniform int8
 *         in [-127,127]
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint64_t mix64(uint64_t z)
{
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ULL;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBULL;
    z ^= z >> 31;
    return z;
}

typedef struct { uint64_t s; uint64_t bits; int nbytes; } rng_t;

static inline void rng_init(rng_t *r, uint64_t seed, uint64_t i)
{
    r->s = mix64(seed ^ mix64(i + 1));
    r->bits = 0;
    r->nbytes = 0;
}

static inline uint64_t rng_next(rng_t *r)
{
    r->s += 0x9E3779B97F4A7C15ULL;
    return mix64(r->s);
}

static inline uint8_t rng_byte(rng_t *r)
{
    if (r->nbytes == 0) {
        r->bits = rng_next(r);
        r->nbytes = 8;
    }
    uint8_t b = (uint8_t)(r->bits & 0xFF);
    r->bits >>= 8;
    r->nbytes--;
    return b;
}

static inline int8_t rng_i127(rng_t *r)
{
    for (;;) {
        uint8_t b = rng_byte(r);
        if (b != 255) return (int8_t)((int)b - 127);
    }
}

static inline double rng_normal(rng_t *r)
{
    double u1 = 1.0 - (double)(rng_next(r) >> 11) * 0x1.0p-53;
    double u2 = (double)(rng_next(r) >> 11) * 0x1.0p-53;
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925286766559 * u2);
}

/* f32 -> f16 bits, round to nearest even, subnormals and overflow handled. */
uint16_t holo_synth_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u)
        return (uint16_t)(sign | (ax == 0x7F800000u ? 0x7C00u : (0x7E00u | ((ax >> 13) & 0x3FFu))));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t sh = 126u - e;  /* value = m * 2^(e-150) = (m >> sh) * 2^-24 */
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static inline uint16_t scale_f16(rng_t *r, double c)
{
    return holo_synth_f32_to_f16((float)(fabs(rng_normal(r)) * c));
}

static inline void put16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

void holo_synth_q8_0(void *dst, int64_t n_blocks, uint64_t seed)
{
    uint8_t *out = (uint8_t *)dst;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < n_blocks; b++) {
        rng_t r;
        rng_init(&r, seed, (uint64_t)b);
        uint8_t *p = out + b * 34;
        put16(p, scale_f16(&r, 0.01));
        for (int j = 0; j < 32; j++) p[2 + j] = (uint8_t)rng_i127(&r);
    }
}

void holo_synth_q4_0(void *dst, int64_t n_blocks, uint64_t seed)
{
    uint8_t *out = (uint8_t *)dst;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < n_blocks; b++) {
        rng_t r;
        rng_init(&r, seed, (uint64_t)b);
        uint8_t *p = out + b * 18;
        put16(p, scale_f16(&r, 0.02));
        for (int j = 0; j < 16; j++) p[2 + j] = rng_byte(&r);
    }
}

void holo_synth_q4_k(void *dst, int64_t n_blocks, uint64_t seed)
{
    uint8_t *out = (uint8_t *)dst;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < n_blocks; b++) {
        rng_t r;
        rng_init(&r, seed, (uint64_t)b);
        uint8_t *p = out + b * 144;
        put16(p, scale_f16(&r, 0.01));
        put16(p + 2, scale_f16(&r, 0.01));
        for (int j = 0; j < 12; j++) p[4 + j] = rng_byte(&r);
        for (int j = 0; j < 128; j++) p[16 + j] = rng_byte(&r);
    }
}

void holo_synth_q6_k(void *dst, int64_t n_blocks, uint64_t seed)
{
    uint8_t *out = (uint8_t *)dst;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < n_blocks; b++) {
        rng_t r;
        rng_init(&r, seed, (uint64_t)b);
        uint8_t *p = out + b * 210;
        uint16_t d = scale_f16(&r, 0.01);
        for (int j = 0; j < 192; j++) p[j] = rng_byte(&r);
        for (int j = 0; j < 16; j++) p[192 + j] = (uint8_t)rng_i127(&r);
        put16(p + 208, d);
    }
}

/* N(0,1) fp32, element i from stream(seed, i). */
void holo_synth_normal_f32(float *dst, int64_t n, uint64_t seed)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        rng_t r;
        rng_init(&r, seed, (uint64_t)i);
        dst[i] = (float)rng_normal(&r);
    }
}

/* Seed of one tensor: mix64 over (base seed, config, layer, matrix). */
uint64_t holo_synth_tensor_seed(uint64_t base, uint32_t config, uint32_t layer, uint32_t matrix)
{
    uint64_t z = mix64(base ^ 0x5851F42D4C957F2DULL);
    z = mix64(z ^ ((uint64_t)config << 40) ^ ((uint64_t)layer << 16) ^ (uint64_t)matrix);
    return z;
}
