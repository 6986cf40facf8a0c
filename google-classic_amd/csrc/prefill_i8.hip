// prefill_i8.hip -- the Q8_0 product (holo_gemm_q4_0_q8_0) on the int8 matrix
// cores.
//
// Specification (the same as the f16-MFMA kernel of prefill.hip, restated
// by oracle_gemm_q4_0_q8_0): X quantised per 32-block to Q8_0 (qx, dx) and W
// in Q4_0 (qw, dw); per block b, I = sum_k qx[m,k] * (qw[n,k] - 8) in exact
// integer arithmetic, s = dw * dx (two f16 values, exact in fp32), and
// acc = fmaf(I, s, acc) in block order.  The reference has no batched path
// (its prompt loop multiplies one token at a time, src/ai/llm.c:1049).
//
// Here one v_mfma_i32_32x32x32_i8 gives I for a 32 x 32 tile and a whole
// block: lane (c, h) supplies the 16 activation bytes x[r][16h .. 16h + 15]
// of row r = c and the 16 weight nibbles of column c at the same k, so the
// pairing of operand bytes does not depend on how the matrix core orders k
// inside a lane.  The weights enter as raw nibbles qw (0..15, one AND per
// four); the -8 goes into the accumulator input: C = -8 * sum_k qx[m,k] per
// row, from the panel, so D = I exactly.  s comes from a one-term f16 MFMA
// (A[i][0] = dx[i], B[0][j] = dw[j], every other term zero), which lands in
// the output layout; the epilogue is a convert and an fmaf per output.
//
// Tiling as the exact product's second form (prefill_exact.hip): 64 x 256
// workgroup tiles, wave w takes 64 columns and all 64 rows (2 x 2 tiles of
// 32 x 32); the activation tile (int8 rows, per-block d and C) is shared in
// LDS, S blocks a stage; each lane loads its columns' Q4_0 blocks straight
// into registers through a buffer resource, one stage ahead (an even block
// count per row keeps every row 4-byte aligned, so block b sits 2 (b & 1)
// bytes into its first dword).
#include "common.h"
#include "quant_blocks.h"

#include <limits.h>

namespace holo {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr uint32_t kI8BufWord3 = kRawBufWord3;
constexpr int kI8Mats = 3;

// ---- activation panel: Q8_0 blocks -> int8 rows, d bits, C = -8 sum q ----------
// Block g = m * nb + b: its 32 qx at P + 32 g (so P is the row-major [M][K]
// int8 matrix), its d bits at DH[g], -8 * sum qx at C8[g].
__global__ __launch_bounds__(256) void i8_panel_k(uint4 *__restrict__ P, uint16_t *__restrict__ DH,
                                                  int *__restrict__ C8, const uint8_t *__restrict__ Xq,
                                                  int64_t nblocks, int64_t total)
{
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= nblocks) return;
    const Q8_0Unit u = load_q8_0(Xq, g, total);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) s += (int)(int8_t)(u.q[i] >> (8 * j));
    P[2 * g] = make_uint4(u.q[0], u.q[1], u.q[2], u.q[3]);
    P[2 * g + 1] = make_uint4(u.q[4], u.q[5], u.q[6], u.q[7]);
    DH[g] = (uint16_t)u.dh;
    C8[g] = -8 * s;
}

struct I8Args {
    float *Y[kI8Mats];
    const uint8_t *W[kI8Mats];   // Q4_0 block streams
    int n_end[kI8Mats];          // prefix sums of N_i; unused entries INT_MAX
    const uint8_t *P;            // [M][K] int8
    const uint16_t *DH;          // [M][nb] d bits
    const int *C8;               // [M][nb] -8 * sum qx
    int M, N, nb, ntm, tiles;
};

template <int S>
struct I8Geo {
    static constexpr int RB = S * 32 + 16;     // LDS bytes per activation row (S blocks + pad)
    static constexpr int A = 64 * RB;
    static constexpr int DHO = A;              // d bits [S][64]
    static constexpr int C8O = DHO + S * 64 * 2;  // C [S][64]
    static constexpr int STAGE = (C8O + S * 64 * 4 + 255) & ~255;
    static constexpr int LDS = 2 * STAGE;
};

// The Q4_0 block b of the lane's row, as loaded: 20 bytes from the block's
// start rounded down (P = b & 1: 2 bytes before it for odd b).
struct I8Raw {
    uint32_t w[5];
};

template <int P>
__device__ __forceinline__ I8Raw i8_fetch(__amdgpu_buffer_rsrc_t r, uint32_t vo, int b)
{
    I8Raw x;
    const int so = 18 * b - 2 * P;
    const u32x4 t = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)vo, so, 0));
    x.w[0] = t.x;
    x.w[1] = t.y;
    x.w[2] = t.z;
    x.w[3] = t.w;
    x.w[4] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)vo, so + 16, 0);
    return x;
}

// The B operand (the 16 nibbles of k = 16h .. 16h + 15: the low nibbles of
// qs[0..15] for h = 0, the high ones for h = 1) and the scale MFMA's B
// operand ({dw, 0, 0, 0} in the h = 0 lanes, zeros else); live: the block is
// in range (else dw is zero).
template <int P>
__device__ __forceinline__ void i8_unpack(const I8Raw &x, int h, bool live, v4i &b, v4h &bs)
{
    uint32_t q[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        q[i] = P ? x.w[i + 1] : __builtin_amdgcn_alignbyte(x.w[i + 1], x.w[i], 2);
    const uint32_t sh = 4u * (uint32_t)h;
    b = v4i{(int)((q[0] >> sh) & 0x0F0F0F0Fu), (int)((q[1] >> sh) & 0x0F0F0F0Fu), (int)((q[2] >> sh) & 0x0F0F0F0Fu),
            (int)((q[3] >> sh) & 0x0F0F0F0Fu)};
    const uint32_t dbits = (P ? (x.w[0] >> 16) : (x.w[0] & 0xFFFFu)) & (0u - (uint32_t)(live && h == 0));
    bs = v4h{__builtin_bit_cast(_Float16, (uint16_t)dbits), (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
}

template <int S>
__global__ __launch_bounds__(256, 2) void gemm_q8i8_k(I8Args a)
{
    static_assert(S % 2 == 0, "blocks of a stage alternate in parity: S even");
    using G = I8Geo<S>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, c32 = lane & 31;
    const int nb = a.nb;

    // workgroup -> tile: the workgroups of one XCD take a contiguous run of
    // tiles (the row tiles of a column tile share its weights in that L2)
    const int g = blockIdx.x;
    const int t = (a.tiles & 7) ? g : (g & 7) * (a.tiles >> 3) + (g >> 3);
    const int m0 = (t % a.ntm) * 64, n0 = (t / a.ntm) * 256 + 64 * wave;
    const bool live = n0 < a.N;
    const int nc = min(n0, a.N - 1);
    const int sel = (nc >= a.n_end[0]) + (nc >= a.n_end[1]);
    const uint8_t *Wm = sel == 2 ? a.W[2] : sel == 1 ? a.W[1] : a.W[0];
    float *Ym = sel == 2 ? a.Y[2] : sel == 1 ? a.Y[1] : a.Y[0];
    const int nbase = sel == 2 ? a.n_end[1] : sel == 1 ? a.n_end[0] : 0;
    const int Nm = (sel == 2 ? a.n_end[2] : sel == 1 ? a.n_end[1] : a.n_end[0]) - nbase;
    const int nl = nc - nbase;
    const uint32_t rowb = (uint32_t)nb * 18u;
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void *)Wm, (short)0, (int)((uint32_t)Nm * rowb), kI8BufWord3);
    uint32_t vo[2];
#pragma unroll
    for (int ni = 0; ni < 2; ni++) vo[ni] = (uint32_t)min(nl + 32 * ni + c32, Nm - 1) * rowb;

    // activation staging: 16-byte pieces of [64 rows][S blocks x 32 bytes],
    // piece tid + 256 i (row p / 2S, piece p % 2S); the scales by threads < 64 S
    constexpr int NP = 2 * S;          // pieces per row in a stage
    constexpr int NA = (64 * NP) / 256;  // pieces per thread
    static_assert((64 * NP) % 256 == 0, "pieces split evenly over the threads");
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.P, (short)0, (int)((uint32_t)a.M * (uint32_t)nb * 32u), kI8BufWord3);
    uint32_t aoff[NA], lw[NA];
    int ablk[NA];
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int pc = tid + 256 * i, r = pc / NP, c = pc % NP;
        aoff[i] = (uint32_t)min(m0 + r, a.M - 1) * (uint32_t)(nb * 32) + (uint32_t)(c & 1) * 16u;
        ablk[i] = c >> 1;
        lw[i] = (uint32_t)(r * G::RB + c * 16);
    }
    // scale entry (tid mod 64 S) of the stage: with S = 2 two threads stage each
    // one, the same value, and no thread branches (a divergent branch here splits
    // the stage's code and the scheduler then keeps every block's results live)
    const int sidx = tid % (64 * S);
    const int srow = min(m0 + (sidx & 63), a.M - 1), sblk = sidx >> 6;
    v4u sa[NA];
    uint32_t sdh = 0;
    int sc8 = 0;
    auto fetch_a = [&](int kb) {
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const uint32_t o = aoff[i] + (uint32_t)min(kb + ablk[i], nb - 1) * 32u;
            sa[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rp, (int)o, 0, 0));
        }
        const int64_t gi = (int64_t)srow * nb + min(kb + sblk, nb - 1);
        sdh = a.DH[gi];
        sc8 = a.C8[gi];
    };
    auto stash_a = [&](int buf) {
        uint8_t *base = lds + buf * G::STAGE;
#pragma unroll
        for (int i = 0; i < NA; i++) *(v4u *)(base + lw[i]) = sa[i];
        ((uint16_t *)(base + G::DHO))[sidx] = (uint16_t)sdh;  // [S][64]
        ((int *)(base + G::C8O))[sidx] = sc8;
    };

    v16f acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;

    const int nst = (nb + S - 1) / S;
    I8Raw ring[S][2];
#pragma unroll
    for (int s = 0; s < S; s++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) ring[s][ni] = (s & 1) ? i8_fetch<1>(rw, vo[ni], s) : i8_fetch<0>(rw, vo[ni], s);
    fetch_a(0);
    stash_a(0);
    fetch_a(S);
    __syncthreads();
    for (int st = 0; st < nst; st++) {
        const uint8_t *base = lds + (st & 1) * G::STAGE;
#pragma unroll
        for (int s = 0; s < S; s++) {
            const int b = st * S + s;
            // this block's weight operands, then its ring slot fetches block
            // b + S (past the row's end: the next row, or zeros past the
            // matrix; never used)
            v4i bq[2];
            v4h bs[2];
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                if (s & 1) {
                    i8_unpack<1>(ring[s][ni], h, b < nb, bq[ni], bs[ni]);
                    ring[s][ni] = i8_fetch<1>(rw, vo[ni], b + S);
                } else {
                    i8_unpack<0>(ring[s][ni], h, b < nb, bq[ni], bs[ni]);
                    ring[s][ni] = i8_fetch<0>(rw, vo[ni], b + S);
                }
            }
#pragma unroll
            for (int mi = 0; mi < 2; mi++) {
                const int r = 32 * mi + c32;
                const v4i aq = __builtin_bit_cast(v4i, *(const v4u *)(base + r * G::RB + s * 32 + 16 * h));
                const uint16_t dx = ((const uint16_t *)(base + G::DHO))[s * 64 + r];
                const v4h as = v4h{__builtin_bit_cast(_Float16, (uint16_t)(h ? 0 : dx)), (_Float16)0.0f,
                                   (_Float16)0.0f, (_Float16)0.0f};
                // C = -8 sum qx of the lane's rows 4h + 8q + j (register 4q + j)
                v16i c8;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4i v = *(const v4i *)(base + G::C8O + (s * 64 + 32 * mi + 8 * q + 4 * h) * 4);
                    c8[4 * q] = v.x;
                    c8[4 * q + 1] = v.y;
                    c8[4 * q + 2] = v.z;
                    c8[4 * q + 3] = v.w;
                }
#pragma unroll
                for (int ni = 0; ni < 2; ni++) {
                    const v16i dot = __builtin_amdgcn_mfma_i32_32x32x32_i8(aq, bq[ni], c8, 0, 0, 0);
                    const v16f zero = {};
                    const v16f sc = __builtin_amdgcn_mfma_f32_32x32x8f16(as, bs[ni], zero, 0, 0, 0);
#pragma unroll
                    for (int rr = 0; rr < 16; rr++)
                        acc[mi][ni][rr] = __builtin_fmaf((float)dot[rr], sc[rr], acc[mi][ni][rr]);
                }
            }
        }
        stash_a((st + 1) & 1);
        fetch_a((st + 2) * S);
        __syncthreads();
    }

#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
            const int n = nl + 32 * ni + c32;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + 32 * mi + (r & 3) + 4 * h + 8 * (r >> 2);
                if (live && m < a.M && n < Nm) Ym[(int64_t)m * Nm + n] = acc[mi][ni][r];
            }
        }
}

}  // namespace

// Panel bytes of the int8 form: [M][K] int8, [M][nb] d bits, [M][nb] C.
size_t q8i8_panel_bytes(int M, int K)
{
    const size_t nblk = (size_t)M * (K / 32);
    return nblk * 32 + ((nblk * 2 + 255) & ~(size_t)255) + nblk * 4;
}

// Whether the int8 form takes the product: an even block count per row (the
// weight rows 4-byte aligned), 4-byte aligned matrices, every N_i but the
// last a multiple of 64 (a wave's columns in one matrix), each matrix and the
// int8 panel under 2 GiB (32-bit offsets).
bool q8i8_fits(const void *const *W, const int *N, int nmat, int M, int K)
{
    const int nb = K / 32;
    if (nb % 2 || (int64_t)M * K >= (1LL << 31)) return false;
    for (int i = 0; i < nmat; i++) {
        if (((uintptr_t)W[i]) & 3u) return false;
        if (i < nmat - 1 && N[i] % 64) return false;
        if ((int64_t)N[i] * nb * 18 >= (1LL << 31)) return false;
    }
    return true;
}

// Y[i] = the Q8_0 product of Xq (M x K, Q8_0 blocks) and W[i] (Q4_0), on the
// int8 matrix cores; ws: at least q8i8_panel_bytes(M, K).
void q8i8_product(float *const *Y, const void *const *W, const int *N, int nmat, const void *Xq, int M, int K,
                  void *ws)
{
    constexpr int S = 2;
    using G = I8Geo<S>;
    const int nb = K / 32;
    const int64_t nblk = (int64_t)M * nb;
    uint8_t *P = (uint8_t *)ws;
    uint16_t *DH = (uint16_t *)(P + nblk * 32);
    int *C8 = (int *)((uint8_t *)DH + ((nblk * 2 + 255) & ~(int64_t)255));
    hipLaunchKernelGGL(i8_panel_k, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, stream(), (uint4 *)P, DH, C8,
                       (const uint8_t *)Xq, nblk, nblk * 34);
    HOLO_LAUNCH_CHECK();
    I8Args a = {};
    int acc = 0;
    for (int i = 0; i < kI8Mats; i++) {
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
    a.P = P;
    a.DH = DH;
    a.C8 = C8;
    a.M = M;
    a.N = acc;
    a.nb = nb;
    a.ntm = (M + 63) / 64;
    a.tiles = a.ntm * ((acc + 255) / 256);
    auto kern = gemm_q8i8_k<S>;
    static bool attr = false;
    if (!attr) {
        HOLO_CHECK(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS));
        attr = true;
    }
    launch_timed(kern, dim3(a.tiles), dim3(256), G::LDS, a);
    HOLO_LAUNCH_CHECK();
}

}  // namespace holo
