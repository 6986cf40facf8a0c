// gemv.hip -- fused dequant + matrix-vector product over GGUF Q8_0, Q4_0 and
// Q4_K blocks with fp32 activations and fp32 accumulation (decode path).
//
// Replaces cuda_matmul_q8_0 / q4_0 / q4_k and the two fused Q8_0 multi-GEMVs
// of the reference (src/ai/cuda_ops.cu:1132-1175, 1184-1395).  The reference
// CPU path (src/ai/llm.c:770-926, src/ai/quant.c:541-633) defines the result.
//
// Work mapping (wave64):
//   * lane <-> one 32-weight unit of a row (Q8_0/Q4_0 block, Q4_K sub-block);
//     the 64 lanes of a wave read 64 consecutive units of one row, so each
//     load instruction covers one contiguous run of the row (1152 B for
//     Q4_0, 2176 B for Q8_0, 8 superblocks for Q4_K);
//   * a wave owns a task of R rows and walks the row in 64-unit segments;
//     the lane's 32 activations are read once per segment and reused for
//     the R rows;
//   * activations are staged once per workgroup in LDS (16-byte chunks
//     XOR-swizzled within each unit so a ds_read_b128 of 8 neighbouring lanes
//     hits distinct banks), together with the per-unit sum of activations;
//   * the quant offset is folded out of the inner loop:
//       Q4_0  d * (sum q*x - 8 * sum x)
//       Q8_0  d * (sum (q+128)*x - 128 * sum x)   (q+128 = byte ^ 0x80)
//       Q4_K  (d*sc) * sum q*x - (dmin*m) * sum x
//     so the inner loop is unpack, v_cvt_f32_ubyte and one FMA per weight;
//   * the R row sums are reduced across the wave with DPP.
#include "common.h"
#include "quant_blocks.h"

namespace holo {

enum Fmt { FMT_Q4_0 = 0, FMT_Q8_0 = 1, FMT_Q4_K = 2 };
enum Mode { MODE_PLAIN = 0, MODE_GATEUP = 1 };

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxSeg = 3;

struct GemvArgs {
    const uint8_t *W[kMaxSeg];
    float *y[kMaxSeg];
    int64_t bytes[kMaxSeg];
    int rows[kMaxSeg];
    int task_end[kMaxSeg];  // inclusive prefix sums of tasks per segment
    int nseg;
    int ntasks;
    const float *x;
    int units;  // 32-weight units per row
};

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_shift_add(float v)
{
    int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false);
    return v + __int_as_float(t);
}

// Sum over the 64 lanes; the result is returned in every lane.
__device__ __forceinline__ float wave_sum(float v)
{
    v = dpp_shift_add<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_shift_add<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_shift_add<0x141, 0xF>(v);  // row_half_mirror
    v = dpp_shift_add<0x140, 0xF>(v);  // row_mirror: every lane of a row holds its row sum
    v = dpp_shift_add<0x142, 0xA>(v);  // row_bcast:15 -> rows 1, 3
    v = dpp_shift_add<0x143, 0xC>(v);  // row_bcast:31 -> rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Hides a value's known bits from the optimiser, so that
// (float)((v >> 8k) & 0xFF) selects v_cvt_f32_ubyte{k} instead of being
// narrowed to a 4-bit v_bfe_u32 plus v_cvt_f32_ubyte0 (one op per weight
// instead of two).  Emits no instruction.
__device__ __forceinline__ void opaque(uint32_t &v) { asm volatile("" : "+v"(v)); }

// Dot of one unit's 32 nibbles with its 32 activations: sum q*x, q in 0..15.
__device__ __forceinline__ float nib_dot(const uint32_t (&q)[4], const float4 (&x)[8])
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

// sum (q+128)*x over a Q8_0 unit, q int8 stored in bytes.
__device__ __forceinline__ float byte_dot(const uint32_t (&q)[8], const float4 (&x)[8])
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

template <int FMT>
__device__ __forceinline__ float unit_dot(const uint8_t *__restrict__ W, int64_t bytes, int64_t gunit,
                                          const float4 (&x)[8], float sx)
{
    if constexpr (FMT == FMT_Q4_0) {
        Q4_0Unit u = load_q4_0(W, gunit, bytes);
        return u.d * fmaf(-8.0f, sx, nib_dot(u.q, x));
    } else if constexpr (FMT == FMT_Q8_0) {
        Q8_0Unit u = load_q8_0(W, gunit, bytes);
        return u.d * fmaf(-128.0f, sx, byte_dot(u.q, x));
    } else {
        Q4_KUnit u = load_q4_k(W, gunit);
        return fmaf(u.dsc, nib_dot(u.q, x), -u.dmn * sx);
    }
}

// x staged in LDS: unit u occupies 8 float4 chunks; chunk c sits at slot
// c ^ (u & 7).  sx[u] = sum of the unit's 32 activations (fixed order).
template <bool XLDS>
struct XSource;

template <>
struct XSource<true> {
    const float4 *lx;
    const float *lsx;
    __device__ __forceinline__ void get(int u, float4 (&x)[8], float &sx) const
    {
        const float4 *p = lx + u * 8;
        int sw = u & 7;
#pragma unroll
        for (int c = 0; c < 8; c++) x[c] = p[c ^ sw];
        sx = lsx[u];
    }
};

template <>
struct XSource<false> {
    const float *gx;
    __device__ __forceinline__ void get(int u, float4 (&x)[8], float &sx) const
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

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int FMT, int R, int MODE, bool XLDS>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs args)
{
    extern __shared__ float4 lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int units = args.units;

    XSource<XLDS> xs;
    if constexpr (XLDS) {
        float *lsx = (float *)(lds + units * 8);
        for (int i = tid; i < units * 8; i += kThreads) {
            int u = i >> 3, c = i & 7;
            const float *g = args.x + (int64_t)i * 4;
            lds[u * 8 + (c ^ (u & 7))] = make_float4(g[0], g[1], g[2], g[3]);
        }
        __syncthreads();
        for (int u = tid; u < units; u += kThreads) {
            const float4 *p = lds + u * 8;
            float s = 0.f;
#pragma unroll
            for (int c = 0; c < 8; c++) {
                float4 v = p[c ^ (u & 7)];
                s += (v.x + v.y) + (v.z + v.w);
            }
            lsx[u] = s;
        }
        __syncthreads();
        xs.lx = lds;
        xs.lsx = lsx;
    } else {
        xs.gx = args.x;
    }

    const int nsegs = (units + 63) >> 6;
    for (int task = blockIdx.x * kWaves + wave; task < args.ntasks; task += gridDim.x * kWaves) {
        int seg = 0;
        int tbase = 0;
        if constexpr (MODE == MODE_PLAIN) {
            while (seg + 1 < args.nseg && task >= args.task_end[seg]) {
                tbase = args.task_end[seg];
                seg++;
            }
        }
        const int rows = args.rows[seg];
        const int row0 = (task - tbase) * R;
        constexpr int NM = MODE == MODE_GATEUP ? 2 : 1;

        float acc[NM][R];
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
            for (int r = 0; r < R; r++) acc[m][r] = 0.f;

        for (int sg = 0; sg < nsegs; sg++) {
            int u = sg * 64 + lane;
            bool active = u < units;
            int uc = active ? u : units - 1;
            float4 x[8];
            float sx;
            xs.get(uc, x, sx);
#pragma unroll
            for (int m = 0; m < NM; m++) {
                const int mi = MODE == MODE_GATEUP ? m : seg;
                const uint8_t *W = args.W[mi];
                const int64_t bytes = args.bytes[mi];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    int row = min(row0 + r, rows - 1);
                    float v = unit_dot<FMT>(W, bytes, (int64_t)row * units + uc, x, sx);
                    acc[m][r] += active ? v : 0.f;
                }
            }
        }

#pragma unroll
        for (int r = 0; r < R; r++) {
            float s0 = wave_sum(acc[0][r]);
            if constexpr (MODE == MODE_GATEUP) {
                float s1 = wave_sum(acc[1][r]);
                if (lane == 0 && row0 + r < rows) args.y[0][row0 + r] = silu(s0) * s1;
            } else {
                if (lane == 0 && row0 + r < rows) args.y[seg][row0 + r] = s0;
            }
        }
    }
}

// ---- host side ---------------------------------------------------------------

constexpr int kMaxLdsBytes = 64 * 1024;

struct Tuning {
    int max_wg_per_cu = 8;
};
static Tuning g_tuning;

static int units_per_row(int fmt, int in_dim)
{
    if (fmt == FMT_Q4_K) return (in_dim / 256) * 8;
    return in_dim / 32;
}

static int64_t row_bytes(int fmt, int in_dim)
{
    if (fmt == FMT_Q4_0) return (int64_t)(in_dim / 32) * 18;
    if (fmt == FMT_Q8_0) return (int64_t)(in_dim / 32) * 34;
    return (int64_t)(in_dim / 256) * 144;
}

template <int FMT, int R, int MODE>
static void launch_t(GemvArgs &a)
{
    size_t lds = (size_t)a.units * (128 + 4);
    int blocks = (a.ntasks + kWaves - 1) / kWaves;
    int cap = num_cus() * g_tuning.max_wg_per_cu;
    if (blocks > cap) blocks = cap;
    if (lds <= (size_t)kMaxLdsBytes)
        hipLaunchKernelGGL((gemv_kernel<FMT, R, MODE, true>), dim3(blocks), dim3(kThreads), lds, stream(), a);
    else
        hipLaunchKernelGGL((gemv_kernel<FMT, R, MODE, false>), dim3(blocks), dim3(kThreads), 0, stream(), a);
    HOLO_LAUNCH_CHECK();
}

constexpr int kRows = 4;

static bool check_ptr(const void *p, const char *what)
{
    if (((uintptr_t)p & 3u) != 0) {
        HOLO_REJECT(what);
        return false;
    }
    return true;
}

// One launch over up to three matrices sharing x and in_dim.
static void gemv_multi(int fmt, int mode, int nseg, const void *const *W, float *const *y, const int *rows,
                       const float *x, int in_dim)
{
    GemvArgs a = {};
    a.units = units_per_row(fmt, in_dim);
    a.x = x;
    a.nseg = nseg;
    int tasks = 0;
    for (int s = 0; s < nseg; s++) {
        if (!check_ptr(W[s], "weight matrix must be 4-byte aligned")) return;
        a.W[s] = (const uint8_t *)W[s];
        a.y[s] = y[s];
        a.rows[s] = rows[s];
        a.bytes[s] = row_bytes(fmt, in_dim) * rows[s];
        if (mode == MODE_PLAIN) tasks += (rows[s] + kRows - 1) / kRows;
        a.task_end[s] = tasks;
    }
    if (mode == MODE_GATEUP) tasks = (rows[0] + kRows - 1) / kRows;
    a.ntasks = tasks;
    if (tasks == 0) return;
    if (a.units == 0) {
        // No complete block per row: every dot product is empty.
        for (int s = 0; s < (mode == MODE_GATEUP ? 1 : nseg); s++)
            HOLO_CHECK(hipMemsetAsync(y[s], 0, sizeof(float) * rows[s], stream()));
        return;
    }
    if (fmt == FMT_Q4_0) {
        if (mode == MODE_PLAIN) launch_t<FMT_Q4_0, kRows, MODE_PLAIN>(a);
        else launch_t<FMT_Q4_0, kRows, MODE_GATEUP>(a);
    } else if (fmt == FMT_Q8_0) {
        if (mode == MODE_PLAIN) launch_t<FMT_Q8_0, kRows, MODE_PLAIN>(a);
        else launch_t<FMT_Q8_0, kRows, MODE_GATEUP>(a);
    } else {
        if (mode == MODE_PLAIN) launch_t<FMT_Q4_K, kRows, MODE_PLAIN>(a);
        else launch_t<FMT_Q4_K, kRows, MODE_GATEUP>(a);
    }
}

static void gemv_one(int fmt, float *dst, const void *M, const float *v, int out_dim, int in_dim)
{
    if (out_dim <= 0) return;
    if (!M) {
        // matmul_q with a NULL matrix writes zeros (llm.c:772-775).
        HOLO_CHECK(hipMemsetAsync(dst, 0, sizeof(float) * out_dim, stream()));
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
