// gemv_stream.hip -- a whole chain of dependent GEMV stages (a decode step:
// every layer's q/k/v, o, gate/up and down) in one persistent launch that
// keeps the weight stream running across the stage boundaries.
//
// The reference issues one launch per matrix and token (the decode loop of
// src/ai/llm_cuda.c:604-918; kernels cuda_ops.cu:618-676, 976-1060); the
// results here are those of separate GEMVs (int8 planes of the activations
// in 22-bit fixed point, exact int32 block dots, fp32 accumulation), with
// the rms_norm of the stage's input folded into its staging (or into the
// output scale, below) and the residual add into its stores.  The planes'
// scale runs per 16 activations (two per 32-weight block, against one in the
// separate GEMV kernels), so a 16-row tile of outputs owns whole scale
// groups of the next stage's input.
//
// Why one launch: a GEMV launch pays its ramp (dispatch, activation staging,
// the first HBM round trip of its weights) and its tail (the slowest
// workgroup), and a decode step's stages depend on each other, so those
// costs add up stage after stage.  Here the weight loads do not wait for
// the stage boundary: weights do not depend on the activations, so each
// compute wave keeps D items of its own future work in flight in registers
// and issues the next one as soon as a register set frees, whatever stage it
// belongs to.  While the grid synchronises between two stages, the weight
// stream for the next stage keeps arriving.
//
// Workgroup (one per CU, all resident): 8 compute waves and 1 control wave.
//   compute wave w  items of its tiles (an item is 16 rows x one 16-unit
//                   segment, as the MFMA GEMV), dots on v_mfma_i32_16x16x64_i8,
//                   one partial per row and tile into LDS; it never stores to
//                   global memory, so its vector-memory counter holds only
//                   loads and each item's wait is exact.  A tile is 16 output
//                   rows: 16 rows of the matrices (plain), or 16 gate and the
//                   same 16 up rows (gate/up: a gate item and an up item per
//                   segment).
//   control wave    at a stage's end: sums the 8 partials of each of the
//                   workgroup's rows (64 rows at a time, one per lane), applies
//                   the epilogue (silu(g)*u, or r + acc), stores the outputs,
//                   then gathers the next stage's input.  It issues no weight
//                   loads.
//
// How a stage's output reaches the next stage (no grid barrier): besides the
// plain fp32 output, every output value is also stored as one 64-bit word
// ((tag ^ value bits) << 32 | value bits) with a single agent-scope store, into the plan's
// exchange buffer of that output vector.  The tag names the launch and the
// stage (base + s + 1, base = launch count * (stages + 1)), so a word is
// either this stage's value or visibly stale.  When a later stage is the
// designated reader of the output (the first stage that reads it as x), the
// producer also stores, per 16 outputs, a plane record: the 16 values
// already in the reader's int8 planes (times the reader's norm weight),
// their scale and sums, 16 exchange words.  The reader then only copies
// words into place, instead of every CU converting the whole vector.  A
// consumer copies the words of its whole input into LDS (device-coherent
// global_load_lds), checks every tag and copies again until all are current.
// Value and tag travel in one single-copy-atomic 64-bit store, and the high
// half carries the tag XORed with the value, so a word that checks as
// current holds the current value even if a 16-byte copy paired the halves
// of two stores: no fence, no store-completion wait and no arrival counter
// sit between a producer's epilogue and its consumers.  The
// launch count advances when the last workgroup of a launch ends (a counter
// in the plan), so the next launch's tags differ from every word this launch
// left behind.
//
// Stage boundary (3 workgroup barriers): A  all partials of stage s in LDS;
// the control wave stores, then gathers the input of stage s+1 (and its norm
// weight) into LDS, in the space of the compute waves' item stages, which are
// idle until C; B  the input is in LDS; all waves place the plane records (or
// convert fp32 input: rms_norm if asked, then the int8 planes); C  compute
// resumes.  The compute waves never load activations, so nothing but their
// own weight items counts against their vector-memory counter.
#include "gemv_mfma.h"

#include <hip/hip_ext.h>
#include <limits.h>

#include <vector>

namespace holo {

namespace {

constexpr int kNCW = 8;                      // compute waves
constexpr int kStreamThreads = 64 * (kNCW + 1);
constexpr int kStreamMaxTiles = 16;          // tiles (16 output rows) of one stage per workgroup
constexpr uint32_t kStreamPolls = 1u << 18;  // bounded exchange wait (~0.3 s)
constexpr int kRecWords = 16;                // exchange words of a plane record (16 values)

// Staged activations of a stage in LDS, per 32-value unit u: the three int8
// planes (96 bytes at 96 u, as the MFMA GEMV stages them) and, at 96 units +
// 16 u, the unit's scales {dx of values 0-15, dx of values 16-31, sum of
// values 0-15, sum of values 16-31}.
constexpr int kUnitLds = 96 + 16;

// One stage of the plan, in device memory (read with scalar loads).
struct StreamStage {
    uint64_t W[3];        // matrices (gate/up: gate, up)
    uint64_t y[3];        // outputs (gate/up: y[0])
    uint64_t x;           // input vector, units * 32 floats
    uint64_t nw;          // rms-norm weight (units * 32 floats) or 0
    uint64_t r;           // residual: y[0] = r + W x (plain, one matrix), or 0
    int64_t row_bytes;
    int row_end[3];       // prefix sums of the matrices' rows (plain); INT_MAX unused
    int ystart[3];        // output rows below this are written again by a later stage of the
                          // plan: no plain store for them (exchange words only)
    int mode;             // MODE_PLAIN / MODE_GATEUP
    int units;            // 32-weight units per row
    int G;                // 16-unit segments per row
    int NI;               // items per tile: G (plain), 2 G (gate/up: gate items, then up items)
    int P;                // item slots per compute wave per tile: ceil(NI / kNCW)
    int total_rows;       // output rows (plain: of all matrices; gate/up: of h)
    int full_tiles;       // tiles dealt round robin to every workgroup
    int rem_start;        // first row of the remainder (dealt in 16-row tiles)
    float eps;
    uint64_t dup;         // gate/up: up base minus gate base
    uint64_t lly[3];      // exchange words of the outputs (gate/up: lly[0])
    uint64_t llp[3];      // plane records of an output for its designated reader, or 0
    uint64_t pnw[3];      // that reader's norm weight, or 0
    uint64_t llx;         // exchange words of x when an earlier stage wrote it, else 0
    uint64_t lpx;         // plane records of x when this stage is their designated reader, else 0
    uint64_t llr;         // exchange words of r when an earlier stage wrote it, else 0
    int xsrc, rsrc;       // the stage that wrote x / r last before this one
};

// The stage table is read through the constant address space: its loads are
// then scalar (the kernel's own global stores cannot make the compiler fall
// back to vector loads, whose waits would also drain the weight ring).
typedef __attribute__((address_space(4))) const StreamStage cstage;

struct StreamArgs {
    uint64_t table;       // device address of the stage table (read as cstage)
    uint64_t slots;       // device address of int[grid]: item slots per compute
                          // wave of each workgroup, rounded up to a multiple of D
    int nstages;
    uint32_t *seq;        // [0] launches so far, [64] workgroups done in this launch,
                          // [128 + b] the tag of the last stage workgroup b stored
    uint32_t *flag;       // set when an exchange wait gives up
    uint32_t zero_off;    // LDS: zero region (after the largest stage's planes)
    uint32_t stage_off;   // LDS: the compute waves' item stages
    uint32_t tpart_off;   // LDS: tile partials [kStreamMaxTiles][kNCW][32]
    uint32_t red_off;     // LDS: reductions, tag base, stale-piece masks [kRedWords]
    uint32_t pack_off;    // LDS: the control wave's plane bytes [64]
    uint32_t ss_off;      // LDS: sums of squares of a plane-record input [2 units]
    uint32_t xbuf_off;    // LDS: x of the next stage (fp32 or words), then its norm weight
};

__device__ __forceinline__ cstage &stage_at(const StreamArgs &a, int s) { return ((cstage *)(uintptr_t)a.table)[s]; }

// Wave-uniform by construction; readfirstlane tells the compiler, so stage
// table reads become scalar loads (a vector load would need a vmcnt wait
// that also drains the compute waves' weight ring).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint64_t uni64(uint64_t v)
{
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ float unif(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// The remainder rows of workgroup b (rem = total - rem_start < 16 W): tile
// [b * nt / W, (b + 1) * nt / W) of the nt = ceil(rem / 16) 16-row tiles, at
// most one.  Every tile starts at a multiple of 16, so a tile's outputs form
// whole plane-record groups.  (Splitting the remainder into equal runs of
// rows balances the HBM bytes better, but a short tile costs the compute
// waves as much as a full one; measured on the decode chain, the 16-row
// tiles are faster.)
__host__ __device__ inline void rem_rows(int total, int rem_start, uint32_t W, uint32_t b, int &e0, int &e1)
{
    const uint32_t nt = (uint32_t)(total - rem_start + 15) / 16u;
    e0 = rem_start + 16 * (int)((b * nt) / W);
    e1 = min(rem_start + 16 * (int)(((b + 1) * nt) / W), total);
}

// This workgroup's tiles of a stage: F full tiles dealt round robin (tile k
// = global tile k*W + b), then at most one remainder tile.
struct Tiles {
    int F, ex0, ex1, n;
    __device__ __forceinline__ void init(cstage &s, uint32_t W, uint32_t b)
    {
        F = uni(s.full_tiles);
        int e0, e1;
        rem_rows(s.total_rows, s.rem_start, W, b, e0, e1);
        ex0 = uni(e0);
        ex1 = uni(e1);
        n = uni(F + (ex1 > ex0 ? 1 : 0));
    }
    __device__ __forceinline__ void rows(int k, uint32_t W, uint32_t b, int &row0, int &rend) const
    {
        if (k < F) {
            row0 = (k * (int)W + (int)b) * 16;
            rend = row0 + 16;
        } else {
            row0 = ex0;
            rend = ex1;
        }
    }
};

__device__ __forceinline__ void split_row(cstage &s, int v, int &m, int &r)
{
    const int re0 = uni(s.row_end[0]), re1 = uni(s.row_end[1]);
    const int a1 = v >= re0, a2 = v >= re1;
    m = a1 + a2;
    r = v - (a2 ? re1 : a1 ? re0 : 0);
}

// A compute wave's walk over its item slots, in order: stage s, tile k of
// this workgroup's n tiles, slot p < P of the tile (item cw + kNCW * p).
// Tracked incrementally (no division per slot); the stage constants are
// read once per stage, into scalar registers.  A stage with no tile for this
// workgroup is skipped; s = nstages is past the end, where the issue fields
// are those of the last stage (the dummy loads read its first item).
struct Walk {
    int s, k, p;
    int n, P, G, NI, F, units;
    int row0, rend, ex0, ex1;

    __device__ __forceinline__ void set_tile(uint32_t W, uint32_t b)
    {
        if (k < F) {
            row0 = uni((k * (int)W + (int)b) * 16);
            rend = row0 + 16;
        } else {
            row0 = ex0;
            rend = ex1;
        }
    }
    __device__ __forceinline__ void enter(const StreamArgs &a, int stage, uint32_t W, uint32_t b)
    {
        // locals, assigned to the members once: a loop over the members
        // themselves keeps the struct in scratch memory
        int ss = stage, f = 0, e0 = 0, e1 = 0, nn = 0;
        for (; ss < a.nstages; ss++) {
            cstage &st = stage_at(a, ss);
            f = st.full_tiles;
            rem_rows(st.total_rows, st.rem_start, W, b, e0, e1);
            nn = f + (e1 > e0 ? 1 : 0);
            if (nn > 0) break;
        }
        s = uni(ss);
        F = uni(f);
        ex0 = uni(e0);
        ex1 = uni(e1);
        n = uni(nn);
        k = 0;
        p = 0;
        cstage &st = stage_at(a, s < a.nstages ? s : a.nstages - 1);
        G = uni(st.G);
        NI = uni(st.NI);
        units = uni(st.units);
        if (s >= a.nstages) {
            // past the last stage: the (unused) item 0 of the last stage's row 0
            P = 1;
            row0 = 0;
            rend = 1;
            return;
        }
        P = uni(st.P);
        set_tile(W, b);
    }
    // to the next slot: 0 same tile, 1 another tile of the stage, 2 another
    // stage (or past the last)
    __device__ __forceinline__ int next(const StreamArgs &a, uint32_t W, uint32_t b)
    {
        if (s >= a.nstages) return 0;
        p = uni(p + 1);
        if (p < P) return 0;
        p = 0;
        k = uni(k + 1);
        if (k < n) {
            set_tile(W, b);
            return 1;
        }
        enter(a, s + 1, W, b);
        return 2;
    }
};

// The issue side of a compute wave: every item load is a global load of
// piece i at rowaddr[i] + col + the segment's offset (+ the up matrix's
// offset for an up item), one code path for every tile and segment.  rowaddr
// (per tile) is the lane's row: its piece row clamped to the tile's last row
// (short tiles re-read that row), in the matrix the row falls in.  The
// column part is the piece's 16-byte column (colF), or in an 8-unit last
// segment the column taken modulo half the segment (item_piece's half
// mapping: the missing half re-reads the first), so no load leaves the row.
template <int FMT>
struct Issuer {
    uint32_t colF[Geo<FMT>::NL];
    uint64_t rowaddr[Geo<FMT>::NL];

    __device__ __forceinline__ void init(int lane)
    {
#pragma unroll
        for (int i = 0; i < Geo<FMT>::NL; i++) colF[i] = 16u * (uint32_t)item_piece(FMT, 64 * i + lane, false).col;
    }
    __device__ __forceinline__ void set_tile(cstage &st, const Walk &c, int lane)
    {
        const uint64_t rb = uni64((uint64_t)st.row_bytes);
        const uint64_t w0 = uni64(st.W[0]), w1 = uni64(st.W[1]), w2 = uni64(st.W[2]);
        const int re0 = uni(st.row_end[0]), re1 = uni(st.row_end[1]);
        const int row0 = c.row0, last = c.rend - 1;
#pragma unroll
        for (int i = 0; i < Geo<FMT>::NL; i++) {
            const int pr = item_piece(FMT, 64 * i + lane, false).row;
            const int v = min(row0 + pr, last);
            const int a1 = v >= re0, a2 = v >= re1;  // gate/up: row_end = {INT_MAX, INT_MAX}
            const int r = v - (a2 ? re1 : a1 ? re0 : 0);
            rowaddr[i] = (a2 ? w2 : a1 ? w1 : w0) + (uint64_t)r * rb;
        }
    }
};

// Item of the issue walk's slot into registers: NL 16-byte loads per lane,
// the kernel's only weight loads.  Every slot issues exactly NL loads from
// this one site, so the compiler's vmcnt wait for any slot is exact: a slot
// with no item for this wave re-reads the tile's last item, and a slot past
// the last stage re-reads item 0 of the last stage.  The data of such slots
// is never used.
template <int FMT>
__device__ __forceinline__ void stream_issue(Raw2<FMT> &buf, const Walk &c, const Issuer<FMT> &is, cstage &st, int cw)
{
    using GE = Geo<FMT>;
    const int item = uni(min(cw + kNCW * c.p, c.NI - 1));
    const bool up = item >= c.G;  // gate/up: items G..2G-1 are the up matrix's
    const int seg = item - (up ? c.G : 0);
    const bool half = 16 * seg + 16 > c.units;
    const uint64_t off = (uint64_t)seg * GE::SEGB + (up ? uni64(st.dup) : 0);
#pragma unroll
    for (int i = 0; i < GE::NL; i++) {
        const uint32_t col = half && is.colF[i] >= 8u * GE::PR ? is.colF[i] - 8u * GE::PR : is.colF[i];
        buf.v[i] = __builtin_nontemporal_load((gu32x4a *)(is.rowaddr[i] + (off + col)));
    }
}

// The item into the wave's LDS stage (row n at n * RS).
template <int FMT>
__device__ __forceinline__ void stream_stage_write(const Raw2<FMT> &b, uint8_t *stage, int lane)
{
    using GE = Geo<FMT>;
#pragma unroll
    for (int i = 0; i < GE::NL; i++) {
        const int pc = 64 * i + lane;
        if (GE::NP % 64 == 0 || pc < GE::NP) {
            uint8_t *p = stage + 16 * pc + (GE::RS - GE::SEGB) * (pc / GE::PR);
            *(u32x2a *)p = (u32x2a){b.v[i].x, b.v[i].y};
            *(u32x2a *)(p + 8) = (u32x2a){b.v[i].z, b.v[i].w};
        }
    }
}

// ---- unit dots with two activation scales per 32-weight unit ------------------------
//
// As item_unit of the MFMA GEMV, but the unit's weights 0-15 and 16-31 meet
// activation planes of separate scales: the two MFMAs stay apart and the
// epilogue is, per unit (d = block scale, S = 65536 Sh + 256 Sm + Sl per half,
// {dx0, dx1, s0, s1} the unit's staged scales and half sums):
//   Q4_0  d * (dx0*S0 + dx1*S1 - 8 (s0 + s1))
//   Q4_K  (d*sc) * (dx0*S0 + dx1*S1) - (dmin*m) * (s0 + s1)
template <int T, int FMT>
__device__ __forceinline__ void item_unit2(float &acc, const Chunk<FMT> &c, const uint8_t *ldsb, uint32_t abase,
                                           uint32_t sbase, int skip, bool tail, float dk, float mk, uint32_t sc,
                                           uint32_t mn)
{
    const v4i a0 = *(const v4i *)(ldsb + abase + 96 * T);
    const v4i a1 = *(const v4i *)(ldsb + abase + 96 * T + 16);
    const float4 xs = *(const float4 *)(ldsb + sbase + 16 * T);
    v4i lo, hi;
    uint32_t dbits;
    chunk_unit<T, FMT>(c, lo, hi, dbits);
    const v4i zero = {0, 0, 0, 0};
    const v4i s0 = mfma_i8(a0, lo, zero), s1 = mfma_i8(a1, hi, zero);
    // |Sh| <= 16*128*127, so 256*Sh + Sm is exact in int32
    const float S0 = fmaf(256.0f, (float)((s0[0] << 8) + s0[1]), (float)s0[2]);
    const float S1 = fmaf(256.0f, (float)((s1[0] << 8) + s1[1]), (float)s1[2]);
    const float dS = fmaf(xs.x, S0, xs.y * S1);
    const float sx = xs.z + xs.w;
    if constexpr (FMT == FMT_Q4_K) {
        float dsc = dk * (float)((sc >> (8 * T)) & 0xFFu);
        float dmn = mk * (float)((mn >> (8 * T)) & 0xFFu);
        if (tail && T < skip) dsc = dmn = 0.f;
        acc = fmaf(dsc, dS, fmaf(-dmn, sx, acc));
    } else {
        float d = half_bits_to_float(dbits);
        if (tail && T < skip) d = 0.f;
        acc = fmaf(d, fmaf(-8.0f, sx, dS), acc);
    }
}

template <int FMT>
__device__ __forceinline__ float item_dot2(const Chunk<FMT> &c, const uint8_t *ldsb, uint32_t abase, uint32_t sbase,
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
    item_unit2<0, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    item_unit2<1, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    item_unit2<2, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    item_unit2<3, FMT>(acc, c, ldsb, abase, sbase, skip, tail, dk, mk, sc, mn);
    return acc;
}

// ---- activations into planes ------------------------------------------------------------

// Sum / maximum of non-negative floats over the 4 lanes of an aligned quad
// and over the 16 lanes of a row (all lanes active); every lane gets the result.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float quad_sum(float v)
{
    v += dpp_f<0xB1>(v);
    return v + dpp_f<0x4E>(v);
}
__device__ __forceinline__ float quad_max_nonneg(float f)
{
    uint32_t v = __float_as_uint(f);
    v = max(v, dpp_u<0xB1>(v));
    return __uint_as_float(max(v, dpp_u<0x4E>(v)));
}
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror
    return v + dpp_f<0x140>(v);  // row_mirror
}
__device__ __forceinline__ float row16_max_nonneg(float f)
{
    uint32_t v = __float_as_uint(f);
    v = max(v, dpp_u<0xB1>(v));
    v = max(v, dpp_u<0x4E>(v));
    v = max(v, dpp_u<0x141>(v));
    return __uint_as_float(max(v, dpp_u<0x140>(v)));
}

// xi + 0x808080 for xi = rint(x * inv), |x * inv| < 2^22 (x_convert's rounding
// identity: the planes are the three low bytes with the top bit flipped).
__device__ __forceinline__ uint32_t biased_xi(float x, float inv)
{
    return __float_as_uint(__builtin_fmaf(x, inv, 12582912.0f)) - (0x4B400000u - 0x808080u);
}

// Chunk i (4 values: unit i >> 3, chunk c = i & 7) into the planes and the
// unit's scales.  The 4 chunks of a 16-value half sit in an aligned lane
// quad (the caller's i = tid + stride*k keeps quads aligned).
__device__ __forceinline__ void x_convert2(const float4 v, int i, int units, uint8_t *ldsb)
{
    const int u = i >> 3, c = i & 7;
    const float amax = quad_max_nonneg(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float sx = quad_sum((v.x + v.y) + (v.z + v.w));
    const float dx = amax * (1.0f / (float)kQmax);
    const float inv = amax > 0.f ? (float)kQmax * __builtin_amdgcn_rcpf(amax) : 0.f;
    const uint32_t w0 = biased_xi(v.x, inv), w1 = biased_xi(v.y, inv), w2 = biased_xi(v.z, inv),
                   w3 = biased_xi(v.w, inv);
    const uint32_t p01 = __builtin_amdgcn_perm(w1, w0, 0x05010400u);
    const uint32_t p23 = __builtin_amdgcn_perm(w3, w2, 0x05010400u);
    const uint32_t r01 = __builtin_amdgcn_perm(w1, w0, 0x0c0c0602u);
    const uint32_t r23 = __builtin_amdgcn_perm(w3, w2, 0x0c0c0602u);
    uint32_t *lq = (uint32_t *)(ldsb + 96 * u);
    lq[c] = __builtin_amdgcn_perm(r23, r01, 0x05040100u) ^ 0x80808080u;       // h plane
    lq[8 + c] = __builtin_amdgcn_perm(p23, p01, 0x07060302u) ^ 0x80808080u;   // m plane
    lq[16 + c] = __builtin_amdgcn_perm(p23, p01, 0x05040100u) ^ 0x80808080u;  // l plane
    if ((c & 3) == 0) {
        float *scl = (float *)(ldsb + 96 * units + 16 * u);
        scl[c >> 2] = dx;
        scl[2 + (c >> 2)] = sx;
    }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(1))) uint64_t gword;

// The input of a stage that no earlier stage of the plan wrote (plain fp32,
// units * 32 floats), by one wave: each global_load_lds_dwordx4 moves 64 lanes
// x 16 contiguous bytes into 1 KB of LDS.  The caller waits (vmcnt) before the
// workgroup barrier that publishes the buffer.
__device__ __forceinline__ void stream_fetch_plain(cstage &st, uint8_t *xbuf, int lane)
{
    const int units = uni(st.units), n = units / 8;  // 1 KB pieces (units is a multiple of 8)
    const float *x = (const float *)uni64(st.x);
    for (int j = 0; j < n; j++)
        __builtin_amdgcn_global_load_lds((gvoid *)(x + 256 * j + 4 * lane), (lds_void *)(xbuf + 1024 * j), 16, 0, 0);
}

// The stage's norm weight (plain fp32) after its input in LDS.
__device__ __forceinline__ void stream_fetch_norm(cstage &st, uint8_t *wbuf, int lane)
{
    const int units = uni(st.units), n = units / 8;
    const float *w = (const float *)uni64(st.nw);
    for (int j = 0; j < n; j++)
        __builtin_amdgcn_global_load_lds((gvoid *)(w + 256 * j + 4 * lane), (lds_void *)(wbuf + 1024 * j), 16, 0, 0);
}

// Exchange words of a stage input (the fp32 words, or the plane records:
// either way 8 bytes per input value) into LDS, 1 KB pieces of 128 words,
// device-coherent (sc1: never answered from a line this XCD's L2 held before
// another XCD's store).  The tags are checked while the words are put in
// place (stream_stage_in), which copies again the pieces that were not
// current.  One plain loop: the one issuing wave's scalar work per piece
// bounds the copy (a choice of source per piece made it 2.5x slower).
__device__ __forceinline__ const uint8_t *words_src(cstage &st)
{
    const uint64_t lp = uni64(st.lpx);
    return (const uint8_t *)(lp ? lp : uni64(st.llx));
}
__device__ __forceinline__ void stream_fetch_words(cstage &st, uint8_t *xbuf, int lane)
{
    const int units = uni(st.units), nch = units / 4;  // 128 words = 4 units per piece
    const uint8_t *src = words_src(st) + 16 * lane;
    for (int j = 0; j < nch; j++)
        __builtin_amdgcn_global_load_lds((gvoid *)(src + 1024 * j), (lds_void *)(xbuf + 1024 * j), 16, 0,
                                         kDeviceScope);
}

// A wait that reaches kStreamPolls gives up: it sets the library's flag
// (what holo_gemv_stream_status reports) and records the launch in the
// plan's give-up word (its tag base + 1).  Every later wait of the same
// launch sees that record and returns at once, on every workgroup, so a
// launch whose workgroups are not all resident costs one bounded wait, not
// one per stage.
struct StreamFlag {
    uint32_t *flag;  // the library's sticky flag
    uint32_t *rec;   // the plan's give-up word (header word 1, zeroed at creation)
};
__device__ __forceinline__ bool stream_gave_up(StreamFlag f, uint32_t base)
{
    return __hip_atomic_load(f.rec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == base + 1u;
}
__device__ __forceinline__ void stream_give_up(StreamFlag f, uint32_t base)
{
    __hip_atomic_store(f.flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(f.rec, base + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until every workgroup has stored its rows of the stage with tag
// `tag` (its done word holds that tag or a later one of this launch).  A done
// word is stored right after the workgroup's exchange words, without waiting
// for them to complete, so it only says that the words are on their way: the
// gather still checks every word's tag.  The wait keeps the polling to 4
// bytes per workgroup instead of the whole input.
__device__ __forceinline__ void stream_wait_done(const uint32_t *done, uint32_t tag, uint32_t base, StreamFlag flag,
                                                 int lane)
{
    const int G = (int)gridDim.x;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)done, (short)0, G * 4, kBufferWord3);
    for (uint32_t polls = 0;; polls++) {
        bool late = false;
        for (int j = 0; 256 * j < G; j++) {
            const u32x4 d = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, 1024 * j + 16 * lane, 0, kDeviceScope));
            const int i0 = 256 * j + 4 * lane;
#pragma unroll
            for (int e = 0; e < 4; e++) late |= i0 + e < G && (int32_t)(d[e] - tag) < 0;
        }
        if (__ballot(late) == 0) return;
        if (polls == kStreamPolls) {
            stream_give_up(flag, base);
            return;
        }
        if ((polls & 255u) == 0 && stream_gave_up(flag, base)) return;
        __builtin_amdgcn_s_sleep(2);
    }
}

// Two exchange words (value, tag ^ value) as a uint4: both current?
__device__ __forceinline__ bool words_ok(uint4 a, uint32_t tag) { return ((a.y ^ a.x) == tag) & ((a.w ^ a.z) == tag); }

// x value chunk i (4 values) of the staged input: plain fp32, or exchange
// words, which must all carry `tag` (else `bad`).
__device__ __forceinline__ float4 staged_x4(const uint8_t *xbuf, int i, bool tagged, uint32_t tag, bool &bad)
{
    if (tagged) {
        const uint4 a = *(const uint4 *)(xbuf + 32 * i), b = *(const uint4 *)(xbuf + 32 * i + 16);
        bad |= !(words_ok(a, tag) & words_ok(b, tag));
        return make_float4(__uint_as_float(a.x), __uint_as_float(a.z), __uint_as_float(b.x), __uint_as_float(b.z));
    }
    return *(const float4 *)(xbuf + 16 * i);
}

constexpr int kRedBase = 14;   // red[14]: this launch's tag base, from the control wave
constexpr int kRedQuit = 15;   // red[15]: the control wave gave the current input's wait up
constexpr int kRedMask = 16;   // red[16..31]: two stale-piece masks (1 KB pieces of the staged words)
constexpr int kMaskWords = 8;  // pieces up to 256: in_dim up to 32768
constexpr int kRedWords = kRedMask + 2 * kMaskWords;

__device__ __forceinline__ bool piece_set(const uint32_t *m, int j) { return (m[j >> 5] >> (j & 31)) & 1u; }
__device__ __forceinline__ void mark_piece(uint32_t *m, int j)
{
    __hip_atomic_fetch_or(m + (j >> 5), 1u << (j & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The staged input of stage st into the planes and scales, by all threads.
// A staged word whose tag is not `tag` marks its 1 KB piece in `stale`.
//   plane records (st.lpx): 4 lanes per record g (16 values: unit g/2, half
//     g&1), lane j of them takes words 4j..4j+3: for j < 3 the 4 dwords of
//     plane j (one 16-byte store), for j = 3 the half's dx, its sum and its
//     sum of squares (ss[g], for the output's norm scale).  With `only`, just
//     the pieces marked there (the others are in place already).
//   fp32 (plain or exchange words): converted as x_convert does, with
//     x * (1/sqrt(mean(x^2) + eps)) * w first when the stage has a norm
//     weight (cuda_rms_norm's formula, cuda_ops.cu:1479-1504), the 9 waves'
//     sums of squares meeting in red; always the whole input.
__device__ __forceinline__ void stream_convert_x(cstage &st, uint8_t *ldsb, const uint8_t *xbuf, float *red, float *ss,
                                                 uint32_t tag, const uint32_t *only, uint32_t *stale)
{
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int units = uni(st.units);
    if (uni64(st.lpx)) {
        const int nq = units * 8;
        for (int q = tid; q < nq; q += kStreamThreads) {
            if (only && !piece_set(only, q >> 5)) continue;
            const uint4 a = *(const uint4 *)(xbuf + 32 * q), c = *(const uint4 *)(xbuf + 32 * q + 16);
            if (!(words_ok(a, tag) & words_ok(c, tag))) mark_piece(stale, q >> 5);
            const int g = q >> 2, j = q & 3, u = g >> 1, hf = g & 1;
            if (j < 3) {
                *(uint4 *)(ldsb + 96 * u + 32 * j + 16 * hf) = make_uint4(a.x, a.z, c.x, c.z);
            } else {
                uint32_t *scl = (uint32_t *)(ldsb + 96 * units + 16 * u);
                scl[hf] = a.x;
                scl[2 + hf] = a.z;
                ((uint32_t *)ss)[g] = c.x;
            }
        }
        return;
    }
    // (the norm's pass reads the same words as the conversion, which marks them)
    const int chunks = units * 8;
    const bool norm = uni64(st.nw) != 0;
    const bool tagged = uni64(st.llx) != 0;
    float scale = 1.f;
    bool bad = false;
    if (norm) {
        float s2 = 0.f;
        for (int i = tid; i < chunks; i += kStreamThreads) {
            const float4 v = staged_x4(xbuf, i, tagged, tag, bad);
            s2 += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        s2 = wave_sum(s2);
        if (lane == 0) red[wave] = s2;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w <= kNCW; w++) tot += red[w];
        scale = 1.0f / sqrtf(tot / (float)(units * 32) + unif(st.eps));
    }
    const float4 *wv = (const float4 *)(xbuf + units * (tagged ? 256 : 128));
    for (int i = tid; i < chunks; i += kStreamThreads) {
        bool b1 = false;
        float4 v = staged_x4(xbuf, i, tagged, tag, b1);
        if (b1) mark_piece(stale, i >> 5);
        if (norm) {
            const float4 w4 = wv[i];
            v = make_float4(v.x * scale * w4.x, v.y * scale * w4.y, v.z * scale * w4.z, v.w * scale * w4.w);
        }
        x_convert2(v, i, units, ldsb);
    }
}

// Copies again the 1 KB pieces of the staged words marked in `m` (control
// wave).
__device__ __forceinline__ void stream_refetch(cstage &st, uint8_t *xbuf, const uint32_t *m, int lane)
{
    for (int w = 0; w < kMaskWords; w++) {
        uint32_t bits = (uint32_t)uni((int)m[w]);
        while (bits) {
            const int j = 32 * w + __builtin_ctz(bits);
            bits &= bits - 1u;
            __builtin_amdgcn_global_load_lds((gvoid *)(words_src(st) + 1024 * j + 16 * lane),
                                             (lds_void *)(xbuf + 1024 * j), 16, 0, kDeviceScope);
        }
    }
}

// After the input of stage `st` was staged (B): all waves place or convert it
// (C); while pieces with stale exchange words remain, the control wave copies
// those pieces again and all waves place them again (plane records: only
// those pieces; fp32: the whole input, whose norm and planes depend on every
// word).  Round r reads the marks of mask r&1 and sets those of the next; every
// wave reads the same mask after the same barrier, so all take the same rounds
// and the barrier counts agree.  After kStreamPolls rounds the wait gives up
// and sets the plan's flag.  The control wave cleared mask 0 before B.
__device__ __forceinline__ void stream_stage_in(cstage &st, uint8_t *ldsb, uint8_t *xbuf, float *red, float *ss,
                                                uint32_t base, StreamFlag flag, bool control, int lane)
{
    const uint32_t tag = base + (uint32_t)uni(st.xsrc) + 1u;
    uint32_t *mask = (uint32_t *)red + kRedMask;
    stream_convert_x(st, ldsb, xbuf, red, ss, tag, nullptr, mask);
    __syncthreads();  // C
    const bool records = uni64(st.lpx) != 0;
    if (uni64(st.llx) == 0 && !records) return;
    for (uint32_t round = 0;; round++) {
        const uint32_t *cur = mask + kMaskWords * (round & 1u);
        uint32_t *nxt = mask + kMaskWords * ((round + 1u) & 1u);
        uint32_t any = 0;
#pragma unroll
        for (int w = 0; w < kMaskWords; w++) any |= cur[w];
        if ((uint32_t)uni((int)any) == 0) break;
        __syncthreads();  // every wave has read the mask
        if (control) {
            if (lane < kMaskWords) nxt[lane] = 0u;
            const bool quit = round == kStreamPolls || stream_gave_up(flag, base);
            if (lane == 0) ((uint32_t *)red)[kRedQuit] = quit ? 1u : 0u;
            if (quit) {
                stream_give_up(flag, base);
            } else {
                __builtin_amdgcn_s_sleep(2);
                stream_refetch(st, xbuf, cur, lane);
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            }
        }
        __syncthreads();  // B again
        // quitting leaves the next mask clear, so every wave leaves the loop
        if (uni((int)((const uint32_t *)red)[kRedQuit]) == 0)
            stream_convert_x(st, ldsb, xbuf, red, ss, tag, records ? cur : nullptr, nxt);
        __syncthreads();  // C again
    }
}

// Row v of this workgroup's rows of a stage for lane `lane` in pass q: 64
// rows a pass, tile k = 4 q + lane / 16, row lane % 16 of it.
__device__ __forceinline__ bool own_row(const Tiles &t, int q, int lane, uint32_t W, uint32_t b, int &k, int &i,
                                        int &v)
{
    k = 4 * q + (lane >> 4);
    i = lane & 15;
    int row0, rend;
    t.rows(k, W, b, row0, rend);
    v = row0 + i;
    return k < t.n && v < rend;
}

constexpr int kStreamPasses = kStreamMaxTiles / 4;  // passes of 64 rows over at most 16 tiles

// An exchange word is (tag ^ v) << 32 | v, stored with one 64-bit agent-scope
// store, and it is current when its halves XOR to the tag (word_ok).  The
// copies that read words into LDS are 16-byte loads, not 64-bit atomic
// loads, so a read could in principle pair the halves of two stores.  Such a
// pair passes the check only when its low half equals the current store's
// value: a torn read is either caught or harmless.
__device__ __forceinline__ uint64_t exchange_word_u(uint32_t v, uint32_t tag)
{
    return ((uint64_t)(tag ^ v) << 32) | v;
}
__device__ __forceinline__ uint64_t exchange_word(float v, uint32_t tag)
{
    return exchange_word_u(__float_as_uint(v), tag);
}

// The residual rows r[v] of this workgroup's rows of stage s (plain stages
// with r), one per lane and pass: exchange words when an earlier stage wrote
// r (waited for like the input), else the caller's fp32 values.
__device__ __forceinline__ void stream_prefetch_rr(cstage &st, const Tiles &t, float (&rr)[kStreamPasses],
                                                   uint32_t base, StreamFlag flag, uint32_t W, uint32_t b, int lane)
{
#pragma unroll
    for (int q = 0; q < kStreamPasses; q++) rr[q] = 0.f;
    const uint64_t rp = uni64(st.r), llr = uni64(st.llr);
    if (!rp || uni(st.mode) != MODE_PLAIN) return;
    const uint32_t tag = base + (uint32_t)uni(st.rsrc) + 1u;
#pragma unroll
    for (int q = 0; q < kStreamPasses; q++) {
        int k, i, v;
        const bool mine = own_row(t, q, lane, W, b, k, i, v);
        if (!llr) {
            if (mine) rr[q] = ((gcfloat *)rp)[v];
            continue;
        }
        uint64_t w = 0;
        for (uint32_t polls = 0;; polls++) {
            if (mine) w = __hip_atomic_load((gword *)llr + v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__ballot(mine && ((uint32_t)(w >> 32) ^ (uint32_t)w) != tag) == 0) break;
            if (polls == kStreamPolls) {
                stream_give_up(flag, base);
                break;
            }
            if ((polls & 255u) == 0 && stream_gave_up(flag, base)) break;
            __builtin_amdgcn_s_sleep(2);
        }
        rr[q] = __uint_as_float((uint32_t)w);
    }
}


// What the control wave's epilogue of stage s reads from global memory, read
// while the stage still runs, one value per lane and pass:
//   pw  the norm weight of the designated reader of the row's output, for
//       the plane records (1 without one);
//   rr  the residual rows (stream_prefetch_rr).
// The wave waits for these loads here, so the epilogue issues no load: a
// load there would wait (vmcnt) for the epilogue's own stores as well.
__device__ __forceinline__ void stream_prefetch(cstage &st, const Tiles &t, float (&rr)[kStreamPasses],
                                                float (&pw)[kStreamPasses], uint32_t base, StreamFlag flag, uint32_t W,
                                                uint32_t b, int lane)
{
    stream_prefetch_rr(st, t, rr, base, flag, W, b, lane);
    const uint64_t p0 = uni64(st.llp[0]), p1 = uni64(st.llp[1]), p2 = uni64(st.llp[2]);
    const uint64_t n0 = uni64(st.pnw[0]), n1 = uni64(st.pnw[1]), n2 = uni64(st.pnw[2]);
    const bool gu = uni(st.mode) == MODE_GATEUP;
#pragma unroll
    for (int q = 0; q < kStreamPasses; q++) {
        pw[q] = 1.f;
        int k, i, v, m = 0, row;
        const bool mine = own_row(t, q, lane, W, b, k, i, v);
        row = v;
        if (mine && !gu) split_row(st, v, m, row);
        const uint64_t rec = m == 2 ? p2 : m == 1 ? p1 : p0, nw = m == 2 ? n2 : m == 1 ? n1 : n0;
        if (mine && rec && nw) pw[q] = ((gcfloat *)nw)[row];
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
}

// The plane record of the 16 outputs of lanes 16t..16t+15 (one tile, one
// scale group of the designated reader's input): each lane holds its value o
// (its row's output) and nw, the reader's norm weight of that row (1 without
// a norm): the planes are of o * nw, and word 14 is the group's sum of o^2, from which the reader
// computes its norm scale.  Lane L stores word L % 16 of group L / 16.
__device__ __forceinline__ void stream_plane_record(float o, float nw, bool valid, uint64_t rec, uint32_t tag,
                                                    uint32_t *pack, int lane)
{
    const float xw = o * nw;
    const float amax = row16_max_nonneg(valid ? fabsf(xw) : 0.f);
    const float sum = row16_sum(valid ? xw : 0.f);
    const float sq = row16_sum(valid ? o * o : 0.f);
    const float dx = amax * (1.0f / (float)kQmax);
    const float inv = amax > 0.f ? (float)kQmax * __builtin_amdgcn_rcpf(amax) : 0.f;
    pack[lane] = biased_xi(valid ? xw : 0.f, inv);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's pack stores landed (one wave: in order)
    const int w = lane & 15, base = lane & ~15;
    uint32_t data = 0u;
    if (w < 12) {
        // plane p (h, m, l = bytes 2, 1, 0 of the biased values), values 4j..4j+3
        const int p = w >> 2, j = w & 3, byte = 2 - p;
        const uint4 d = *(const uint4 *)(pack + base + 4 * j);
        const uint32_t sel = (uint32_t)byte | ((uint32_t)(byte + 4) << 8) | 0x0c0c0000u;
        const uint32_t lo = __builtin_amdgcn_perm(d.y, d.x, sel), hi = __builtin_amdgcn_perm(d.w, d.z, sel);
        data = (lo | (hi << 16)) ^ 0x80808080u;
    } else if (w == 12) {
        data = __float_as_uint(dx);
    } else if (w == 13) {
        data = __float_as_uint(sum);
    } else if (w == 14) {
        data = __float_as_uint(sq);
    }
    if (valid)
        __hip_atomic_store((gword *)rec + w, exchange_word_u(data, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The control wave's stores of stage s: each of the workgroup's rows (one per
// lane and pass), the 8 compute waves' partials summed in wave order, times
// the norm scale cn of a stage whose input came as plane records; the plain
// fp32 output, its exchange word and, for an output with a designated
// reader, the plane records.  The plain store is made only by the last stage
// of the plan that writes the row: plain stores are cached in the storing
// XCD's L2 until written back, so two workgroups on different XCDs storing
// one row in two stages of a launch would race at write-back.  (Exchange
// words and records are agent-scope stores, written through; each row has
// one writer per stage.)
__device__ __forceinline__ void stream_epilogue(cstage &st, const Tiles &t, const float *tpart,
                                                const float (&rr)[kStreamPasses], const float (&pw)[kStreamPasses],
                                                float cn, uint32_t tag, uint32_t W, uint32_t b, uint32_t *pack,
                                                int lane)
{
    const bool gu = uni(st.mode) == MODE_GATEUP;
    const uint64_t y0 = uni64(st.y[0]), y1 = uni64(st.y[1]), y2 = uni64(st.y[2]);
    const uint64_t l0 = uni64(st.lly[0]), l1 = uni64(st.lly[1]), l2 = uni64(st.lly[2]);
    const uint64_t p0 = uni64(st.llp[0]), p1 = uni64(st.llp[1]), p2 = uni64(st.llp[2]);
    const bool res = uni64(st.r) != 0;
    const int ys0 = uni(st.ystart[0]), ys1 = uni(st.ystart[1]), ys2 = uni(st.ystart[2]);
#pragma unroll
    for (int q = 0; q < kStreamPasses; q++) {
        if (4 * q >= t.n) break;
        int k, i, v;
        const bool mine = own_row(t, q, lane, W, b, k, i, v);
        const float *pt = tpart + (k < kStreamMaxTiles ? k : 0) * (kNCW * 32);
        float o = 0.f;
        int m = 0, row = v;
        if (mine) {
            float s0 = 0.f;
#pragma unroll
            for (int w = 0; w < kNCW; w++) s0 += pt[w * 32 + i];
            s0 *= cn;
            if (gu) {
                float s1 = 0.f;
#pragma unroll
                for (int w = 0; w < kNCW; w++) s1 += pt[w * 32 + 16 + i];
                o = silu(s0) * (s1 * cn);
            } else {
                split_row(st, v, m, row);
                o = res ? rr[q] + s0 : s0;
            }
            if (row >= (m == 2 ? ys2 : m == 1 ? ys1 : ys0)) ((gfloat *)(m == 2 ? y2 : m == 1 ? y1 : y0))[row] = o;
            __hip_atomic_store((gword *)(m == 2 ? l2 : m == 1 ? l1 : l0) + row, exchange_word(o, tag),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // plane records: a tile's 16 rows are one group of one output (the
        // host designates outputs only in stages whose matrices' rows are all
        // multiples of 16, where every tile is 16 rows of one matrix)
        const uint64_t rec0 = mine ? (m == 2 ? p2 : m == 1 ? p1 : p0) : 0;
        if (__ballot(rec0 != 0) != 0) {
            const int g = (row - i) >> 4;  // the group: the tile's first row / 16
            stream_plane_record(o, pw[q], rec0 != 0, rec0 + 8ull * kRecWords * (uint64_t)g, tag, pack, lane);
        }
    }
}

__device__ __forceinline__ void stream_mark_done(uint32_t *done, uint32_t tag, uint32_t b, int lane)
{
    if (lane == 0) __hip_atomic_store(done + b, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The norm scale of a stage whose input came as plane records with a norm:
// 1/sqrt(mean(x^2) + eps) from the records' sums of squares, summed in a fixed
// order (lane l: groups l, l + 64, ..., then the wave reduction).
__device__ __forceinline__ float stream_norm_scale(cstage &st, const float *ss, int lane)
{
    if (!uni64(st.lpx) || !uni64(st.nw)) return 1.f;
    const int units = uni(st.units), ng = 2 * units;
    float s = 0.f;
    for (int g = lane; g < ng; g += 64) s += ss[g];
    s = wave_sum(s);
    return 1.0f / sqrtf(s / (float)(units * 32) + unif(st.eps));
}

template <int FMT, int D>
__global__ __launch_bounds__(kStreamThreads) void gemv_stream_kernel(StreamArgs a)
{
    using GE = Geo<FMT>;
    extern __shared__ uint4 lds_[];
    uint8_t *ldsb = (uint8_t *)lds_;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t W = gridDim.x, b = blockIdx.x;
    float *tpart = (float *)(ldsb + a.tpart_off);
    float *red = (float *)(ldsb + a.red_off);
    float *ss = (float *)(ldsb + a.ss_off);
    const int nst = a.nstages;

    uint8_t *xbuf = ldsb + a.xbuf_off;

    if (tid < kZeroBytes / 16) ((uint4 *)(ldsb + a.zero_off))[tid] = make_uint4(0, 0, 0, 0);

    if (wave < kNCW) {
        // ---- compute wave ----
        const int cw = wave;
        const int n = lane & 15, g = lane >> 4;
        const bool plane_lane = (n >> 2) == g && (n & 3) < 3;
        const uint32_t plane_off = (uint32_t)(n & 3) * 32u;
        uint8_t *stage = ldsb + a.stage_off + cw * GE::STAGE;
        Walk ci, cp;  // the issue walk runs D slots ahead of the process walk
        ci.enter(a, 0, W, b);
        cp = ci;
        Issuer<FMT> is;
        is.init(lane);
        {
            cstage &st = stage_at(a, ci.s < nst ? ci.s : nst - 1);
            is.set_tile(st, ci, lane);
        }
        // the issue walk to its next slot, with the issuer's stage and tile
        auto advance = [&]() {
            const int ev = ci.next(a, W, b);
            if (ev) {
                cstage &st = stage_at(a, ci.s < nst ? ci.s : nst - 1);
                is.set_tile(st, ci, lane);
            }
        };
        Raw2<FMT> ring[D];
#pragma unroll
        for (int d = 0; d < D; d++) {
            stream_issue<FMT>(ring[d], ci, is, stage_at(a, ci.s < nst ? ci.s : nst - 1), cw);
            advance();
        }
        __syncthreads();  // B of stage 0: x in LDS
        const uint32_t base = (uint32_t)uni((int)((uint32_t *)red)[kRedBase]);
        const StreamFlag fl{a.flag, a.seq + 1};
        stream_convert_x(stage_at(a, 0), ldsb, xbuf, red, ss, 0u, nullptr, (uint32_t *)red + kRedMask);
        __syncthreads();  // C of stage 0
        int s = 0;        // the stage whose boundary comes next
        float acc0 = 0.f, acc1 = 0.f;  // the tile's gate (or plain) and up partials
        // The loop has one exit, at its latch, and a trip count known up front
        // (the wave's slots, padded to a multiple of D with slots past the last
        // stage).  An exit inside the unrolled body would be merged into the
        // latch by the control-flow structurizer, and the compiler's
        // vector-memory wait analysis would then wait for every load in flight
        // (vmcnt(0)) at the loop head: the ring would drain once per D slots.
        // With one exit, the wait before slot d's stage write is exactly its own
        // loads (vmcnt((D-1)*NL + NL-1-i) for piece i).
        const int iters = uni(((const __attribute__((address_space(4))) int *)(uintptr_t)a.slots)[b]) / D;
        for (int it = 0; it < iters; it++) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                // the boundaries of every stage before this slot's (cp.s is nst
                // once this wave's slots are all done)
                while (s < cp.s) {
                    __syncthreads();  // A
                    __syncthreads();  // B
                    if (s + 1 < nst) stream_stage_in(stage_at(a, s + 1), ldsb, xbuf, red, ss, base, fl, false, lane);
                    s++;
                }
                // a slot past the last stage writes its (unused) item too, so
                // every slot's wait counts the same loads
                stream_stage_write<FMT>(ring[d], stage, lane);
                stream_issue<FMT>(ring[d], ci, is, stage_at(a, ci.s < nst ? ci.s : nst - 1), cw);
                advance();
                // the slot's dots against the staged x of stage s
                const int item = cw + kNCW * cp.p;
                if (cp.s < nst && item < cp.NI) {
                    const int units = cp.units;
                    const bool up = item >= cp.G;
                    const int j = item - (up ? cp.G : 0);
                    Chunk<FMT> c;
                    read_chunk<FMT>(c, stage, n, g);
                    const int cs0 = 16 * j + 4 * g;
                    const bool valid = cs0 < units;  // false only in an 8-unit last segment
                    const int cs = valid ? cs0 : units - 4;
                    const uint32_t abase = plane_lane ? (uint32_t)cs * 96u + plane_off : a.zero_off;
                    const float r = item_dot2<FMT>(c, ldsb, abase, (uint32_t)units * 96u + (uint32_t)cs * 16u,
                                                   (uint32_t)cs, valid ? 0 : 4, j == cp.G - 1);
                    if (up) acc1 += r;
                    else acc0 += r;
                }
                if (cp.s < nst && cp.p == cp.P - 1) {
                    float r0 = acc0, r1 = acc1;
                    r0 += __shfl_xor(r0, 16);
                    r0 += __shfl_xor(r0, 32);
                    r1 += __shfl_xor(r1, 16);
                    r1 += __shfl_xor(r1, 32);
                    acc0 = acc1 = 0.f;
                    float *pt = tpart + (cp.k * kNCW + cw) * 32;
                    if (lane < 16) pt[lane] = r0;
                    else if (lane < 32) pt[lane] = r1;  // lanes 16-31 hold the same sums
                }
                cp.next(a, W, b);
            }
        }
        // the boundaries after this wave's last slot
        while (s < nst) {
            __syncthreads();  // A
            __syncthreads();  // B
            if (s + 1 < nst) stream_stage_in(stage_at(a, s + 1), ldsb, xbuf, red, ss, base, fl, false, lane);
            s++;
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the last (dummy) item loads have returned
    } else {
        // ---- control wave ----
        uint32_t *pack = (uint32_t *)(ldsb + a.pack_off);
        const uint32_t seq0 = __hip_atomic_load(a.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t base = uni((int)(seq0 * (uint32_t)(nst + 1)));
        const StreamFlag fl{a.flag, a.seq + 1};
        {
            cstage &st0 = stage_at(a, 0);
            stream_fetch_plain(st0, xbuf, lane);
            if (uni64(st0.nw)) stream_fetch_norm(st0, xbuf + uni(st0.units) * 128, lane);
        }
        if (lane == 0) ((uint32_t *)red)[kRedBase] = base;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the LDS-direct loads have landed
        __syncthreads();                     // B of stage 0
        stream_convert_x(stage_at(a, 0), ldsb, xbuf, red, ss, 0u, nullptr, (uint32_t *)red + kRedMask);
        __syncthreads();  // C of stage 0
        float cn = 1.f;   // norm scale of the current stage's output
        for (int s = 0; s < nst; s++) {
            cstage &st = stage_at(a, s);
            Tiles t;
            t.init(st, W, b);
            // the output scale and the residual rows, while the stage runs
            if (s > 0) cn = stream_norm_scale(st, ss, lane);
            float rr[kStreamPasses], pw[kStreamPasses];
            stream_prefetch(st, t, rr, pw, base, fl, W, b, lane);
            __syncthreads();  // A: every partial of stage s is in LDS
            stream_epilogue(st, t, tpart, rr, pw, cn, base + (uint32_t)s + 1u, W, b, pack, lane);
            stream_mark_done(a.seq + 128, base + (uint32_t)s + 1u, b, lane);
            if (s + 1 < nst) {
                cstage &st1 = stage_at(a, s + 1);
                const int units1 = uni(st1.units);
                const bool words = uni64(st1.llx) != 0 || uni64(st1.lpx) != 0;
                // the partial reads above are done before any copy lands in
                // their space (xbuf aliases the item stages and partials)
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                if (uni64(st1.nw) && !uni64(st1.lpx)) stream_fetch_norm(st1, xbuf + units1 * (words ? 256 : 128), lane);
                if (words) {
                    if (lane < kMaskWords) ((uint32_t *)red)[kRedMask + lane] = 0u;
                    stream_wait_done(a.seq + 128, base + (uint32_t)uni(st1.xsrc) + 1u, base, fl, lane);
                    stream_fetch_words(st1, xbuf, lane);
                } else {
                    stream_fetch_plain(st1, xbuf, lane);
                }
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            }
            __syncthreads();  // B
            if (s + 1 < nst) stream_stage_in(stage_at(a, s + 1), ldsb, xbuf, red, ss, base, fl, true, lane);
        }
        // the last workgroup to finish advances the launch count (every
        // workgroup read it at its start, before counting itself done)
        if (lane == 0) {
            const uint32_t done = __hip_atomic_fetch_add(a.seq + 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (done == W - 1) {
                __hip_atomic_store(a.seq + 64, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(a.seq, seq0 + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

// ---- host ----------------------------------------------------------------------------

uint32_t *g_stream_flag = nullptr;  // set by an exchange wait that gave up

struct StreamPlan {
    StreamStage *dev = nullptr;  // the stage table
    int *slots = nullptr;        // item slots per compute wave of each workgroup
    uint8_t *words = nullptr;    // launch counter line, done counter line, exchange words
    int nstages = 0;
    int fmt = 0;
    size_t lds = 0;
    StreamArgs args{};
};

// LDS: [x planes + unit scales][zero region][reductions][plane bytes][sums of
// squares][region], where the region holds the compute waves' item stages and
// the tile partials during a stage, and the staged input (fp32, exchange
// words or plane records, then the norm weight) during a boundary.
size_t stream_lds(int fmt, int max_units, int max_xbuf, StreamArgs &a)
{
    const size_t x_lds = ((size_t)max_units * kUnitLds + 15) & ~(size_t)15;
    a.zero_off = zero_region_off((uint32_t)x_lds);
    a.red_off = a.zero_off + kZeroBytes;
    a.pack_off = a.red_off + kRedWords * 4;
    a.ss_off = a.pack_off + 64 * 4;
    a.stage_off = (a.ss_off + 2 * 4 * (uint32_t)max_units + 15) & ~15u;
    const int stage = fmt == FMT_Q4_0 ? Geo<FMT_Q4_0>::STAGE : Geo<FMT_Q4_K>::STAGE;
    a.tpart_off = (a.stage_off + kNCW * stage + 15) & ~15u;
    a.xbuf_off = a.stage_off;
    const size_t during = a.tpart_off + (size_t)kStreamMaxTiles * kNCW * 32 * 4;
    const size_t boundary = a.xbuf_off + (size_t)max_xbuf;
    return during > boundary ? during : boundary;
}

template <int FMT, int D>
bool stream_launch_t(StreamPlan &p)
{
    auto kern = gemv_stream_kernel<FMT, D>;
    static bool attr = false;
    if (!attr) {
        HOLO_CHECK(hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        attr = true;
    }
    // every workgroup must be resident at once (grid barrier): one per CU
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void *)kern, kStreamThreads, p.lds) != hipSuccess)
        per_cu = 0;
    if (per_cu < 1) return false;
    hipEvent_t e0, e1;
    if (take_launch_events(&e0, &e1))
        hipExtLaunchKernelGGL(kern, dim3(num_cus()), dim3(kStreamThreads), p.lds, stream(), e0, e1, 0, p.args);
    else
        hipLaunchKernelGGL(kern, dim3(num_cus()), dim3(kStreamThreads), p.lds, stream(), p.args);
    HOLO_LAUNCH_CHECK();
    return true;
}

constexpr int kStreamD = 3;  // items in flight per compute wave (4 spills at 168 VGPRs)

template <int FMT>
bool stream_launch_f(StreamPlan &p)
{
    return stream_launch_t<FMT, kStreamD>(p);
}

}  // namespace

bool gemv_stream_init()
{
    if (g_stream_flag) return true;
    if (hipMalloc((void **)&g_stream_flag, 256) != hipSuccess) {
        g_stream_flag = nullptr;
        return false;
    }
    return hipMemset(g_stream_flag, 0, 256) == hipSuccess && hipDeviceSynchronize() == hipSuccess;
}

void gemv_stream_release()
{
    if (g_stream_flag) hipFree(g_stream_flag);
    g_stream_flag = nullptr;
}

}  // namespace holo

using namespace holo;

extern "C" {

void *holo_gemv_stream_create(const holo_stream_stage_t *stages, int nstages, int type)
{
    const int fmt = type == HOLO_TYPE_Q4_0 ? FMT_Q4_0 : type == HOLO_TYPE_Q4_K ? FMT_Q4_K : -1;
    if (!stages || nstages < 1 || fmt < 0 || !g_stream_flag) {
        HOLO_REJECT("holo_gemv_stream_create: no stages, a type other than Q4_0/Q4_K, or cuda_init not called");
        return nullptr;
    }
    if (stream_capturing()) {
        HOLO_REJECT("holo_gemv_stream_create: allocates; create the plan outside graph capture");
        return nullptr;
    }
    const int grid = num_cus();
    StreamStage *host = new StreamStage[nstages];
    int max_units = 0, max_xbuf = 0;
    bool rows16 = true;  // per stage below: every matrix's rows a multiple of 16
    std::vector<char> aligned16(nstages, 0);
    for (int s = 0; s < nstages; s++) {
        const holo_stream_stage_t &in = stages[s];
        StreamStage &o = host[s];
        o = StreamStage{};
        const bool gu = in.gate_up != 0;
        const int nmat = gu ? 2 : in.nmat;
        bool ok = nmat >= 1 && nmat <= 3 && in.x && !((uintptr_t)in.x & 15u) && in.in_dim > 0;
        o.units = units_per_row(fmt, in.in_dim);
        o.row_bytes = row_bytes_of(fmt, in.in_dim);
        ok = ok && o.units >= 8 && (o.units & 7) == 0 && o.units * 32 == in.in_dim && o.units <= 576;
        ok = ok && (!in.norm_w || !((uintptr_t)in.norm_w & 15u));
        ok = ok && (!in.r || (!gu && nmat == 1));
        int total = 0;
        rows16 = true;
        for (int m = 0; m < 3; m++) {
            if (m < nmat) {
                const int rows = in.rows[gu ? 0 : m];
                float *y = in.y[gu ? 0 : m];
                ok = ok && in.W[m] && !((uintptr_t)in.W[m] & 15u) && rows > 0 && y;
                o.W[m] = (uint64_t)in.W[m];
                o.y[m] = (uint64_t)y;
                total += rows;
                o.row_end[m] = gu ? INT_MAX : total;  // gate/up rows all index W[0] (up: + dup)
                rows16 = rows16 && rows % 16 == 0;
            } else {
                o.W[m] = (uint64_t)in.W[0];
                o.y[m] = (uint64_t)in.y[0];
                o.row_end[m] = INT_MAX;
            }
        }
        if (!ok) {
            delete[] host;
            HOLO_REJECT("holo_gemv_stream_create: a stage outside the supported set (16-byte aligned matrices and "
                        "vectors, in_dim a multiple of 256 up to 18432, 1-3 matrices, residual on one plain matrix)");
            return nullptr;
        }
        o.mode = gu ? MODE_GATEUP : MODE_PLAIN;
        o.x = (uint64_t)in.x;
        o.nw = (uint64_t)in.norm_w;
        o.eps = in.eps;
        o.r = (uint64_t)in.r;
        o.G = (o.units + 15) / 16;
        o.NI = gu ? 2 * o.G : o.G;
        o.P = (o.NI + kNCW - 1) / kNCW;
        o.dup = gu ? (uint64_t)in.W[1] - (uint64_t)in.W[0] : 0;
        o.total_rows = gu ? in.rows[0] : total;
        o.full_tiles = o.total_rows / (grid * 16);
        o.rem_start = o.full_tiles * grid * 16;
        aligned16[s] = rows16;
        if (o.full_tiles + 1 > kStreamMaxTiles) {
            delete[] host;
            HOLO_REJECT("holo_gemv_stream_create: a stage with more rows than 16 tiles per CU");
            return nullptr;
        }
        max_units = o.units > max_units ? o.units : max_units;
    }
    // Exchange buffers: a word per row of a stage output (stage s, output m),
    // and for an output with a designated reader a record buffer of the same
    // size.  A stage's x or r that an earlier stage wrote is read from the
    // buffers of its last writer (xsrc / rsrc, output xm / rm) and must not
    // extend past what that writer stored; an input that overlaps an earlier
    // output in any other way, an output that overlaps its own stage's x, two
    // outputs of one stage in one vector, or outputs that partly overlap are
    // rejected (the caller's vectors are keyed by address for these rules).
    struct OutVec {
        uint64_t ptr;
        int rows;        // the most rows any stage wrote there (for the overlap rules)
        int last, lastm; // the last writer so far and its output index
    };
    std::vector<OutVec> outs;
    std::vector<int> xo(nstages, -1), ro(nstages, -1), yo(3 * (size_t)nstages, -1);
    std::vector<int> xm(nstages, 0), rm(nstages, 0);
    auto out_rows = [&](int s, int m) { return stages[s].rows[stages[s].gate_up ? 0 : m]; };
    auto overlap = [](uint64_t a, uint64_t an, uint64_t b, uint64_t bn) { return a < b + bn && b < a + an; };
    auto source = [&](uint64_t ptr, int n, int &idx, int &src, int &srcm) {
        idx = -1;
        src = -1;
        for (size_t i = 0; i < outs.size(); i++) {
            if (outs[i].ptr == ptr) {
                if (out_rows(outs[i].last, outs[i].lastm) < n) return false;
                idx = (int)i;
                src = outs[i].last;
                srcm = outs[i].lastm;
            } else if (overlap(ptr, 4ull * n, outs[i].ptr, 4ull * outs[i].rows)) {
                return false;
            }
        }
        return true;
    };
    // Caller memory that a stage reads with plain loads (an x or r no earlier
    // stage wrote, and every norm weight).  A workgroup reads it at or before
    // the reading stage t, so a later stage s may store over it only once
    // every workgroup is past t: some stage u in (t, s] copies a whole input
    // whose producer is t or later (the copy waits for every workgroup's done
    // word of that producer).  Otherwise a fast workgroup's plain stores could
    // reach memory that a slow one still has to read.  The one exception is a
    // stage's residual at exactly its own output (y += W x in place): each row
    // is read and stored by the one workgroup that owns it.
    struct CallerSpan {
        uint64_t ptr, bytes;
        int reader;
        bool residual;
    };
    std::vector<CallerSpan> spans;
    auto ordered_after = [&](int t, int s) {
        for (int u = t + 1; u <= s; u++)
            if (xo[u] >= 0 && host[u].xsrc >= t) return true;
        return false;
    };
    bool xok = true;
    for (int s = 0; s < nstages && xok; s++) {
        const holo_stream_stage_t &in = stages[s];
        StreamStage &o = host[s];
        xok = source(o.x, in.in_dim, xo[s], o.xsrc, xm[s]);
        if (xok && in.r) xok = source(o.r, in.rows[0], ro[s], o.rsrc, rm[s]);
        // a norm weight is plain-loaded: never from memory a stage stores to
        for (size_t i = 0; i < outs.size() && xok && o.nw; i++)
            if (overlap(o.nw, 4ull * in.in_dim, outs[i].ptr, 4ull * outs[i].rows)) xok = false;
        if (!xok) break;
        if (xo[s] < 0) spans.push_back(CallerSpan{o.x, 4ull * in.in_dim, s, false});
        if (in.r && ro[s] < 0) spans.push_back(CallerSpan{o.r, 4ull * in.rows[0], s, true});
        if (o.nw) spans.push_back(CallerSpan{o.nw, 4ull * in.in_dim, s, false});
        const int nout = in.gate_up ? 1 : in.nmat;
        for (int m = 0; m < nout && xok; m++) {
            const uint64_t y = (uint64_t)in.y[m];
            const int rows = in.rows[m];
            if (overlap(y, 4ull * rows, o.x, 4ull * in.in_dim)) xok = false;
            for (size_t i = 0; i < spans.size() && xok; i++) {
                const CallerSpan &c = spans[i];
                if (!overlap(y, 4ull * rows, c.ptr, c.bytes)) continue;
                if (c.reader == s) xok = c.residual && c.ptr == y && c.bytes == 4ull * rows;
                else xok = ordered_after(c.reader, s);
            }
            int hit = -1;
            for (size_t i = 0; i < outs.size() && xok; i++) {
                if (outs[i].ptr == y) hit = (int)i;
                else if (overlap(y, 4ull * rows, outs[i].ptr, 4ull * outs[i].rows)) xok = false;
            }
            if (!xok) break;
            if (hit < 0) {
                outs.push_back(OutVec{y, rows, s, m});
                hit = (int)outs.size() - 1;
            } else if (outs[hit].last == s) {
                xok = false;
                break;
            } else {
                outs[hit].rows = rows > outs[hit].rows ? rows : outs[hit].rows;
                outs[hit].last = s;
                outs[hit].lastm = m;
            }
            yo[3 * (size_t)s + m] = hit;
        }
    }
    if (!xok) {
        delete[] host;
        HOLO_REJECT("holo_gemv_stream_create: a stage input that overlaps an earlier output other than exactly or "
                    "reads past what its last writer stored, a norm weight in stage output memory, an output "
                    "overlapping its own input or another output, or an output over caller memory that a stage "
                    "not yet ordered before it reads");
        return nullptr;
    }
    // the plain stores of a row go to its last writer in the plan
    for (int s = 0; s < nstages; s++) {
        const int nout = stages[s].gate_up ? 1 : stages[s].nmat;
        for (int m = 0; m < 3; m++) host[s].ystart[m] = 0;
        for (int m = 0; m < nout; m++) {
            int later = 0;
            for (int s2 = s + 1; s2 < nstages; s2++) {
                const int n2 = stages[s2].gate_up ? 1 : stages[s2].nmat;
                for (int m2 = 0; m2 < n2; m2++)
                    if (yo[3 * (size_t)s2 + m2] == yo[3 * (size_t)s + m] && stages[s2].rows[m2] > later)
                        later = stages[s2].rows[m2];
            }
            host[s].ystart[m] = later;
        }
    }
    // Plane records: each written output (stage s, output m) is designated to
    // the first later stage that reads exactly that output as its x (its
    // in_dim = the output's rows) when the 16-row tiles of stage s each fall in
    // one matrix (every matrix's rows a multiple of 16).
    std::vector<int> lp(nstages, -1), rd(3 * (size_t)nstages, -1);
    for (int t = 0; t < nstages; t++) {
        const int s = host[t].xsrc;
        if (xo[t] < 0 || s < 0 || !aligned16[s]) continue;
        const int nout = stages[s].gate_up ? 1 : stages[s].nmat;
        for (int m = 0; m < nout; m++) {
            if (yo[3 * (size_t)s + m] != xo[t] || rd[3 * (size_t)s + m] >= 0) continue;
            if (stages[s].rows[m] != stages[t].in_dim) continue;
            rd[3 * (size_t)s + m] = t;
            lp[t] = xo[t];
        }
    }
    // Which stage outputs share buffers.  A later writer of a vector reuses
    // the previous writer's buffers only when every stage that reads the
    // previous version has finished reading it, on every workgroup, before any
    // workgroup can store the new one: some stage u after the reader t, up to
    // the new writer, waits for the whole output of a stage p >= t (its x is
    // an earlier output: its copy checks every word's tag, so every workgroup
    // has stored p's outputs, after having read t's inputs).  A residual read
    // by the new writer itself is of its own rows and needs no order.  Else
    // the new writer gets buffers of its own: a fast workgroup's store would
    // overwrite words that a slow one still has to read.  (The decode step's
    // chain shares throughout.)
    std::vector<int> grp(3 * (size_t)nstages, -1);
    std::vector<int> grows;  // rows of each buffer group
    std::vector<char> grec;  // the group holds plane records
    {
        std::vector<int> last_k(outs.size(), -1);  // key 3 s + m of the vector's last writer so far
        for (int s = 0; s < nstages; s++) {
            const int nout = stages[s].gate_up ? 1 : stages[s].nmat;
            for (int m = 0; m < nout; m++) {
                const size_t k = 3 * (size_t)s + m;
                const int i = yo[k], pk = last_k[i];
                bool share = pk >= 0;
                if (share) {
                    const int ps = pk / 3, pm = pk % 3;
                    for (int t = ps + 1; t <= s && share; t++) {
                        const bool rx = xo[t] == i && host[t].xsrc == ps && xm[t] == pm;
                        const bool rr = ro[t] == i && host[t].rsrc == ps && rm[t] == pm;
                        if (!rx && !(rr && t < s)) continue;
                        bool ordered = false;
                        for (int u = t + 1; u <= s && !ordered; u++) ordered = xo[u] >= 0 && host[u].xsrc >= t;
                        share = ordered;
                    }
                }
                if (share) {
                    grp[k] = grp[(size_t)pk];
                    grows[grp[k]] = out_rows(s, m) > grows[grp[k]] ? out_rows(s, m) : grows[grp[k]];
                } else {
                    grp[k] = (int)grows.size();
                    grows.push_back(out_rows(s, m));
                    grec.push_back(0);
                }
                if (rd[k] >= 0) grec[grp[k]] = 1;
                last_k[i] = (int)k;
            }
        }
    }
    std::vector<size_t> gw(grows.size()), gr(grows.size());
    size_t nwords = 0, nrec = 0;
    for (size_t g = 0; g < grows.size(); g++) {
        gw[g] = nwords;
        nwords += (size_t)grows[g];
        gr[g] = nrec;
        if (grec[g]) nrec += (size_t)grows[g];
    }
    auto woff = [&](size_t k) { return gw[grp[k]]; };
    auto roff = [&](size_t k) { return gr[grp[k]]; };
    // launch counter line, done counter line, one done word per workgroup
    const size_t kWordsHeader = (512 + 4 * (size_t)grid + 255) & ~(size_t)255;
    const size_t words_bytes = kWordsHeader + 8 * (nwords + nrec);
    uint8_t *words = nullptr;
    if (hipMalloc((void **)&words, words_bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete[] host;
        HOLO_REJECT("holo_gemv_stream_create: device memory for the exchange buffers");
        return nullptr;
    }
    HOLO_CHECK(hipMemset(words, 0, words_bytes));
    const uint64_t wbase = (uint64_t)(uintptr_t)words + kWordsHeader;
    const uint64_t rbase = wbase + 8 * nwords;  // the record buffers follow the words
    for (int s = 0; s < nstages; s++) {
        const holo_stream_stage_t &in = stages[s];
        StreamStage &o = host[s];
        const int nout = in.gate_up ? 1 : in.nmat;
        for (int m = 0; m < 3; m++) {
            const size_t k = 3 * (size_t)s + (m < nout ? m : 0);
            const int t = rd[k];
            o.lly[m] = wbase + 8 * woff(k);
            o.llp[m] = m < nout && t >= 0 ? rbase + 8 * roff(k) : 0;
            o.pnw[m] = m < nout && t >= 0 ? (uint64_t)stages[t].norm_w : 0;
        }
        const size_t kx = 3 * (size_t)(o.xsrc >= 0 ? o.xsrc : 0) + xm[s];
        o.llx = xo[s] >= 0 && lp[s] < 0 ? wbase + 8 * woff(kx) : 0;
        o.lpx = lp[s] >= 0 ? rbase + 8 * roff(kx) : 0;
        o.llr = ro[s] >= 0 ? wbase + 8 * woff(3 * (size_t)o.rsrc + rm[s]) : 0;
        const int xb = o.lpx ? o.units * 256 : o.units * (o.llx ? 256 : 128) + (in.norm_w ? o.units * 128 : 0);
        max_xbuf = xb > max_xbuf ? xb : max_xbuf;
    }
    StreamPlan *p = new StreamPlan;
    p->words = words;
    p->nstages = nstages;
    p->fmt = fmt;
    p->lds = stream_lds(fmt, max_units, max_xbuf, p->args);
    if (p->lds > 160 * 1024 || hipMalloc((void **)&p->dev, sizeof(StreamStage) * nstages) != hipSuccess) {
        (void)hipGetLastError();
        delete[] host;
        HOLO_CHECK(hipFree(words));
        delete p;
        HOLO_REJECT("holo_gemv_stream_create: LDS or device memory for the plan");
        return nullptr;
    }
    HOLO_CHECK(hipMemcpy(p->dev, host, sizeof(StreamStage) * nstages, hipMemcpyHostToDevice));
    // each workgroup's slot count (the compute waves' trip count): its tiles of
    // every stage times the stage's slots per tile, as the kernel's walk deals
    // them, rounded up to a multiple of the ring depth
    std::vector<int> slots(grid, 0);
    for (int b = 0; b < grid; b++) {
        long long n = 0;
        for (int s = 0; s < nstages; s++) {
            const StreamStage &o = host[s];
            int e0, e1;
            rem_rows(o.total_rows, o.rem_start, (uint32_t)grid, (uint32_t)b, e0, e1);
            n += (long long)(o.full_tiles + (e1 > e0 ? 1 : 0)) * o.P;
        }
        n = (n + kStreamD - 1) / kStreamD * kStreamD;
        slots[b] = n > INT_MAX ? INT_MAX / kStreamD * kStreamD : (int)n;
    }
    delete[] host;
    if (hipMalloc((void **)&p->slots, sizeof(int) * grid) != hipSuccess) {
        (void)hipGetLastError();
        p->slots = nullptr;
        HOLO_CHECK(hipFree(p->dev));
        HOLO_CHECK(hipFree(words));
        delete p;
        HOLO_REJECT("holo_gemv_stream_create: device memory for the plan");
        return nullptr;
    }
    HOLO_CHECK(hipMemcpy(p->slots, slots.data(), sizeof(int) * grid, hipMemcpyHostToDevice));
    p->args.slots = (uint64_t)(uintptr_t)p->slots;
    p->args.table = (uint64_t)(uintptr_t)p->dev;
    p->args.nstages = nstages;
    p->args.seq = (uint32_t *)words;
    p->args.flag = g_stream_flag;
    return p;
}

int holo_gemv_stream_launch(void *plan)
{
    StreamPlan *p = (StreamPlan *)plan;
    if (!p || !p->dev) {
        HOLO_REJECT("holo_gemv_stream_launch: no plan");
        return HOLO_EINVAL;
    }
    const bool ok = p->fmt == FMT_Q4_0 ? stream_launch_f<FMT_Q4_0>(*p) : stream_launch_f<FMT_Q4_K>(*p);
    if (!ok) {
        HOLO_REJECT("holo_gemv_stream_launch: a workgroup per CU does not fit");
        return HOLO_EINVAL;
    }
    return 0;
}

void holo_gemv_stream_destroy(void *plan)
{
    StreamPlan *p = (StreamPlan *)plan;
    if (!p) return;
    if (p->dev) HOLO_CHECK(hipFree(p->dev));
    if (p->slots) HOLO_CHECK(hipFree(p->slots));
    if (p->words) HOLO_CHECK(hipFree(p->words));
    delete p;
}

int holo_gemv_stream_status(void)
{
    if (!g_stream_flag) return 0;
    uint32_t flag = 0;
    HOLO_CHECK(hipStreamSynchronize(stream()));
    HOLO_CHECK(hipMemcpy(&flag, g_stream_flag, sizeof(flag), hipMemcpyDeviceToHost));
    if (flag == 0) return 0;
    HOLO_CHECK(hipMemset(g_stream_flag, 0, 256));
    HOLO_CHECK(hipDeviceSynchronize());
    return HOLO_ECHAIN;
}

}  // extern "C"
