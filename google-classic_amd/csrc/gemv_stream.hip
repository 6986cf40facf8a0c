// gemv_stream.hip -- a whole chain of dependent GEMV stages (a decode step:
// every layer's q/k/v, o, gate/up and down) in one persistent launch that
// keeps the weight stream running across the stage boundaries.
//
// The reference issues one launch per matrix and token (the decode loop of
// src/ai/llm_cuda.c:604-918; kernels cuda_ops.cu:618-676, 976-1060); the
// results here are those of the separate GEMV calls (the MFMA path of
// gemv.hip: 24-bit activations in three int8 planes, exact int32 block dots,
// fp32 accumulation), with the rms_norm of the stage's input folded into its
// staging and the residual add into its stores.
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
//                   loads and each item's wait is exact.
//   control wave    at a stage's end: sums the 8 partials of each of the
//                   workgroup's rows (64 rows at a time, one per lane), applies
//                   the epilogue (silu(g)*u, or r + acc), stores the outputs,
//                   then gathers the next stage's input.  It issues no weight
//                   loads.
//
// How a stage's output reaches the next stage (no grid barrier): besides the
// plain fp32 output, every output value is also stored as one 64-bit word
// (tag << 32 | value bits) with a single agent-scope store, into the plan's
// exchange buffer of that output vector.  The tag names the launch and the
// stage (base + s + 1, base = launch count * (stages + 1)), so a word is
// either this stage's value or visibly stale.  A consumer copies the words
// of its whole input into LDS (device-coherent global_load_lds), checks every
// tag and copies again only the 1 KB pieces that are not yet current, until
// all are.  Value and tag travel in one single-copy-atomic 64-bit store, so a
// current tag implies the current value: no fence, no store-completion wait
// and no arrival counter sit between a producer's epilogue and its
// consumers.  The launch count advances when the last workgroup of a launch
// ends (a counter in the plan), so the next launch's tags differ from every
// word this launch left behind.
//
// Stage boundary (3 workgroup barriers): A  all partials of stage s in LDS;
// the control wave stores, then gathers the input of stage s+1 (and its norm
// weight) into LDS, in the space of the compute waves' item stages, which are
// idle until C; B  the input is in LDS; all waves convert it (rms_norm if
// asked, then the int8 planes); C  compute resumes.  The compute waves never
// load activations, so nothing but their own weight items counts against
// their vector-memory counter.
#include "gemv_mfma.h"

#include <hip/hip_ext.h>
#include <limits.h>

#include <vector>

namespace holo {

namespace {

constexpr int kNCW = 8;                     // compute waves
constexpr int kStreamThreads = 64 * (kNCW + 1);
constexpr int kStreamMaxTiles = 16;         // tiles of one stage per workgroup
constexpr uint32_t kStreamPolls = 1u << 18;  // bounded exchange wait (~0.3 s)
constexpr int kStreamMaxChunks = 192;        // 1 KB exchange pieces of one input (in_dim <= 24576)

// One stage of the plan, in device memory (read with scalar loads).
struct StreamStage {
    uint64_t W[3];        // matrices (gate/up: gate, up)
    uint64_t y[3];        // outputs (gate/up: y[0])
    uint64_t x;           // input vector, units * 32 floats
    uint64_t nw;          // rms-norm weight (units * 32 floats) or 0
    uint64_t r;           // residual: y[0] = r + W x (plain, one matrix), or 0
    int64_t row_bytes;
    int row_end[3];       // prefix sums of the matrices' rows (plain); INT_MAX unused
    int mode;             // MODE_PLAIN / MODE_GATEUP
    int units;            // 32-weight units per row
    int G;                // 16-unit segments per row
    int P;                // item slots per compute wave per tile: ceil(G / kNCW)
    int total_rows;       // rows of all matrices (plain) or of one (gate/up)
    int full_tiles;       // tiles dealt round robin to every workgroup
    int rem_start;        // first row of the remainder
    float eps;
    uint64_t lly[3];      // exchange words of the outputs (gate/up: lly[0])
    uint64_t llx;         // exchange words of x when an earlier stage wrote it, else 0
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
    uint32_t tpart_off;   // LDS: tile partials [kStreamMaxTiles][kNCW][16]
    uint32_t red_off;     // LDS: norm reduction [16]
    uint32_t xbuf_off;    // LDS: x of the next stage as fp32, then its norm weight
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

// This workgroup's tiles of a stage: F full tiles dealt round robin (tile k
// = global tile k*W + b), then an even share of the remaining rows as one
// short tile.
struct Tiles {
    int F, ex0, ex1, n, TR;
    __device__ __forceinline__ void init(cstage &s, uint32_t W, uint32_t b)
    {
        TR = uni(s.mode == MODE_GATEUP ? 8 : 16);
        F = uni(s.full_tiles);
        const uint32_t rem = (uint32_t)(s.total_rows - s.rem_start);
        ex0 = uni(s.rem_start + (int)((b * rem) / W));
        ex1 = uni(s.rem_start + (int)(((b + 1) * rem) / W));
        n = uni(F + (ex1 > ex0 ? 1 : 0));
    }
    __device__ __forceinline__ void rows(int k, uint32_t W, uint32_t b, int &row0, int &rend) const
    {
        if (k < F) {
            row0 = (k * (int)W + (int)b) * TR;
            rend = row0 + TR;
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
// this workgroup's n tiles, slot p < P of the tile (segment cw + kNCW * p).
// Tracked incrementally (no division per slot); the stage constants are
// read once per stage, into scalar registers.  A stage with no tile for this
// workgroup is skipped; s = nstages is past the end, where the issue fields
// are those of the last stage (the dummy loads read its first item).
struct Walk {
    int s, k, p;
    int n, P, G, F, TR, units;
    int row0, rend, ex0, ex1;

    __device__ __forceinline__ void set_tile(uint32_t W, uint32_t b)
    {
        if (k < F) {
            row0 = uni((k * (int)W + (int)b) * TR);
            rend = row0 + TR;
        } else {
            row0 = ex0;
            rend = ex1;
        }
    }
    __device__ __forceinline__ void enter(const StreamArgs &a, int stage, uint32_t W, uint32_t b)
    {
        // locals, assigned to the members once: a loop over the members
        // themselves keeps the struct in scratch memory
        int ss = stage, tr = 16, f = 0, e0 = 0, e1 = 0, nn = 0;
        for (; ss < a.nstages; ss++) {
            cstage &st = stage_at(a, ss);
            tr = st.mode == MODE_GATEUP ? 8 : 16;
            f = st.full_tiles;
            const uint32_t rem = (uint32_t)(st.total_rows - st.rem_start);
            e0 = st.rem_start + (int)((b * rem) / W);
            e1 = st.rem_start + (int)(((b + 1) * rem) / W);
            nn = f + (e1 > e0 ? 1 : 0);
            if (nn > 0) break;
        }
        s = uni(ss);
        TR = uni(tr);
        F = uni(f);
        ex0 = uni(e0);
        ex1 = uni(e1);
        n = uni(nn);
        k = 0;
        p = 0;
        cstage &st = stage_at(a, s < a.nstages ? s : a.nstages - 1);
        G = uni(st.G);
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
// piece i at rowaddr[i] + col + the 16-unit segment's offset, one code path
// for every tile and segment.  rowaddr (per tile) is the lane's row: its
// piece row clamped to the tile's last row (short tiles re-read that row), in
// the matrix the row falls in (rows of several matrices, or 8 gate + 8 up
// rows).  The column part is the piece's 16-byte column (colF), or in an
// 8-unit last segment the column taken modulo half the segment (item_piece's
// half mapping: the missing half re-reads the first), so no load leaves the
// row.
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
        const bool gu = uni(st.mode) == MODE_GATEUP;
        const uint64_t w0 = uni64(st.W[0]), w1 = uni64(st.W[1]), w2 = uni64(st.W[2]);
        const int re0 = uni(st.row_end[0]), re1 = uni(st.row_end[1]);
        const int row0 = c.row0, last = c.rend - 1;
#pragma unroll
        for (int i = 0; i < Geo<FMT>::NL; i++) {
            const int pr = item_piece(FMT, 64 * i + lane, false).row;
            if (gu) {
                const int v = min(row0 + (pr & 7), last);
                rowaddr[i] = ((pr >> 3) ? w1 : w0) + (uint64_t)v * rb;
            } else {
                const int v = min(row0 + pr, last);
                const int a1 = v >= re0, a2 = v >= re1;
                const int r = v - (a2 ? re1 : a1 ? re0 : 0);
                rowaddr[i] = (a2 ? w2 : a1 ? w1 : w0) + (uint64_t)r * rb;
            }
        }
    }
};

// Item of the issue walk's slot into registers: NL 16-byte loads per lane,
// the kernel's only weight loads.  Every slot issues exactly NL loads from
// this one site, so the compiler's vmcnt wait for any slot is exact: a slot
// with no segment for this wave re-reads the tile's last segment, and a slot
// past the last stage re-reads item 0 of the last stage.  The data of such
// slots is never used.
template <int FMT>
__device__ __forceinline__ void stream_issue(Raw2<FMT> &buf, const Walk &c, const Issuer<FMT> &is, int cw)
{
    using GE = Geo<FMT>;
    const int seg = uni(min(cw + kNCW * c.p, c.G - 1));
    const bool half = 16 * seg + 16 > c.units;
    const uint32_t segoff = (uint32_t)seg * GE::SEGB;
#pragma unroll
    for (int i = 0; i < GE::NL; i++) {
        const uint32_t col = half && is.colF[i] >= 8u * GE::PR ? is.colF[i] - 8u * GE::PR : is.colF[i];
        buf.v[i] = __builtin_nontemporal_load((gu32x4a *)(is.rowaddr[i] + (col + segoff)));
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

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void gvoid;

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

// Waits until every workgroup has stored its rows of the stage with tag
// `tag` (its done word holds that tag or a later one of this launch).  A done
// word is stored right after the workgroup's exchange words, without waiting
// for them to complete, so it only says that the words are on their way: the
// gather still checks every word's tag.  The wait keeps the polling to 4
// bytes per workgroup instead of the whole input.
__device__ __forceinline__ void stream_wait_done(const uint32_t *done, uint32_t tag, uint32_t *flag, int lane)
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
            __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        __builtin_amdgcn_s_sleep(2);
    }
}

// The input of a stage that an earlier stage wrote: its exchange words
// (8 bytes per value) into LDS, 1 KB pieces of 128 words, device-coherent
// (sc1: never answered from a line this XCD's L2 held before another XCD's
// store).  The tags are checked while the words are converted
// (stream_convert_x); stream_stage_in copies again what was not current.
__device__ __forceinline__ void stream_fetch_tagged(cstage &st, uint8_t *xbuf, int lane)
{
    const int units = uni(st.units), nch = units / 4;  // 128 words = 4 units per piece
    const uint8_t *src = (const uint8_t *)uni64(st.llx);
    for (int j = 0; j < nch; j++)
        __builtin_amdgcn_global_load_lds((gvoid *)(src + 1024 * j + 16 * lane), (lds_void *)(xbuf + 1024 * j), 16, 0,
                                         kDeviceScope);
}

// x value chunk i (4 values) of the staged input: plain fp32, or exchange
// words (value, tag) pairs, whose tags must all be `tag` (else `bad`).
__device__ __forceinline__ float4 staged_x4(const uint8_t *xbuf, int i, bool tagged, uint32_t tag, bool &bad)
{
    if (tagged) {
        const uint4 a = *(const uint4 *)(xbuf + 32 * i), b = *(const uint4 *)(xbuf + 32 * i + 16);
        bad |= (a.y != tag) | (a.w != tag) | (b.y != tag) | (b.w != tag);
        return make_float4(__uint_as_float(a.x), __uint_as_float(a.z), __uint_as_float(b.x), __uint_as_float(b.z));
    }
    return *(const float4 *)(xbuf + 16 * i);
}

constexpr int kRedBad = 15;   // red[15]: a stale exchange word was staged
constexpr int kRedBase = 14;  // red[14]: this launch's tag base, from the control wave

// The staged x in LDS into the int8 planes and {dx, c} pairs, by all threads;
// with a norm weight, x * (1/sqrt(mean(x^2) + eps)) * w first (cuda_rms_norm's
// formula, cuda_ops.cu:1479-1504), the 9 waves' sums of squares meeting in red.
template <int FMT>
__device__ __forceinline__ void stream_convert_x(cstage &st, uint8_t *ldsb, const uint8_t *xbuf, float *red,
                                                 uint32_t tag)
{
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int units = uni(st.units), chunks = units * 8;
    const bool norm = uni64(st.nw) != 0;
    const bool tagged = uni64(st.llx) != 0;
    bool bad = false;
    float scale = 1.f;
    if (norm) {
        float ss = 0.f;
        for (int i = tid; i < chunks; i += kStreamThreads) {
            const float4 v = staged_x4(xbuf, i, tagged, tag, bad);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w <= kNCW; w++) tot += red[w];
        scale = 1.0f / sqrtf(tot / (float)(units * 32) + unif(st.eps));
    }
    const float4 *wv = (const float4 *)(xbuf + units * (tagged ? 256 : 128));
    for (int i = tid; i < chunks; i += kStreamThreads) {
        float4 v = staged_x4(xbuf, i, tagged, tag, bad);
        if (norm) {
            const float4 w4 = wv[i];
            v = make_float4(v.x * scale * w4.x, v.y * scale * w4.y, v.z * scale * w4.z, v.w * scale * w4.w);
        }
        x_convert<FMT, XM_MFMA>(v, i, units, (void *)ldsb);
    }
    if (tagged && __ballot(bad) != 0 && lane == 0) ((uint32_t *)red)[kRedBad] = 1u;
}

// After the input of stage `st` was staged (B): all waves convert it (C), and
// while a stale exchange word was among it, the control wave copies the words
// again and all waves convert again.  Every wave takes the same rounds (each
// reads the flag after the same barrier), so the barrier counts agree.  After
// kStreamPolls rounds the wait gives up and sets the plan's flag.
template <int FMT>
__device__ __forceinline__ void stream_stage_in(cstage &st, uint8_t *ldsb, uint8_t *xbuf, float *red, uint32_t base,
                                                uint32_t *flag, bool control, int lane)
{
    const uint32_t tag = base + (uint32_t)uni(st.xsrc) + 1u;
    stream_convert_x<FMT>(st, ldsb, xbuf, red, tag);
    __syncthreads();  // C
    if (uni64(st.llx) == 0) return;
    uint32_t *badp = (uint32_t *)red + kRedBad;
    for (uint32_t round = 0; uni((int)*badp) != 0; round++) {
        __syncthreads();  // every wave has read the flag
        if (control) {
            if (lane == 0) *badp = 0u;
            if (round == kStreamPolls) {
                __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __builtin_amdgcn_s_sleep(4);
                stream_fetch_tagged(st, xbuf, lane);
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            }
        }
        __syncthreads();  // B again
        if (round < kStreamPolls) stream_convert_x<FMT>(st, ldsb, xbuf, red, tag);
        __syncthreads();  // C again
    }
}

// Row v of this workgroup's rows of a stage for lane `lane` in pass q: 64
// rows a pass, tile k = q * (64 / TR) + lane / TR, row lane % TR of it.
__device__ __forceinline__ bool own_row(const Tiles &t, int q, int lane, uint32_t W, uint32_t b, int &k, int &i,
                                        int &v)
{
    const int per = 64 / t.TR;
    k = q * per + lane / t.TR;
    i = lane % t.TR;
    int row0, rend;
    t.rows(k, W, b, row0, rend);
    v = row0 + i;
    return k < t.n && v < rend;
}

constexpr int kStreamPasses = kStreamMaxTiles * 16 / 64;  // passes of 64 rows over at most 16 tiles

__device__ __forceinline__ uint64_t exchange_word(float v, uint32_t tag)
{
    return ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}

// The residual rows r[v] of this workgroup's rows of stage s (plain stages
// with r), one per lane and pass: exchange words when an earlier stage wrote
// r (waited for like the input), else the caller's fp32 values.
__device__ __forceinline__ void stream_residual(cstage &st, const Tiles &t, float (&rr)[kStreamPasses], uint32_t base,
                                                uint32_t *flag, uint32_t W, uint32_t b, int lane)
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
            if (mine)
                w = __hip_atomic_load((__attribute__((address_space(1))) uint64_t *)llr + v, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
            if (__ballot(mine && (uint32_t)(w >> 32) != tag) == 0) break;
            if (polls == kStreamPolls) {
                __hip_atomic_store(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        rr[q] = __uint_as_float((uint32_t)w);
    }
}

// The control wave's stores of stage s: each of the workgroup's rows (one per
// lane and pass), the 8 compute waves' partials summed in wave order; the
// plain fp32 output and its exchange word.
__device__ __forceinline__ void stream_epilogue(cstage &st, const Tiles &t, const float *tpart,
                                                const float (&rr)[kStreamPasses], uint32_t tag, uint32_t W,
                                                uint32_t b, int lane)
{
    typedef __attribute__((address_space(1))) uint64_t gword;
    const bool gu = uni(st.mode) == MODE_GATEUP;
    const uint64_t y0 = uni64(st.y[0]), y1 = uni64(st.y[1]), y2 = uni64(st.y[2]);
    const uint64_t l0 = uni64(st.lly[0]), l1 = uni64(st.lly[1]), l2 = uni64(st.lly[2]);
    const bool res = uni64(st.r) != 0;
    const int per = 64 / t.TR;
#pragma unroll
    for (int q = 0; q < kStreamPasses; q++) {
        if (q * per >= t.n) break;
        int k, i, v;
        if (own_row(t, q, lane, W, b, k, i, v)) {
            const float *pt = tpart + k * (kNCW * 16);
            float s0 = 0.f;
#pragma unroll
            for (int w = 0; w < kNCW; w++) s0 += pt[w * 16 + i];
            if (gu) {
                float s1 = 0.f;
#pragma unroll
                for (int w = 0; w < kNCW; w++) s1 += pt[w * 16 + 8 + i];
                const float o = silu(s0) * s1;
                ((gfloat *)y0)[v] = o;
                __hip_atomic_store((gword *)l0 + v, exchange_word(o, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                int m, row;
                split_row(st, v, m, row);
                if (res) s0 = rr[q] + s0;
                ((gfloat *)(m == 2 ? y2 : m == 1 ? y1 : y0))[row] = s0;
                __hip_atomic_store((gword *)(m == 2 ? l2 : m == 1 ? l1 : l0) + row, exchange_word(s0, tag),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
}

__device__ __forceinline__ void stream_mark_done(uint32_t *done, uint32_t tag, uint32_t b, int lane)
{
    if (lane == 0) __hip_atomic_store(done + b, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
            stream_issue<FMT>(ring[d], ci, is, cw);
            advance();
        }
        __syncthreads();  // B of stage 0: x in LDS
        const uint32_t base = (uint32_t)uni((int)((uint32_t *)red)[kRedBase]);
        stream_convert_x<FMT>(stage_at(a, 0), ldsb, xbuf, red, 0u);
        __syncthreads();  // C of stage 0
        int s = 0;        // the stage whose boundary comes next
        float acc = 0.f;
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
                    if (s + 1 < nst) stream_stage_in<FMT>(stage_at(a, s + 1), ldsb, xbuf, red, base, a.flag, false, lane);
                    s++;
                }
                // a slot past the last stage writes its (unused) item too, so
                // every slot's wait counts the same loads
                stream_stage_write<FMT>(ring[d], stage, lane);
                stream_issue<FMT>(ring[d], ci, is, cw);
                advance();
                // the slot's dots against the staged x of stage s
                const int j = cw + kNCW * cp.p;
                if (cp.s < nst && j < cp.G) {
                    const int units = cp.units;
                    Chunk<FMT> c;
                    read_chunk<FMT>(c, stage, n, g);
                    const int cs0 = 16 * j + 4 * g;
                    const bool valid = cs0 < units;  // false only in an 8-unit last segment
                    const int cs = valid ? cs0 : units - 4;
                    const uint32_t abase = plane_lane ? (uint32_t)cs * 96u + plane_off : a.zero_off;
                    acc += item_dot<FMT>(c, ldsb, abase, (uint32_t)units * 96u + (uint32_t)cs * 8u, (uint32_t)cs,
                                         valid ? 0 : 4, j == cp.G - 1);
                }
                if (cp.s < nst && cp.p == cp.P - 1) {
                    float r = acc;
                    r += __shfl_xor(r, 16);
                    r += __shfl_xor(r, 32);
                    acc = 0.f;
                    if (lane < 16) tpart[(cp.k * kNCW + cw) * 16 + lane] = r;
                }
                cp.next(a, W, b);
            }
        }
        // the boundaries after this wave's last slot
        while (s < nst) {
            __syncthreads();  // A
            __syncthreads();  // B
            if (s + 1 < nst) stream_stage_in<FMT>(stage_at(a, s + 1), ldsb, xbuf, red, base, a.flag, false, lane);
            s++;
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the last (dummy) item loads have returned
    } else {
        // ---- control wave ----
        const uint32_t seq0 = __hip_atomic_load(a.seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t base = uni((int)(seq0 * (uint32_t)(nst + 1)));
        {
            cstage &st0 = stage_at(a, 0);
            stream_fetch_plain(st0, xbuf, lane);
            if (uni64(st0.nw)) stream_fetch_norm(st0, xbuf + uni(st0.units) * 128, lane);
        }
        if (lane == 0) ((uint32_t *)red)[kRedBase] = base;
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the LDS-direct loads have landed
        __syncthreads();                     // B of stage 0
        stream_convert_x<FMT>(stage_at(a, 0), ldsb, xbuf, red, 0u);
        __syncthreads();  // C of stage 0
        for (int s = 0; s < nst; s++) {
            cstage &st = stage_at(a, s);
            Tiles t;
            t.init(st, W, b);
            // residual rows of this stage's rows, gathered while the stage runs
            float rr[kStreamPasses];
            stream_residual(st, t, rr, base, a.flag, W, b, lane);
            __syncthreads();  // A: every partial of stage s is in LDS
            stream_epilogue(st, t, tpart, rr, base + (uint32_t)s + 1u, W, b, lane);
            stream_mark_done(a.seq + 128, base + (uint32_t)s + 1u, b, lane);
            if (s + 1 < nst) {
                cstage &st1 = stage_at(a, s + 1);
                const int units1 = uni(st1.units);
                const bool tagged = uni64(st1.llx) != 0;
                // the partial reads above are done before any copy lands in
                // their space (xbuf aliases the item stages and partials)
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                if (uni64(st1.nw)) stream_fetch_norm(st1, xbuf + units1 * (tagged ? 256 : 128), lane);
                if (tagged) {
                    if (lane == 0) ((uint32_t *)red)[kRedBad] = 0u;
                    stream_wait_done(a.seq + 128, base + (uint32_t)uni(st1.xsrc) + 1u, a.flag, lane);
                    stream_fetch_tagged(st1, xbuf, lane);
                }
                else
                    stream_fetch_plain(st1, xbuf, lane);
                __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            }
            __syncthreads();  // B
            if (s + 1 < nst) stream_stage_in<FMT>(stage_at(a, s + 1), ldsb, xbuf, red, base, a.flag, true, lane);
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

// LDS: [x planes + {dx, c}][zero region][norm reduction][region], where the
// region holds the compute waves' item stages and the tile partials during a
// stage, and the staged input (fp32 or exchange words, then the norm weight)
// during a boundary.
size_t stream_lds(int fmt, int max_units, int max_xbuf, uint32_t &zero_off, uint32_t &stage_off,
                  uint32_t &tpart_off, uint32_t &red_off, uint32_t &xbuf_off)
{
    const size_t x_lds = ((size_t)max_units * lds_bytes_per_unit<XM_I24>() + 15) & ~(size_t)15;
    zero_off = zero_region_off((uint32_t)x_lds);
    red_off = zero_off + kZeroBytes;
    stage_off = (red_off + 16 * 4 + 15) & ~15u;
    const int stage = fmt == FMT_Q4_0 ? Geo<FMT_Q4_0>::STAGE : fmt == FMT_Q8_0 ? Geo<FMT_Q8_0>::STAGE
                                                                                : Geo<FMT_Q4_K>::STAGE;
    tpart_off = (stage_off + kNCW * stage + 15) & ~15u;
    xbuf_off = stage_off;
    const size_t during = tpart_off + (size_t)kStreamMaxTiles * kNCW * 16 * 4;
    const size_t boundary = xbuf_off + (size_t)max_xbuf;
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

constexpr int kStreamD = 4;  // items in flight per compute wave

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
        for (int m = 0; m < 3; m++) {
            if (m < nmat) {
                const int rows = in.rows[gu ? 0 : m];
                float *y = in.y[gu ? 0 : m];
                ok = ok && in.W[m] && !((uintptr_t)in.W[m] & 15u) && rows > 0 && y;
                o.W[m] = (uint64_t)in.W[m];
                o.y[m] = (uint64_t)y;
                total += rows;
                o.row_end[m] = total;
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
        o.P = (o.G + kNCW - 1) / kNCW;
        const int tr = gu ? 8 : 16;
        o.total_rows = gu ? in.rows[0] : total;
        o.full_tiles = o.total_rows / (grid * tr);
        o.rem_start = o.full_tiles * grid * tr;
        if (o.full_tiles + 1 > kStreamMaxTiles) {
            delete[] host;
            HOLO_REJECT("holo_gemv_stream_create: a stage with more rows than 16 tiles per CU");
            return nullptr;
        }
        max_units = o.units > max_units ? o.units : max_units;
    }
    // Exchange buffers: one per distinct output vector (keyed by its address),
    // as many words as the most rows any stage writes there.  A stage's x or r
    // that an earlier stage wrote is read from that buffer (xsrc / rsrc: the
    // last writer before it); an input that overlaps an earlier output in any
    // other way, an output that overlaps its own stage's x, two outputs of one
    // stage in one vector, or outputs that partly overlap are rejected.
    struct OutVec {
        uint64_t ptr;
        int rows, last;
        size_t off;
    };
    std::vector<OutVec> outs;
    std::vector<int> xo(nstages, -1), ro(nstages, -1), yo(3 * (size_t)nstages, -1);
    auto overlap = [](uint64_t a, uint64_t an, uint64_t b, uint64_t bn) { return a < b + bn && b < a + an; };
    auto source = [&](uint64_t ptr, int n, int &idx, int &src) {
        idx = -1;
        src = -1;
        for (size_t i = 0; i < outs.size(); i++) {
            if (outs[i].ptr == ptr) {
                if (outs[i].rows < n) return false;
                idx = (int)i;
                src = outs[i].last;
            } else if (overlap(ptr, 4ull * n, outs[i].ptr, 4ull * outs[i].rows)) {
                return false;
            }
        }
        return true;
    };
    bool xok = true;
    for (int s = 0; s < nstages && xok; s++) {
        const holo_stream_stage_t &in = stages[s];
        StreamStage &o = host[s];
        xok = source(o.x, in.in_dim, xo[s], o.xsrc);
        if (xok && in.r) xok = source(o.r, in.rows[0], ro[s], o.rsrc);
        const int nout = in.gate_up ? 1 : in.nmat;
        for (int m = 0; m < nout && xok; m++) {
            const uint64_t y = (uint64_t)in.y[m];
            const int rows = in.rows[m];
            if (overlap(y, 4ull * rows, o.x, 4ull * in.in_dim)) xok = false;
            int hit = -1;
            for (size_t i = 0; i < outs.size() && xok; i++) {
                if (outs[i].ptr == y) hit = (int)i;
                else if (overlap(y, 4ull * rows, outs[i].ptr, 4ull * outs[i].rows)) xok = false;
            }
            if (!xok) break;
            if (hit < 0) {
                outs.push_back(OutVec{y, rows, s, 0});
                hit = (int)outs.size() - 1;
            } else if (outs[hit].last == s) {
                xok = false;
                break;
            } else {
                outs[hit].rows = rows > outs[hit].rows ? rows : outs[hit].rows;
                outs[hit].last = s;
            }
            yo[3 * (size_t)s + m] = hit;
        }
    }
    if (!xok) {
        delete[] host;
        HOLO_REJECT("holo_gemv_stream_create: a stage input that overlaps an earlier output other than exactly, or "
                    "an output overlapping its own input or another output");
        return nullptr;
    }
    size_t nwords = 0;
    for (OutVec &v : outs) {
        v.off = nwords;
        nwords += (size_t)v.rows;
    }
    // launch counter line, done counter line, one done word per workgroup
    const size_t kWordsHeader = (512 + 4 * (size_t)grid + 255) & ~(size_t)255;
    const size_t words_bytes = kWordsHeader + 8 * nwords;
    uint8_t *words = nullptr;
    if (hipMalloc((void **)&words, words_bytes) != hipSuccess) {
        (void)hipGetLastError();
        delete[] host;
        HOLO_REJECT("holo_gemv_stream_create: device memory for the exchange buffers");
        return nullptr;
    }
    HOLO_CHECK(hipMemset(words, 0, words_bytes));
    const uint64_t wbase = (uint64_t)(uintptr_t)words + kWordsHeader;
    for (int s = 0; s < nstages; s++) {
        const holo_stream_stage_t &in = stages[s];
        StreamStage &o = host[s];
        const int nout = in.gate_up ? 1 : in.nmat;
        for (int m = 0; m < 3; m++) o.lly[m] = wbase + 8 * outs[yo[3 * (size_t)s + (m < nout ? m : 0)]].off;
        o.llx = xo[s] >= 0 ? wbase + 8 * outs[xo[s]].off : 0;
        o.llr = ro[s] >= 0 ? wbase + 8 * outs[ro[s]].off : 0;
        const int xb = o.units * (o.llx ? 256 : 128) + (in.norm_w ? o.units * 128 : 0);
        max_xbuf = xb > max_xbuf ? xb : max_xbuf;
    }
    StreamPlan *p = new StreamPlan;
    p->words = words;
    p->nstages = nstages;
    p->fmt = fmt;
    p->lds = stream_lds(fmt, max_units, max_xbuf, p->args.zero_off, p->args.stage_off, p->args.tpart_off,
                        p->args.red_off, p->args.xbuf_off);
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
            const uint32_t rem = (uint32_t)(o.total_rows - o.rem_start);
            const int e0 = o.rem_start + (int)(((uint32_t)b * rem) / (uint32_t)grid);
            const int e1 = o.rem_start + (int)(((uint32_t)(b + 1) * rem) / (uint32_t)grid);
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
