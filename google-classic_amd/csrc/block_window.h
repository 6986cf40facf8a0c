// block_window.h -- byte windows that the GEMV kernels load for one unit.
//
// Shared by the kernels (gemv.hip) and by the CPU bounds check
// (tests/test_block_window.py compiles tests/block_window_check.cpp against
// this header), so the arithmetic that decides every load address is
// checked on the host for each tested shape.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define HOLO_HD __host__ __device__ __forceinline__
#else
#define HOLO_HD static inline
#endif

namespace holo {

// GGUF block formats served by the GEMV.
enum Fmt { FMT_Q4_0 = 0, FMT_Q8_0 = 1, FMT_Q4_K = 2 };

// Units (32-weight groups) per row and bytes per row: in_dim/QK blocks,
// truncating, as the reference (cuda_ops.cu:624, 699).
HOLO_HD int units_per_row(int fmt, int in_dim) { return fmt == FMT_Q4_K ? (in_dim / 256) * 8 : in_dim / 32; }

HOLO_HD int64_t row_bytes_of(int fmt, int in_dim)
{
    return fmt == FMT_Q4_0 ? (int64_t)(in_dim / 32) * 18
         : fmt == FMT_Q8_0 ? (int64_t)(in_dim / 32) * 34
                           : (int64_t)(in_dim / 256) * 144;
}

// Byte offset, within its row, of unit u's block (Q4_0/Q8_0) or superblock (Q4_K).
HOLO_HD uint32_t unit_offset(int fmt, uint32_t u)
{
    return fmt == FMT_Q4_0 ? u * 18u : fmt == FMT_Q8_0 ? u * 34u : (u >> 3) * 144u;
}

// The dword-aligned window holding a Q4_0/Q8_0 block.
//   row_mis  = (row base address) & 3   (rows of an odd block count start on
//              a 2-byte boundary)
//   off      = unit_offset(u)
// The window starts `start` bytes after the row base rounded down to 4, and
// the block sits `s` (0 or 2) bytes into it.  start = (off + row_mis) & ~3
// is never negative, so the window starts at most 2 bytes before the block,
// and only when the block is not the matrix's first.
struct Window {
    uint32_t start;  // relative to (row base & ~3)
    uint32_t s;      // block offset inside the window
};

HOLO_HD Window block_window(uint32_t row_mis, uint32_t off)
{
    uint32_t o = off + row_mis;
    Window w;
    w.start = o & ~3u;
    w.s = o & 3u;
    return w;
}

// Bytes loaded per window: Q4_0 18-byte block -> 5 dwords, Q8_0 34-byte
// block -> 9 dwords.  When s == 0 the last dword holds 2 bytes past the
// block; it is dword-aligned and begins inside the block, so it lies in the
// same memory page as the block and the read cannot fault.
HOLO_HD uint32_t window_bytes(int fmt) { return fmt == FMT_Q4_0 ? 20u : 36u; }

// ---- coalesced item loads of the MFMA GEMV ------------------------------------
// An item is 16 rows x one 16-unit segment: seg_bytes(fmt) contiguous bytes
// of each row, at byte seg * seg_bytes in the row.  A wave loads it as
// 16-byte pieces: piece p = 64*i + lane (load i) is row p / PR, bytes
// [16*(p % PR), +16) of the row's segment, PR = seg_bytes / 16 pieces per
// row (so each load instruction reads whole row runs) and is stored at
// 16*p in the wave's LDS stage.  Requires units % 8 == 0, so a row's byte
// count is a multiple of 16 and a row's last segment holds 16 or 8 units;
// in an 8-unit segment the pieces of the missing half re-read the first
// half (pieces with column >= PR/2 take column - PR/2).
HOLO_HD int seg_bytes(int fmt) { return fmt == FMT_Q8_0 ? 544 : 288; }

HOLO_HD int item_pieces(int fmt) { return 16 * (seg_bytes(fmt) / 16); }

struct Piece {
    int row;   // row within the item (0..15)
    int col;   // 16-byte column within the row's segment
};

HOLO_HD Piece item_piece(int fmt, int p, bool half_segment)
{
    const int pr = seg_bytes(fmt) / 16;
    const int np = 16 * pr;
    if (p > np - 1) p = np - 1;
    Piece q;
    q.row = p / pr;
    q.col = p - q.row * pr;
    if (half_segment && q.col >= pr / 2) q.col -= pr / 2;
    return q;
}

}  // namespace holo
