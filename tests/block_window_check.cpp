// Host-side bounds check of every load window the GEMV kernels issue.
// Usage: block_window_check fmt rows in_dim [fmt rows in_dim ...]
// For each (row, unit) the kernel can touch, it rebuilds the load addresses
// with the kernel's own helpers (google-classic_amd/csrc/block_window.h) for
// a matrix at a 4-byte-aligned base, and checks:
//   * every loaded byte range starts inside the matrix;
//   * the window holds the whole block and starts at most 2 bytes before it;
//   * a dword that reaches past the matrix end starts inside the block and is
//     4-byte aligned (so it cannot leave the block's memory page).
// For shapes the MFMA GEMV takes (units per row a multiple of 8), it also
// rebuilds every 16-byte piece of every item load and checks that it lies
// inside its row and that the stage bytes the lanes decode as valid units hold
// exactly those units' bytes.
// Prints "ok N" (N windows checked) or the first violation, exit status 1.
#include <stdio.h>
#include <stdlib.h>

#include "block_window.h"

using namespace holo;

static int fail(const char *what, int fmt, long row, long u, long a, long b, long total)
{
    printf("FAIL fmt=%d row=%ld u=%ld: %s (a=%ld b=%ld total=%ld)\n", fmt, row, u, what, a, b, total);
    return 1;
}

int main(int argc, char **argv)
{
    long checked = 0;
    for (int i = 1; i + 2 < argc; i += 3) {
        int fmt = atoi(argv[i]);
        long rows = atol(argv[i + 1]);
        int in_dim = atoi(argv[i + 2]);
        long units = units_per_row(fmt, in_dim);
        long rb = (long)row_bytes_of(fmt, in_dim);
        long total = rows * rb;
        for (long row = 0; row < rows; row++) {
            long base = row * rb;  // matrix base at address 0 (4-byte aligned)
            unsigned mis = (unsigned)(base & 3);
            long ba = base - mis;
            for (long u = 0; u < units; u++) {
                unsigned off = unit_offset(fmt, (unsigned)u);
                checked++;
                if (fmt == FMT_Q4_K) {
                    long sb = ba + mis + off;
                    long q = sb + 16 + 16 * (u & 7);
                    if (sb < 0 || sb + 16 > total) return fail("header out of range", fmt, row, u, sb, sb + 16, total);
                    if (q < 0 || q + 16 > total) return fail("quants out of range", fmt, row, u, q, q + 16, total);
                    continue;
                }
                long bsize = fmt == FMT_Q4_0 ? 18 : 34;
                long block = base + off;
                Window w = block_window(mis, off);
                long ws = ba + w.start, we = ws + window_bytes(fmt);
                if (ws + (long)w.s != block) return fail("s does not locate the block", fmt, row, u, ws, block, total);
                if (ws & 3) return fail("window not dword aligned", fmt, row, u, ws, we, total);
                if (ws < 0) return fail("window starts before the matrix", fmt, row, u, ws, we, total);
                if (block - ws > 2) return fail("window starts > 2 bytes early", fmt, row, u, ws, block, total);
                if (we < block + bsize) return fail("window misses block bytes", fmt, row, u, we, block + bsize, total);
                for (long d = ws; d < we; d += 4) {
                    if (d >= total) return fail("dword starts past the matrix", fmt, row, u, d, d + 4, total);
                    if (d + 4 > total && d < block) return fail("straddling dword not inside block", fmt, row, u, d, block, total);
                }
            }
        }
        // MFMA item pieces (units a multiple of 8)
        if (units < 8 || (units & 7)) continue;
        const long segb = seg_bytes(fmt), pr = segb / 16, np = item_pieces(fmt);
        if (rb % 16) return fail("row bytes not a multiple of 16", fmt, 0, 0, rb, 16, total);
        const long nseg = (units + 15) / 16;
        for (long seg = 0; seg < nseg; seg++) {
            const bool half = 16 * seg + 16 > units;
            if (half && units - 16 * seg != 8) return fail("last segment neither 16 nor 8 units", fmt, 0, seg, units, 0, total);
            // stage bytes that valid lane groups read must hold their own row bytes
            const long valid_bytes = half ? segb / 2 : segb;
            for (long p = 0; p < 64 * ((np + 63) / 64); p++) {
                Piece q = item_piece(fmt, (int)p, half);
                checked++;
                if (q.row < 0 || q.row > 15 || q.col < 0 || q.col >= pr) return fail("piece outside the item", fmt, q.row, p, q.col, pr, total);
                long a = seg * segb + 16 * q.col;  // byte in the row
                if (a + 16 > rb) return fail("piece past the row end", fmt, q.row, p, a, rb, total);
                if (p < np) {
                    long stage_col = p % pr;
                    if (stage_col * 16 < valid_bytes && q.col != stage_col)
                        return fail("valid stage bytes not from their own row position", fmt, q.row, p, q.col, stage_col, total);
                    if (p / pr != q.row) return fail("piece row does not match its stage row", fmt, q.row, p, p / pr, 0, total);
                }
            }
        }
    }
    printf("ok %ld\n", checked);
    return 0;
}
