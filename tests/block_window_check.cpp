// Host-side bounds check of every load window the GEMV kernels issue.
// Usage: block_window_check fmt rows in_dim [fmt rows in_dim ...]
// For each (row, unit) the kernel can touch, it rebuilds the load addresses
// with the kernel's own helpers (google-classic_amd/csrc/block_window.h) for
// a matrix at a 4-byte-aligned base, and checks:
//   * every loaded byte range starts inside the matrix;
//   * the window holds the whole block and starts at most 2 bytes before it;
//   * a dword that reaches past the matrix end starts inside the block and is
//     4-byte aligned (so it cannot leave the block's memory page).
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
    }
    printf("ok %ld\n", checked);
    return 0;
}
