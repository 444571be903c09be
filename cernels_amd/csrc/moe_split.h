// Per-XCD item ranges of the packed grouped GEMMs, balanced by estimated cost, and the halves their
// ranges end on (tail_items, below). Host and device
// code: the route kernel evaluates it per expert, and a CPU test checks it against a brute-force
// count over the item list (compiled there with CMOE_HD defined empty).
//
// The items of a packed GEMM are (M-tile, N-tile) pairs, listed expert by expert and N-tile-major
// inside an expert. An item of r rows costs 32 fw + r, in bytes streamed through the CU per row of the
// reduction over 32 columns (its fw weight fragments of 32 columns and its r activation rows). Expert
// e's items cost n_tiles * (32 fw nt_e + run_e) together, so the cost before expert e is
// n_tiles * (32 fw toff_e + off_e), from the two prefixes the route has already scanned. XCD x starts
// at the first item whose cost prefix reaches ceil(x W / 8) of the total W. The split applies where an
// equal split of the items gives each workgroup r = ceil(ceil(items / 8) / slots) >= 8 rounds of
// items, and no range may then hold more than (r + r / 8) * slots items. With fewer rounds the equal
// split stays: there one more item in a workgroup costs a whole round, and the XCD's end is set by how
// its items fall into rounds rather than by their summed cost (measured: at 4 rounds the cost split
// was 1-3% slower, at 8-10 rounds 3.5% faster).
#pragma once

#ifndef CMOE_HD
#define CMOE_HD __host__ __device__
#endif

namespace cmoe {

// floor(a / b) for 0 <= a, 0 < b, quotient < 2^20: a float estimate within one of the quotient
// (relative error a few 2^-24), then one exact correction. Avoids the long 64-bit division sequence.
CMOE_HD inline int split_floordiv(long long a, long long b) {
    int q = (int)((float)a * (1.0f / (float)b));
    const long long r = a - (long long)q * b;
    return q + (r >= b ? 1 : 0) - (r < 0 ? 1 : 0);
}

// Writes b[k] for the boundaries k in 1..7 that fall inside one expert: run pairs in nt M-tiles of
// bm rows, the first one toff, off pairs before it; W = 32 fw tiles + pairs of the whole list (the
// cost of one N-tile of every expert).
CMOE_HD inline void split_expert(int fw, int n_tiles, int bm, int run, int nt, int toff, int off, long long W,
                                 int* b) {
    if (nt <= 0) return;
    const long long Wt = (long long)n_tiles * W;
    const long long c = 32LL * fw * nt + run;  // cost of one N-tile of the expert
    const long long S = (long long)n_tiles * (32LL * fw * toff + off), Se = S + n_tiles * c;
    // boundary k lies in (S, Se]: S < ceil(k Wt / 8) <= Se, i.e. 8 S / Wt < k <= 8 Se / Wt
    const int k0 = split_floordiv(8 * S, Wt) + 1, k1 = split_floordiv(8 * Se, Wt);
    for (int k = k0 < 1 ? 1 : k0; k <= (k1 > 7 ? 7 : k1); ++k) {
        const long long R = (k * Wt + 7) / 8 - S;  // 1 <= R <= n_tiles * c
        const int n = split_floordiv(R - 1, c), r = (int)(R - n * c);
        const int full = 32 * fw + bm;                // cost of a full M-tile; only the last one is partial
        const int m = (r + full - 1) / full;          // M-tiles of N-tile n that start before the boundary
        b[k] = toff * n_tiles + n * nt + (m < nt ? m : nt);
    }
}

// b[1..7] from split_expert -> final bounds b[0..8]: the equal split below 8 rounds, else b clamped
// to at most cap items per range. Any b[1..7] gives a valid split (an empty list gives all zeros).
CMOE_HD inline void split_clamp(int* b, int total, int slots) {
    const int per = (total + 7) / 8, rounds = (per + slots - 1) / slots, cap = (rounds + rounds / 8) * slots;
    b[0] = 0;
    if (rounds < 8) {
        for (int k = 1; k < 9; ++k) b[k] = k * per < total ? k * per : total;
        return;
    }
    for (int k = 1; k < 8; ++k) {
        int v = b[k];
        v = v < b[k - 1] + cap ? v : b[k - 1] + cap;
        v = v > total - (8 - k) * cap ? v : total - (8 - k) * cap;
        b[k] = v > b[k - 1] ? v : b[k - 1];
    }
    b[8] = total;
}

// Rows of M-tile m of an expert with `rows` rows in nt = ceil(rows / bm) M-tiles (bm a multiple of 32): the
// tiles split the rows evenly in 32-row blocks, tile m taking blocks [m nb / nt, (m+1) nb / nt) of the
// nb = ceil(rows / 32), rather than bm, bm, ..., remainder. The tiles that share an N-tile's weights then run
// their k-loops at the same speed and stay together in the XCD's L2 (a remainder tile of a few rows ran ahead of
// its full siblings and fetched the weights again). Every tile has 1 .. bm/32 blocks (nb <= (bm / 32) nt), the
// same number of 32-row MFMA blocks in total.
CMOE_HD inline void tile_rows(int m, int nt, int rows, int& row_begin, int& tile_rows_out) {
    const long long nb = (rows + 31) / 32;
    const int b0 = (int)(m * nb / nt), b1 = (int)((m + 1) * nb / nt);
    row_begin = 32 * b0;
    tile_rows_out = (32 * b1 < rows ? 32 * b1 : rows) - 32 * b0;
}

// The tail of one XCD's item range (the packed gate_up GEMM): where the range holds at least three rounds of items
// for its slots, its last min(tail, max_tail, n_items - 2 slots) items are handed out as two halves when they
// have more than 3/4 bm rows. The first two offsets of every slot (taken before the tail table exists) are
// therefore always whole items. A work code is 4 * item + h: h = 0 the whole item, 1 its rows [0, bm/2), 2 its
// rows [bm/2, rows).
CMOE_HD inline int tail_items(int n_items, int slots, int tail, int max_tail) {
    if (n_items < 3 * slots) return 0;
    const int t = tail < max_tail ? tail : max_tail;
    const int room = n_items - 2 * slots;
    return t < room ? t : room;
}
CMOE_HD inline bool tail_splits(int rows, int bm) { return 4 * rows > 3 * bm; }
// The rows of part h of an item that starts at row_begin and has rows rows (h = 0 leaves them).
CMOE_HD inline void tail_part(int h, int bm, int& row_begin, int& rows) {
    if (h == 1) {
        rows = bm / 2;
    } else if (h == 2) {
        row_begin += bm / 2;
        rows -= bm / 2;
    }
}

}  // namespace cmoe
