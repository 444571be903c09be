// Host driver of the packed GEMMs' per-XCD split (cernels_amd/csrc/moe_split.h), for
// test_xcd_split.py. Reads cases from stdin, one per line:
//   "S E fw n_tiles slots run_0 .. run_{E-1}" -> the 9 bounds, evaluated the way the route kernel
//     does: exclusive prefixes of pairs and of 256-row M-tiles over experts, split_expert per
//     expert, then split_clamp;
//   "D a b" -> split_floordiv(a, b);
//   "T n slots tail bm rows_0 .. rows_{n-1}" (the items of one XCD range) -> one line per work offset,
//     "item h row_begin rows" (row_begin relative to the item), in the order the packed gate_up GEMM hands
//     them out: the whole items before the tail, then the tail table (items in order, halves in order);
//   "R rows bm" -> the M-tiles of an expert with `rows` rows (ceil(rows / bm) of them, tile_rows), one line
//     "row_begin rows" each, then "END".
#include <cstdio>
#include <vector>

#include "moe_split.h"

int main() {
    char op;
    while (std::scanf(" %c", &op) == 1) {
        if (op == 'D') {
            long long a, b;
            if (std::scanf("%lld %lld", &a, &b) != 2) return 1;
            std::printf("%d\n", cmoe::split_floordiv(a, b));
            continue;
        }
        if (op == 'R') {
            int rows, bm;
            if (std::scanf("%d %d", &rows, &bm) != 2) return 1;
            const int nt = (rows + bm - 1) / bm;
            for (int m = 0; m < nt; ++m) {
                int rb = 0, r = 0;
                cmoe::tile_rows(m, nt, rows, rb, r);
                std::printf("%d %d\n", rb, r);
            }
            std::printf("END\n");
            continue;
        }
        if (op == 'T') {
            int n, slots, tail, bm;
            if (std::scanf("%d %d %d %d", &n, &slots, &tail, &bm) != 4) return 1;
            std::vector<int> rows(n);
            for (auto& r : rows) std::scanf("%d", &r);
            const int n_tail = cmoe::tail_items(n, slots, tail, 16);
            std::vector<int> codes;
            for (int i = 0; i < n - n_tail; ++i) codes.push_back(4 * i);
            for (int i = n - n_tail; i < n; ++i) {
                if (cmoe::tail_splits(rows[i], bm)) {
                    codes.push_back(4 * i + 1);
                    codes.push_back(4 * i + 2);
                } else {
                    codes.push_back(4 * i);
                }
            }
            for (int c : codes) {
                int rb = 0, r = rows[c >> 2];
                cmoe::tail_part(c & 3, bm, rb, r);
                std::printf("%d %d %d %d\n", c >> 2, c & 3, rb, r);
            }
            std::printf("END\n");
            continue;
        }
        int E, fw, n_tiles, slots;
        if (std::scanf("%d %d %d %d", &E, &fw, &n_tiles, &slots) != 4) return 1;
        std::vector<int> run(E), nt(E), off(E), toff(E);
        for (auto& r : run) std::scanf("%d", &r);
        long long tiles = 0, pairs = 0;
        for (int e = 0; e < E; ++e) {
            nt[e] = (run[e] + 255) / 256;
            off[e] = (int)pairs;
            toff[e] = (int)tiles;
            tiles += nt[e];
            pairs += run[e];
        }
        int b[9] = {0, 0, 0, 0, 0, 0, 0, 0, 0};
        for (int e = 0; e < E; ++e)
            cmoe::split_expert(fw, n_tiles, 256, run[e], nt[e], toff[e], off[e], 32LL * fw * tiles + pairs, b);
        cmoe::split_clamp(b, (int)tiles * n_tiles, slots);
        for (int k = 0; k < 9; ++k) std::printf("%d%c", b[k], k == 8 ? '\n' : ' ');
    }
    return 0;
}
