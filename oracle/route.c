/*
 * CPU restatement of the routing step of the MoE-experts path — TEST INFRASTRUCTURE ONLY
 * (loaded by tests/ through ctypes; never linked into the product library).
 *
 * Restates, as plain sequential C:
 *   count_tokens_kernel  (src/kops/cohere2_moe_experts/csrc/cohere2_moe_experts.cu:29-37):
 *       per-expert histogram, ids outside [0, E) skipped;
 *   offsets              (.cu:267-270): exclusive prefix sum, offsets[E] = valid pairs;
 *   build_perm_kernel    (.cu:40-55): pairs scattered to their expert's segment — here in the
 *       op_eager order (slot k, then token t, within an expert; transformers
 *       modeling_cohere2_moe.py:122-130) instead of the reference's atomic order;
 *   the M-tile list of the grouped GEMMs: ceil(count_e / tile_m) tiles per expert.
 * Pinned against the numpy closed form (argsort/bincount) and the golden torch.where order in
 * tests/test_oracle.py.
 */
#include <stdint.h>
#include <stdlib.h>

int oracle_route(const int32_t* idx, int T, int K, int E, int tile_m, int32_t* offsets, int32_t* sorted_pairs,
                 int32_t* tile_offsets, int32_t* tile_expert, int32_t* meta) {
    if (T < 0 || K <= 0 || E <= 0 || tile_m <= 0) return 1;
    int64_t* cursor = (int64_t*)calloc((size_t)E, sizeof(int64_t));
    if (!cursor) return 2;
    /* histogram */
    for (int64_t p = 0; p < (int64_t)T * K; ++p) {
        int32_t e = idx[p];
        if (e >= 0 && e < E) cursor[e]++;
    }
    /* exclusive scans: pair offsets and tile offsets */
    int64_t run = 0, trun = 0;
    for (int e = 0; e < E; ++e) {
        int64_t c = cursor[e];
        int64_t nt = (c + tile_m - 1) / tile_m;
        offsets[e] = (int32_t)run;
        tile_offsets[e] = (int32_t)trun;
        for (int64_t j = 0; j < nt; ++j) tile_expert[trun + j] = e;
        cursor[e] = run;
        run += c;
        trun += nt;
    }
    offsets[E] = (int32_t)run;
    tile_offsets[E] = (int32_t)trun;
    meta[0] = (int32_t)trun;
    meta[1] = (int32_t)run;
    /* stable scatter in slot-major visiting order */
    for (int k = 0; k < K; ++k)
        for (int t = 0; t < T; ++t) {
            int32_t e = idx[(int64_t)t * K + k];
            if (e < 0 || e >= E) continue;
            sorted_pairs[cursor[e]++] = t * K + k;
        }
    free(cursor);
    return 0;
}
