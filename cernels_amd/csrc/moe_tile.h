// Tile helpers shared by the prefill GEMMs: LDS tile swizzle, direct global->LDS copies, waits,
// and the work-item decode of the grouped-GEMM schedule.
#pragma once

#include "moe_common.h"
#include "moe_split.h"

namespace cmoe {

constexpr int kBK = 64;  // K elements per LDS stage row (128 bytes of bf16)

// LDS tile layout: row-major 128-byte rows (64 bf16 of K) of eight 16-byte chunks; chunk c of row r
// sits at chunk c ^ ((r >> 1) & 7). gfx950 LDS serves 256 bytes (64 banks) per clock, i.e. 16
// lanes of a 16-byte read; the swizzle puts the same chunk of any 16 consecutive rows (two rows per
// 256-byte bank line) on distinct banks, so MFMA fragment reads (consecutive rows, one chunk) are
// conflict-free.
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int lds_off(int row, int chunk) { return row * (kBK * 2) + ((chunk ^ swz(row)) << 4); }

// ---- direct global -> LDS copies (gfx950 global_load_lds_dwordx4) ---------------------------------
// One instruction moves 16 bytes per lane into LDS at M0 + 16*lane (1 KB per wave). The load is
// issued from inline assembly so the compiler does not wait for every outstanding copy at each
// barrier; completion is awaited explicitly before the barrier that publishes a stage. The compiler
// does not count these copies in its own vmcnt bookkeeping.
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
    return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const unsigned char*)(p));
}
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// vmcnt(0) through the builtin, so that the compiler also knows every load it issued has landed
// and inserts no later waits for them.
__device__ __forceinline__ void wait_all_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Grouped-GEMM work item: items are (expert, N-tile, M-tile) in expert-major order with M fastest,
// numbered over the M-tile list the route kernel wrote (tile_expert, tile_offsets, offsets); an expert's
// M-tiles split its rows as tile_rows does.
struct WorkItem {
    int e, n_idx, row_begin, rows;
};

__device__ __forceinline__ WorkItem decode_item(int it, int n_tiles, const int32_t* __restrict__ tile_expert,
                                                const int32_t* __restrict__ tile_offsets,
                                                const int32_t* __restrict__ offsets) {
    WorkItem w;
    w.e = tile_expert[it / n_tiles];
    const int t0 = tile_offsets[w.e], nt_e = tile_offsets[w.e + 1] - t0;
    const int local = it - t0 * n_tiles;
    w.n_idx = local / nt_e;
    const int m_idx = local - w.n_idx * nt_e;
    const int seg0 = offsets[w.e];
    tile_rows(m_idx, nt_e, offsets[w.e + 1] - seg0, w.row_begin, w.rows);
    w.row_begin += seg0;
    return w;
}

}  // namespace cmoe
