// kk_walk.h -- the persistent MFMA conv kernel's walk over its work: (tile, M-block) units, the
// 64-channel slabs of a unit and the taps of a slab.  These __host__ __device__ functions are the
// only copy of that indexing: conv_mfma_kernel (kk_conv.hip) runs them on the GPU and
// tests/conv_walk_check.hip runs them on the CPU, where it checks every weight-fragment address and
// the units each block visits for every grid and layer shape the engine launches.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace kk {

// Unit U = g * 8 * mblocks + w * 8 + x is M-block w of tile g * 8 + x; false past the last tile.
// Blocks of one tile's M-blocks keep the same x, so they land on the same XCD (workgroup slots go
// to the 8 XCDs round-robin).
__host__ __device__ inline bool walk_unit(int U, int mblocks, int bm, int64_t count, int& tile, int& m0) {
    const int grp = 8 * mblocks;
    const int g = U / grp, within = U - g * grp;
    tile = g * 8 + (within & 7);
    if (tile >= count) return false;
    m0 = (within >> 3) * bm;
    return true;
}

// The number of units block b runs: b, b + grid, b + 2 grid, ... (grid a multiple of 8 * mblocks,
// so b keeps its M-block and x) while the tile exists.
__host__ __device__ inline int walk_n_units(int b, int grid, int mblocks, int64_t count) {
    const int grp = 8 * mblocks;
    const int g0 = b / grp, x = (b - g0 * grp) & 7;
    const int gmax = ((int)count - 1 - x) >> 3;  // last group whose tile g * 8 + x exists
    return (count > x && gmax >= g0) ? (gmax - g0) / (grid / grp) + 1 : 0;
}

// The weight fragments loaded after tap kk of slab sl (a full tap of lead time): the next tap of
// this slab, tap 0 of the next slab, tap 0 of the next unit (M-block next_m0), or -- after the
// block's very last tap -- tap 0 of this slab again (a harmless load that keeps the number of
// loads in flight static).  Fragment group c16 + kc (kc < 4) of tap n_kk at M offset n_m0.
__host__ __device__ inline void walk_next_a(int kk, int k, int sl, int nsl, bool has_next, int m0, int next_m0,
                                            int& n_m0, int& n_kk, int& n_c16) {
    n_m0 = m0, n_kk = kk + 1, n_c16 = 4 * sl;
    if (kk + 1 == k) {
        n_kk = 0;
        if (sl + 1 != nsl)
            n_c16 = 4 * sl + 4;
        else if (has_next)
            n_m0 = next_m0, n_c16 = 0;
    }
}

// The grid of a launch: at most one block per CU, a multiple of 8 * mblocks, no more blocks than
// padded units.
inline int64_t walk_grid(int64_t count, int mblocks, int n_cu) {
    const int64_t grp = 8 * (int64_t)mblocks;
    const int64_t units = (count + 7) / 8 * grp;
    const int64_t fit = (n_cu / grp > 1 ? n_cu / grp : 1) * grp;
    return units < fit ? units : fit;
}

}  // namespace kk
