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

// A ConvT unit's columns (EPI_CONVT / EPI_CONVT_REFLECT): tile column col (of nv valid, from input
// column n0) is output row o = stride (n0 + col) + ph - pad, written -- as row o, or o + 1 with the
// reflection pad -- when o lies in the item's output span [os, os + ol) (ol without the reflected
// row); rows are addressed from ubase = max(os, stride n0 - pad - 1).  The columns written are
// [lo, hi); column col's row relative to ubase is rel0 + stride col; refl is the column whose row
// is os + 1 with the reflection pad (it also fills row os, then = ubase), or -1.  mok: this lane's
// output channels exist (else no column is written).
struct ConvTCols {
    int lo, hi, rel0, refl;
    int64_t ubase;
};
__host__ __device__ inline ConvTCols convt_cols(int64_t n0, int nv, int stride, int pad, int ph, int64_t os, int64_t ol,
                                                bool reflect, bool mok) {
    const int64_t st = stride, o0 = st * n0 + ph - pad;  // the row of column 0
    auto ceil_div = [](int64_t a, int64_t b) { return a >= 0 ? (a + b - 1) / b : -((-a) / b); };  // b > 0
    ConvTCols c;
    c.ubase = os > st * n0 - pad - 1 ? os : st * n0 - pad - 1;
    int64_t lo = ceil_div(os - o0, st), hi = ceil_div(os + ol - o0, st);
    lo = lo > 0 ? lo : 0;
    hi = hi < nv ? hi : nv;
    c.lo = (int)lo;
    c.hi = mok && hi > lo ? (int)hi : (int)lo;
    c.rel0 = (int)(o0 + (reflect ? 1 : 0) - c.ubase);
    c.refl = -1;
    if (reflect) {
        const int64_t a = os + 1 - o0;
        if (a >= 0 && a % st == 0 && a / st >= c.lo && a / st < c.hi) c.refl = (int)(a / st);
    }
    return c;
}

}  // namespace kk
