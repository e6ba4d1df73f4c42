// CPU check of the persistent MFMA conv kernel's walk (kokoro-rust_amd/csrc/kk_walk.h, the code the
// kernel runs): for every layer and grid shape in a sweep, simulates every block's consumer and
// producer iteration and counts violations of
//   - weight-fragment bounds: every A load (M offset, tap, 16-channel group) inside the packed
//     weights [k][cin_pad / 16][m_pad] (the kernel loads groups c16 .. c16 + 3 of a step);
//   - coverage: every (tile, M-block) unit's epilogue runs exactly once over all blocks;
//   - the unit count: a block runs walk_n_units units and never steps past its last one;
//   - producer order: the slabs the producers convert are the consumers' slabs, step for step, and
//     every slab they load belongs to a unit that exists.
// With --plant, the next-tap rule has a planted mistake (the unit's last slab also moves to "the
// next slab") and the check must report violations.  Prints "violations N".
#include "kk_walk.h"

#include <cstdio>
#include <cstring>
#include <vector>

using namespace kk;

static bool plant = false;

static void next_a(int kk, int k, int sl, int nsl, bool has_next, int m0, int nm0, int& a, int& t, int& c) {
    walk_next_a(kk, k, sl, nsl, has_next, m0, nm0, a, t, c);
    if (plant && kk + 1 == k && sl + 1 == nsl) c = 4 * sl + 4;
}

struct Step {
    int tile, m0, sl;
    bool operator!=(const Step& o) const { return tile != o.tile || m0 != o.m0 || sl != o.sl; }
};

static long check(int64_t count, int mblocks, int k, int nsl, int64_t grid) {
    const int bm = 64;
    const int m_pad = mblocks * bm, n16 = 4 * nsl;
    long bad = 0;
    std::vector<int> seen((size_t)count * mblocks, 0);
    for (int b = 0; b < grid; b++) {
        const int n_units = walk_n_units(b, (int)grid, mblocks, count);
        const int G = n_units * nsl;
        if (G == 0) continue;
        auto chk = [&](int m0, int kk, int c16) {
            if (m0 < 0 || m0 + bm > m_pad || m0 % bm || kk < 0 || kk >= k || c16 < 0 || c16 + 3 >= n16) bad++;
        };
        // consumer
        std::vector<Step> steps;
        int U = b, sl = 0, ct = 0, cm = 0, nt = 0, nm = 0;
        if (!walk_unit(U, mblocks, bm, count, ct, cm)) {
            bad++;
            continue;
        }
        bool has_next = walk_unit(U + (int)grid, mblocks, bm, count, nt, nm);
        chk(cm, 0, 0);
        int units_done = 0;
        for (int g = 0; g < G; g++) {
            steps.push_back(Step{ct, cm, sl});
            for (int kk = 0; kk < k; kk++) {
                int a, t, c;
                next_a(kk, k, sl, nsl, has_next, cm, nm, a, t, c);
                chk(a, t, c);
            }
            if (sl + 1 == nsl) {
                if (ct >= 0 && ct < count) seen[(size_t)ct * mblocks + cm / bm]++;
                else bad++;
                units_done++;
                if (!has_next && g + 1 < G) bad++;  // would step past its last unit
                sl = 0;
                U += (int)grid;
                ct = nt, cm = nm;
                has_next = walk_unit(U + (int)grid, mblocks, bm, count, nt, nm);
            } else {
                sl++;
            }
        }
        if (units_done != n_units) bad++;
        // producers: the kernel's two-slot schedule
        int lU = b, ls = 0, cU = b, cs = 0, lt = 0, lm = 0, vt = 0, vm = 0;
        walk_unit(lU, mblocks, bm, count, lt, lm);
        vt = lt, vm = lm;
        std::vector<Step> loads, converts;
        auto adv_l = [&]() {
            if (++ls == nsl) {
                int t, m;
                ls = 0;
                lU += (int)grid;
                if (walk_unit(lU, mblocks, bm, count, t, m)) lt = t, lm = m;
            }
        };
        auto adv_c = [&]() {
            if (++cs == nsl) {
                cs = 0;
                cU += (int)grid;
                walk_unit(cU, mblocks, bm, count, vt, vm);
            }
        };
        auto load = [&]() { loads.push_back(Step{lt, lm, ls}); };
        auto convert = [&]() { converts.push_back(Step{vt, vm, cs}); };
        load(), adv_l(), load(), adv_l(), convert(), adv_c(), load(), adv_l();
        for (int g = 0; g < G; g += 2) {
            if (g + 1 < G) convert(), adv_c();
            load(), adv_l();
            if (g + 1 >= G) break;
            if (g + 2 < G) convert(), adv_c();
            load(), adv_l();
        }
        if (converts.size() != steps.size()) bad++;
        for (size_t i = 0; i < converts.size() && i < steps.size(); i++)
            if (converts[i] != steps[i]) bad++;
        for (size_t i = 0; i < loads.size(); i++) {
            const Step& s = loads[i];
            if (s.tile < 0 || s.tile >= count || s.m0 < 0 || s.m0 + bm > m_pad) bad++;
            if (i < steps.size() && s != steps[i]) bad++;
        }
    }
    for (int v : seen)
        if (v != 1) bad++;
    return bad;
}

// convt_cols against the per-column rule it replaces: tile column col writes output row o =
// stride (n0 + col) + ph - pad (o + 1 with the reflection pad) when col < nv, the lane's channels
// exist and os <= o < os + ol; written rows relative to ubase are non-negative; the reflected
// column is the one writing row os + 1 (reflection pad) and then ubase = os.
static long check_convt_cols() {
    long bad = 0;
    uint64_t st64 = 0x2545F4914F6CDD1Dull;
    auto rnd = [&](int64_t n) { st64 = st64 * 6364136223846793005ull + 1442695040888963407ull; return (int64_t)((st64 >> 33) % (uint64_t)n); };
    for (int it = 0; it < 200000; it++) {
        const int stride = rnd(2) ? 6 : 10, pad = (int)(2 + rnd(6)), ph = (int)rnd(stride), nv = (int)rnd(129);
        const bool reflect = rnd(2), mok = rnd(10) != 0;
        const int64_t n0 = rnd(100000);
        int64_t os = stride * n0 - pad + rnd(41) - 20;
        if (os < 0) os = 0;
        const int64_t ol = 1 + rnd(3000);
        const kk::ConvTCols c = kk::convt_cols(n0, nv, stride, pad, ph, os, ol, reflect, mok);
        if (c.ubase != (os > stride * n0 - pad - 1 ? os : stride * n0 - pad - 1)) bad++;
        for (int col = 0; col < 128; col++) {
            const int64_t o = (int64_t)stride * (n0 + col) + ph - pad;
            const bool ok = col < nv && mok && o >= os && o < os + ol;
            if (ok != (col >= c.lo && col < c.hi)) bad++;
            if (ok) {
                const int64_t rel = (reflect ? o + 1 : o) - c.ubase;
                if (rel < 0 || rel != (int64_t)c.rel0 + (int64_t)stride * col) bad++;
            }
            if (reflect && (ok && o == os + 1) != (col == c.refl)) bad++;
        }
        if (c.refl >= 0 && c.ubase != os) bad++;
    }
    return bad;
}

int main(int argc, char** argv) {
    plant = argc > 1 && std::strcmp(argv[1], "--plant") == 0;
    if (!plant) {
        const long bc = check_convt_cols();
        std::printf("convt columns violations %ld\n", bc);
        if (bc) return 1;
    }
    const int64_t counts[] = {1, 2, 7, 8, 9, 17, 64, 257, 1000};
    const int mbs[] = {1, 2, 3, 4};
    const int ks[] = {1, 2, 3, 5, 7, 11, 12};
    const int nsls[] = {1, 2, 4, 9, 18, 32};
    const int cus[] = {1, 8, 80, 256};
    long total = 0, launches = 0;
    for (int64_t c : counts)
        for (int mb : mbs)
            for (int k : ks)
                for (int nsl : nsls)
                    for (int cu : cus) {
                        const int64_t grid = walk_grid(c, mb, cu);
                        const long v = check(c, mb, k, nsl, grid);
                        if (v && total < 5 * 1000000L)
                            std::printf("count %lld mblocks %d k %d nsl %d n_cu %d grid %lld: %ld\n", (long long)c, mb, k,
                                        nsl, cu, (long long)grid, v);
                        total += v;
                        launches++;
                    }
    std::printf("launches %ld violations %ld\n", launches, total);
    return 0;
}
