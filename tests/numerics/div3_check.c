/* Every finite float x: the conv epilogue's division by 3 (q = x RN(1/3); n = fma(3, q, -x);
 * fma(-n, RN(1/3), q) -- the stage mean's div3 in kokoro-rust_amd/csrc/kk_conv.hip) against the
 * correctly rounded x / 3.0f.  Prints the number of inputs checked and of mismatches (bit patterns;
 * a zero must keep its sign).  The empty asm keeps n as computed: a compiler that folds -fma(3, q, -x)
 * into fma(-3, q, x) would change the sign of a zero remainder (the GPU compiler does not fold it
 * without no-signed-zeros). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t u_of(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

int main(void) {
    const float third = 1.0f / 3.0f;
    long long bad = 0, n = 0;
#pragma omp parallel for reduction(+ : bad, n) schedule(static)
    for (long long i = 0; i < (1LL << 32); i++) {
        const float x = f_of((uint32_t)i);
        if (!isfinite(x)) continue;
        const float q = x * third;
        float nr = fmaf(3.0f, q, -x);
        __asm__ volatile("" : "+x"(nr));
        const float q1 = fmaf(-nr, third, q);
        n++;
        if (u_of(q1) != u_of(x / 3.0f)) bad++;
    }
    printf("%lld %lld\n", n, bad);
    /* The same epilogue's leaky ReLU, max(x, slope x), against x < 0 ? slope x : x for every float
     * x (NaNs included: both give a NaN) at the generator's slopes and near the ends of (0, 1]
     * (slope 0 would differ at x = -inf: 0 (-inf) is a NaN, which max drops). */
    const float slopes[5] = {0.1f, 0.01f, 0.2f, 1e-30f, 1.0f};
    long long lbad = 0, ln = 0;
    for (int si = 0; si < 5; si++) {
        const float s = slopes[si];
#pragma omp parallel for reduction(+ : lbad, ln) schedule(static)
        for (long long i = 0; i < (1LL << 32); i++) {
            const float x = f_of((uint32_t)i);
            const float a = fmaxf(x, x * s), b = x < 0.0f ? x * s : x;
            ln++;
            if (isnan(a) ? !isnan(b) : u_of(a) != u_of(b)) lbad++;
        }
    }
    printf("%lld %lld\n", ln, lbad);
    return 0;
}
