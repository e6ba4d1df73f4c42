/* Every finite float x: the conv epilogue's division by 3 (q = x RN(1/3); r = fma(-3, q, x);
 * r != 0 ? fma(r, RN(1/3), q) : q -- the stage mean's div3 in kokoro-rust_amd/csrc/kk_conv.hip)
 * against the correctly rounded x / 3.0f.  Prints the number of inputs checked and of mismatches
 * (bit patterns; a zero must keep its sign). */
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
        const float r = fmaf(-3.0f, q, x);
        const float q1 = r != 0.0f ? fmaf(r, third, q) : q;
        n++;
        if (u_of(q1) != u_of(x / 3.0f)) bad++;
    }
    printf("%lld %lld\n", n, bad);
    return 0;
}
