/*
 * kk_oracle.c -- CPU fp32 restatement of kokoro-rust's decoder + iSTFTNet generator path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): see kk_oracle.h.
 *
 * Each function cites the reference file:line whose semantics it restates.  The reference has no
 * CPU forward path of its own (docs/USAGE.md:100), so this file is written from the CUDA kernels'
 * arithmetic (kernels/kokoro.cu) and the host op order (src/gpu_batch.rs).
 *
 * Build: oracle/build_oracle.sh (gcc -O3 -fopenmp -ffp-contract=off).
 */
#include "kk_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define PI_F 3.14159274101257324f /* (float)M_PI, kernels/kokoro.cu:9 */
#define STYLE_DIM 128             /* src/model.rs:12 */
#define HARMONICS 9               /* src/vocoder.rs:10 */
#define UPSAMPLE 300              /* src/vocoder.rs:11 */

static int g_bf16 = 0;      /* operand format: 0 off, 1 bf16, 2 fp16 */
static int g_groups = 0xff; /* layer groups the emulation applies to (KO_GROUP_*) */
static int g_fp16 = 0;      /* of those, the groups whose operands round to fp16 instead */
void ko_set_bf16_emulation(int on) { g_bf16 = on ? 1 : 0; g_groups = 0xff; g_fp16 = 0; }
int ko_get_bf16_emulation(void) { return g_bf16; }
void ko_set_operand_emulation(int fmt, int groups) { g_bf16 = fmt; g_groups = groups; g_fp16 = fmt == 2 ? groups : 0; }
/* Mixed operand formats: the groups in fp16_groups round to fp16, the other groups in `groups` to
 * bf16 (the HIP path's decoder convolutions run on fp16 operands). */
void ko_set_operand_formats(int groups, int fp16_groups) {
    g_bf16 = groups ? 1 : 0;
    g_groups = groups;
    g_fp16 = fp16_groups & groups;
}
void ko_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
}

/* Round-to-nearest-even to bf16, returned as the f32 value it represents (NaN kept quiet). */
float ko_bf16_round(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) u |= 0x00400000u;
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    float r;
    memcpy(&r, &u, 4);
    return r;
}

/* Round-to-nearest-even to IEEE binary16, returned as f32 (subnormals on the 2^-24 grid; values
 * beyond the binary16 range become infinities). */
float ko_fp16_round(float x) {
    float ax = fabsf(x);
    if (!(ax < 65520.0f)) return ax != ax ? x : copysignf(INFINITY, x);
    if (ax < 6.103515625e-05f) return nearbyintf(x * 16777216.0f) * (1.0f / 16777216.0f);
    uint32_t u;
    memcpy(&u, &x, 4);
    u += 0x0fffu + ((u >> 13) & 1u);
    u &= 0xffffe000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

static float* round_copy(const float* x, size_t n, int group) {
    float* r = (float*)malloc(n * sizeof(float));
    if (g_bf16 == 2 || (g_fp16 & group))
        for (size_t i = 0; i < n; i++) r[i] = ko_fp16_round(x[i]);
    else
        for (size_t i = 0; i < n; i++) r[i] = ko_bf16_round(x[i]);
    return r;
}

/* ================================================================ hydration */

/* weight_norm (src/ops.rs:9-23): per row r, norm = sqrt(sum of v^2 in f64) rounded to f32,
 * scale = g[r] / norm in f32, w = v * scale in f32. */
void ko_weight_norm(const float* v, const float* g, int64_t rows, int64_t per_row, float* w) {
    for (int64_t r = 0; r < rows; r++) {
        double ss = 0.0;
        for (int64_t j = 0; j < per_row; j++) ss += (double)v[r * per_row + j] * (double)v[r * per_row + j];
        const float nrm = (float)sqrt(ss);
        const float scale = g[r] / nrm;
        for (int64_t j = 0; j < per_row; j++) w[r * per_row + j] = v[r * per_row + j] * scale;
    }
}

/* ================================================================ layout (a1-a3) */

/* src/gpu_batch.rs:250-258: a[b] = running sum of (N_j + GAP_N). */
int ko_layout_frames(const int64_t* nfs, int nb, int gap, int64_t* a_out, int64_t* ln_out) {
    if (nb <= 0 || gap < 0) return -1;
    int64_t ln = 0;
    for (int b = 0; b < nb; b++) {
        if (nfs[b] < 0) return -2;
        a_out[b] = ln;
        ln += nfs[b] + gap;
    }
    *ln_out = ln;
    return 0;
}

/* src/gpu_batch.rs:42-54 (Dom::new): overflow and overlap are errors. */
int ko_layout_col_item(int64_t l, const int64_t* start, const int64_t* len, int nb, int32_t* col_item) {
    for (int64_t t = 0; t < l; t++) col_item[t] = -1;
    for (int b = 0; b < nb; b++) {
        if (start[b] < 0 || len[b] < 0 || start[b] + len[b] > l) return -1;
        for (int64_t t = start[b]; t < start[b] + len[b]; t++) {
            if (col_item[t] >= 0) return -2;
            col_item[t] = b;
        }
    }
    return 0;
}

/* src/gpu_batch.rs:265-276: frames of item b in token order, token tok repeated dur[tok] times. */
int ko_layout_src_row(const int64_t* const* dur, const int64_t* ntok, int nb, const int64_t* tstart,
                      const int64_t* a, int64_t ln, int32_t* src_row) {
    for (int64_t t = 0; t < ln; t++) src_row[t] = -1;
    for (int b = 0; b < nb; b++) {
        int64_t f = a[b];
        for (int64_t tok = 0; tok < ntok[b]; tok++) {
            for (int64_t r = 0; r < dur[b][tok]; r++) {
                if (f >= ln) return -1;
                src_row[f++] = (int32_t)(tstart[b] + tok);
            }
        }
    }
    return 0;
}

/* src/model.rs:90-99 with src/ops.rs:49-51 (sigmoid in f32, left-to-right f32 sum, ties to even). */
void ko_durations_from_logits(const float* logits, int t, float speed, int64_t* out) {
    for (int i = 0; i < t; i++) {
        float s = 0.0f;
        for (int j = 0; j < 50; j++) {
            float v = logits[i * 50 + j];
            s = s + 1.0f / (1.0f + expf(-v));
        }
        float d = nearbyintf(s / speed); /* default rounding mode: to nearest, ties to even */
        /* `d as i64` saturates in Rust (src/model.rs:96): NaN -> 0, at or past 2^63 -> i64::MAX */
        int64_t di = isnan(d) ? 0 : d >= 9.223372036854775808e18f ? INT64_MAX : (int64_t)d;
        out[i] = di < 1 ? 1 : di;
    }
}

/* ================================================================ primitives */

/* Conv1d (src/ops.rs:4-6 output length; kernels/kokoro.cu:517-617 / 660-774 semantics):
 * y = bias, then for each tap k and input channel ci ascending: y += w * x (zero outside [0,T)). */
static void conv1d_raw(const float* x, int cin, int t, const float* w, const float* b, int cout, int k, int stride,
                       int pad, int dil, float* y, int tout) {
#pragma omp parallel for schedule(static)
    for (int co = 0; co < cout; co++) {
        float* yr = y + (size_t)co * tout;
        float bias = b ? b[co] : 0.0f;
        for (int o = 0; o < tout; o++) yr[o] = bias;
        for (int kk = 0; kk < k; kk++) {
            int off = kk * dil - pad; /* input index = o*stride + off */
            /* valid o: 0 <= o*stride + off < t */
            int o_lo = 0, o_hi = tout - 1;
            if (off < 0) o_lo = (-off + stride - 1) / stride;
            {
                int lim = t - 1 - off; /* o*stride <= lim */
                if (lim < 0) continue;
                int oh = lim / stride;
                if (oh < o_hi) o_hi = oh;
            }
            if (o_lo > o_hi) continue;
            for (int ci = 0; ci < cin; ci++) {
                float wv = w[((size_t)co * cin + ci) * k + kk];
                const float* xr = x + (size_t)ci * t + off;
                if (stride == 1) {
                    for (int o = o_lo; o <= o_hi; o++) yr[o] = yr[o] + wv * xr[o];
                } else {
                    for (int o = o_lo; o <= o_hi; o++) yr[o] = yr[o] + wv * xr[(size_t)o * stride];
                }
            }
        }
    }
}

int ko_conv1d(const float* x, int cin, int t, const float* w, const float* b, int cout, int k, int stride, int pad,
              int dil, float* y, int tout) {
    if (stride < 1 || dil < 1 || k < 1) return -1;
    int expect = (t + 2 * pad - dil * (k - 1) - 1) / stride + 1;
    if (t + 2 * pad - dil * (k - 1) - 1 < 0 || expect != tout) return -2;
    conv1d_raw(x, cin, t, w, b, cout, k, stride, pad, dil, y, tout);
    return 0;
}

/* ConvTranspose1d (kernels/kokoro.cu:169-185 + src/gpu.rs:527-537): Z[co,k,i] = sum_ci W[ci][co][k] x[ci][i]
 * (ci ascending), then y[co][o] = b[co] + sum over k ascending with (o+p-k) = s*i, 0 <= i < Tin. */
int ko_conv_transpose1d(const float* x, int cin, int t, const float* w, const float* b, int cout, int k, int stride,
                        int pad, float* y, int tout) {
    if ((t - 1) * stride + k - 2 * pad != tout) return -2;
    float* xt = (float*)malloc((size_t)t * cin * sizeof(float));
    for (int ci = 0; ci < cin; ci++)
        for (int i = 0; i < t; i++) xt[(size_t)i * cin + ci] = x[(size_t)ci * t + i];
#pragma omp parallel
    {
        float* wt = (float*)malloc((size_t)k * cin * sizeof(float));
#pragma omp for schedule(static)
        for (int co = 0; co < cout; co++) {
            for (int kk = 0; kk < k; kk++)
                for (int ci = 0; ci < cin; ci++) wt[(size_t)kk * cin + ci] = w[((size_t)ci * cout + co) * k + kk];
            for (int o = 0; o < tout; o++) {
                float acc = b[co];
                for (int kk = 0; kk < k; kk++) {
                    int num = o + pad - kk;
                    if (num < 0 || num % stride != 0) continue;
                    int i = num / stride;
                    if (i >= t) continue;
                    const float* xr = xt + (size_t)i * cin;
                    const float* wr = wt + (size_t)kk * cin;
                    float z = 0.0f;
                    for (int ci = 0; ci < cin; ci++) z = z + wr[ci] * xr[ci];
                    acc = acc + z;
                }
                y[(size_t)co * tout + o] = acc;
            }
        }
        free(wt);
    }
    free(xt);
    return 0;
}

/* chan_stats_seg (kernels/kokoro.cu:779-810): values shifted by the span's first element, sums in
 * double, var = E[d^2] - E[d]^2 clamped at 0, mean = shift + E[d], rstd = 1/sqrtf((float)var + eps). */
void ko_chan_stats(const float* x, int c, int t, float* mean, float* rstd) {
#pragma omp parallel for schedule(static)
    for (int ch = 0; ch < c; ch++) {
        const float* row = x + (size_t)ch * t;
        float shift = t > 0 ? row[0] : 0.0f;
        double s = 0.0, s2 = 0.0;
        for (int i = 0; i < t; i++) {
            float v = row[i] - shift;
            s += (double)v;
            s2 += (double)v * (double)v;
        }
        double d = s / (double)t;
        double var = s2 / (double)t - d * d;
        if (var < 0.0) var = 0.0;
        mean[ch] = (float)((double)shift + d);
        rstd[ch] = 1.0f / sqrtf((float)var + 1e-5f);
    }
}

/* GLinear in adain_stats (src/gpu.rs:281-301, src/gpu_batch.rs:84): gb = W s + b, f64 accumulation. */
void ko_style_fc(const float* fc_w, const float* fc_b, int c2, const float* s, float* gb) {
    for (int j = 0; j < c2; j++) {
        double acc = 0.0;
        for (int i = 0; i < STYLE_DIM; i++) acc += (double)fc_w[(size_t)j * STYLE_DIM + i] * (double)s[i];
        gb[j] = (float)(acc + (double)fc_b[j]);
    }
}

/* adain_apply_seg (kernels/kokoro.cu:318-334) and the Snake prologue (kernels/kokoro.cu:702-714). */
void ko_adain_apply(const float* x, int c, int t, const float* mean, const float* rstd, const float* nw,
                    const float* nb, const float* gb, int mode, float slope, const float* alpha, float* y) {
#pragma omp parallel for schedule(static)
    for (int ch = 0; ch < c; ch++) {
        float g1 = 1.0f + gb[ch];
        float be = gb[c + ch];
        float a = mode == 1 ? alpha[ch] : 0.0f;
        float inv = mode == 1 ? 1.0f / a : 0.0f;
        for (int i = 0; i < t; i++) {
            float v = (x[(size_t)ch * t + i] - mean[ch]) * rstd[ch];
            v = g1 * (v * nw[ch] + nb[ch]) + be;
            if (mode == 1) {
                float sn = sinf(a * v);
                v = v + inv * (sn * sn);
            } else if (v < 0.0f) {
                v = v * slope;
            }
            y[(size_t)ch * t + i] = v;
        }
    }
}

/* splitmix_at (src/vocoder.rs:22-27): output number ctr of the splitmix64 stream starting at seed. */
uint64_t ko_splitmix_at(uint64_t seed, uint64_t ctr) {
    uint64_t x = seed + (ctr + 1ull) * 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

/* RngNoise::rand_ini (src/vocoder.rs:34-40). */
void ko_rand_ini(uint64_t seed, float* out9) {
    for (int h = 0; h < HARMONICS; h++) out9[h] = (float)(ko_splitmix_at(seed, (uint64_t)h) >> 40) * (1.0f / 16777216.0f);
}

/* gen_noise (kernels/kokoro.cu:291-302): pair i from splitmix_at(seed, 1024 + i), f32 Box-Muller. */
void ko_gen_noise(uint64_t seed, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (n + 1) / 2; i++) {
        uint64_t x = ko_splitmix_at(seed, 1024ull + (uint64_t)i);
        float u1 = (float)((x >> 40) + 1ull) * (1.0f / 16777216.0f);
        float u2 = (float)((x >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
        float r = sqrtf(-2.0f * logf(u1));
        float th = 6.2831855f * u2;
        out[2 * i] = r * cosf(th);
        if (2 * i + 1 < n) out[2 * i + 1] = r * sinf(th);
    }
}

/* torch.remainder(a, 1) (kernels/kokoro.cu:190-194). */
static float remainder1(float a) {
    float m = fmodf(a, 1.0f);
    if (m != 0.0f && m < 0.0f) m = m + 1.0f;
    return m;
}

/* sine_rad (kernels/kokoro.cu:197-204). */
static float sine_rad(const float* f0c, int l, float near_scale, int t, int h, const float* rand_ini) {
    int src = (int)floorf((float)t * near_scale);
    if (src > l - 1) src = l - 1;
    float r = remainder1(f0c[src] * (float)(h + 1) / 24000.0f);
    if (t == 0 && h > 0) r = r + rand_ini[h];
    return r;
}

/* SineGen: sine_phase_pre + sine_har_source (kernels/kokoro.cu:206-254; src/gpu_batch.rs:323-350). */
int ko_sine_source(const float* f0c, int l, const float* rand_ini, const float* noise, const float* lw, float lb,
                   float* phase_pre_out, float* har) {
    if (l <= 0) return -1;
    int s = l * UPSAMPLE;
    const float near_scale = (float)(1.0 / (double)UPSAMPLE);
    const float down_scale = (float)(1.0 / (1.0 / (double)UPSAMPLE));
    const float up_scale = (float)(1.0 / (double)UPSAMPLE);
    int d_len = (int)floor((double)s * (1.0 / (double)UPSAMPLE));
    float* pp = (float*)malloc((size_t)HARMONICS * d_len * sizeof(float));
    for (int h = 0; h < HARMONICS; h++) {
        double acc = 0.0;
        for (int d = 0; d < d_len; d++) {
            float real = fmaf(down_scale, (float)d + 0.5f, -0.5f);
            if (real < 0.0f) real = 0.0f;
            int i0 = (int)floorf(real);
            if (i0 > s - 1) i0 = s - 1;
            float l1 = fminf(fmaxf(real - (float)i0, 0.0f), 1.0f);
            int i1 = i0 < s - 1 ? i0 + 1 : i0;
            float l0 = 1.0f - l1;
            float v = fmaf(sine_rad(f0c, l, near_scale, i0, h, rand_ini), l0,
                           sine_rad(f0c, l, near_scale, i1, h, rand_ini) * l1);
            acc += (double)v;
            pp[(size_t)h * d_len + d] = (((float)acc) * 2.0f * PI_F) * 300.0f;
        }
    }
#pragma omp parallel for schedule(static)
    for (int t = 0; t < s; t++) {
        int src = (int)floorf((float)t * near_scale);
        if (src > l - 1) src = l - 1;
        float f0 = f0c[src];
        float uv = f0 > 10.0f ? 1.0f : 0.0f;
        float noise_amp = uv * 0.003f + (1.0f - uv) * 0.1f / 3.0f;
        float real = fmaf(up_scale, (float)t + 0.5f, -0.5f);
        if (real < 0.0f) real = 0.0f;
        int i0 = (int)floorf(real);
        if (i0 > d_len - 1) i0 = d_len - 1;
        float l1 = fminf(fmaxf(real - (float)i0, 0.0f), 1.0f);
        int i1 = i0 < d_len - 1 ? i0 + 1 : i0;
        float l0 = 1.0f - l1;
        float acc = 0.0f;
        for (int h = 0; h < HARMONICS; h++) {
            float ph = fmaf(pp[(size_t)h * d_len + i0], l0, pp[(size_t)h * d_len + i1] * l1);
            float sine = sinf(ph) * 0.1f;
            float v = sine * uv + noise_amp * noise[(size_t)t * HARMONICS + h];
            acc = acc + lw[h] * v;
        }
        har[t] = tanhf(acc + lb);
    }
    if (phase_pre_out) memcpy(phase_pre_out, pp, (size_t)HARMONICS * d_len * sizeof(float));
    free(pp);
    return 0;
}

/* Twiddles and periodic Hann window (src/gpu.rs:93-101), computed in f64. */
static double g_cos[11][20], g_sin[11][20];
static float g_win[20];
static int g_tables = 0;
static void init_tables(void) {
    if (g_tables) return;
    for (int k = 0; k < 11; k++)
        for (int n = 0; n < 20; n++) {
            double a = 2.0 * M_PI * (double)((k * n) % 20) / 20.0;
            g_cos[k][n] = cos(a);
            g_sin[k][n] = sin(a);
        }
    for (int n = 0; n < 20; n++) g_win[n] = (float)(0.5 - 0.5 * cos(2.0 * M_PI * (double)n / 20.0));
    g_tables = 1;
}

/* stft20_ld (kernels/kokoro.cu:470-490): reflect pad 10, f64 DFT of the windowed frame,
 * Im forced to 0 at k = 0 and 10, outputs |X| and atan2(Im, Re) in f32. */
int ko_stft20(const float* x, int l, float* out, int f) {
    init_tables();
    if (l < 11 || f != 1 + l / 5) return -1;
#pragma omp parallel for schedule(static)
    for (int fr = 0; fr < f; fr++) {
        double buf[20];
        for (int n = 0; n < 20; n++) {
            int p = fr * 5 + n - 10;
            int src = p < 0 ? -p : (p >= l ? 2 * l - 2 - p : p);
            buf[n] = (double)(x[src] * g_win[n]);
        }
        for (int k = 0; k < 11; k++) {
            double re = 0.0, im = 0.0;
            for (int n = 0; n < 20; n++) {
                re += buf[n] * g_cos[k][n];
                im -= buf[n] * g_sin[k][n];
            }
            if (k == 0 || k == 10) im = 0.0;
            float rf = (float)re, imf = (float)im;
            out[(size_t)k * f + fr] = hypotf(rf, imf);
            out[(size_t)(11 + k) * f + fr] = atan2f(imf, rf);
        }
    }
    return 0;
}

/* istft_frames_ld + istft_ola (kernels/kokoro.cu:264-280, 492-508). */
int ko_istft20(const float* post, int f, float* audio) {
    init_tables();
    if (f < 2) return -1;
    double* fr = (double*)malloc((size_t)f * 20 * sizeof(double));
#pragma omp parallel for schedule(static)
    for (int q = 0; q < f; q++) {
        double re[11], im[11];
        for (int k = 0; k < 11; k++) {
            float m = expf(post[(size_t)k * f + q]);
            float p = sinf(post[(size_t)(11 + k) * f + q]);
            re[k] = (double)(m * cosf(p));
            im[k] = (double)(m * sinf(p));
        }
        for (int n = 0; n < 20; n++) {
            double v = re[0] + re[10] * ((n % 2 == 0) ? 1.0 : -1.0);
            for (int k = 1; k < 10; k++) v += 2.0 * (re[k] * g_cos[k][n] - im[k] * g_sin[k][n]);
            v = v / 20.0;
            fr[(size_t)q * 20 + n] = v * (double)g_win[n];
        }
    }
    int len = 5 * (f - 1);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < len; i++) {
        int j = i + 10;
        int f_lo = j - 19 > 0 ? (j - 19 + 4) / 5 : 0;
        int f_hi = j / 5;
        if (f_hi > f - 1) f_hi = f - 1;
        double acc = 0.0, env = 0.0;
        for (int q = f_lo; q <= f_hi; q++) {
            int n = j - 5 * q;
            acc += fr[(size_t)q * 20 + n];
            double w = (double)g_win[n];
            env += w * w;
        }
        audio[i] = (float)(acc / env);
    }
    free(fr);
    return 0;
}

/* ================================================================ model */

typedef struct {
    const float* w;
    const float* b;
    int cin, cout, k, stride, pad, dil;
    int mfma; /* KO_GROUP_* of a layer the HIP path runs on MFMA, 0 for fp32 layers */
} conv_t;
typedef struct {
    const float* w;
    const float* b;
    int cin, cout, k, stride, pad;
} convt_t;
typedef struct {
    const float *nw, *nb, *fw, *fb;
    int c;
} adain_t;
typedef struct {
    conv_t c1[3], c2[3];
    adain_t a1[3], a2[3];
    const float* al1[3];
    const float* al2[3];
    int c;
} snake_t;
typedef struct {
    conv_t conv1, conv2, conv1x1;
    int has_1x1;
    adain_t n1, n2;
    const float *pool_w, *pool_b;
    int din, dout, up;
} resblk_t;

struct ko_model {
    int n;
    char** names;
    float** data;
    int64_t* numel;
    resblk_t encode, decode[4];
    conv_t f0_conv, n_conv, asr_res;
    const float* l_w;
    float l_b;
    conv_t noise_convs[2];
    snake_t noise_res[2];
    convt_t ups[2];
    snake_t resblocks[6];
    conv_t conv_post;
};

static const float* find(const ko_model* m, const char* name, int64_t numel, char* err, size_t errlen) {
    for (int i = 0; i < m->n; i++) {
        if (strcmp(m->names[i], name) == 0) {
            if (m->numel[i] != numel) {
                snprintf(err, errlen, "tensor %s has %lld values, expected %lld", name, (long long)m->numel[i],
                         (long long)numel);
                return NULL;
            }
            return m->data[i];
        }
    }
    snprintf(err, errlen, "missing tensor %s", name);
    return NULL;
}

#define NEED(dst, nm, cnt)                                      \
    do {                                                        \
        (dst) = find(m, (nm), (int64_t)(cnt), err, errlen);     \
        if (!(dst)) return -1;                                  \
    } while (0)

static int load_conv(ko_model* m, conv_t* c, const char* p, int cin, int cout, int k, int stride, int pad, int dil,
                     int bias, int mfma, char* err, size_t errlen) {
    char nm[256];
    c->cin = cin, c->cout = cout, c->k = k, c->stride = stride, c->pad = pad, c->dil = dil, c->mfma = mfma;
    snprintf(nm, sizeof nm, "%s.weight", p);
    NEED(c->w, nm, (int64_t)cout * cin * k);
    c->b = NULL;
    if (bias) {
        snprintf(nm, sizeof nm, "%s.bias", p);
        NEED(c->b, nm, cout);
    }
    return 0;
}

static int load_adain(ko_model* m, adain_t* a, const char* p, int c, char* err, size_t errlen) {
    char nm[256];
    a->c = c;
    snprintf(nm, sizeof nm, "%s.norm.weight", p);
    NEED(a->nw, nm, c);
    snprintf(nm, sizeof nm, "%s.norm.bias", p);
    NEED(a->nb, nm, c);
    snprintf(nm, sizeof nm, "%s.fc.weight", p);
    NEED(a->fw, nm, (int64_t)2 * c * STYLE_DIM);
    snprintf(nm, sizeof nm, "%s.fc.bias", p);
    NEED(a->fb, nm, 2 * c);
    return 0;
}

/* AdaInResBlock1::load (src/nn.rs:154-165): convs1 pad (k*d-d)/2 dil d; convs2 pad (k-1)/2. */
static int load_snake(ko_model* m, snake_t* s, const char* p, int c, int k, char* err, size_t errlen) {
    static const int dil[3] = {1, 3, 5};
    char nm[256];
    s->c = c;
    for (int i = 0; i < 3; i++) {
        int d = dil[i];
        snprintf(nm, sizeof nm, "%s.convs1.%d", p, i);
        if (load_conv(m, &s->c1[i], nm, c, c, k, 1, (k * d - d) / 2, d, 1, KO_GROUP_SNAKE, err, errlen)) return -1;
        snprintf(nm, sizeof nm, "%s.convs2.%d", p, i);
        if (load_conv(m, &s->c2[i], nm, c, c, k, 1, (k - 1) / 2, 1, 1, KO_GROUP_SNAKE, err, errlen)) return -1;
        snprintf(nm, sizeof nm, "%s.adain1.%d", p, i);
        if (load_adain(m, &s->a1[i], nm, c, err, errlen)) return -1;
        snprintf(nm, sizeof nm, "%s.adain2.%d", p, i);
        if (load_adain(m, &s->a2[i], nm, c, err, errlen)) return -1;
        snprintf(nm, sizeof nm, "%s.alpha1.%d", p, i);
        NEED(s->al1[i], nm, c);
        snprintf(nm, sizeof nm, "%s.alpha2.%d", p, i);
        NEED(s->al2[i], nm, c);
    }
    return 0;
}

/* AdainResBlk1d::load (src/nn.rs:119-140). */
static int load_resblk(ko_model* m, resblk_t* r, const char* p, int din, int dout, int up, char* err, size_t errlen) {
    char nm[256];
    r->din = din, r->dout = dout, r->up = up;
    snprintf(nm, sizeof nm, "%s.conv1", p);
    if (load_conv(m, &r->conv1, nm, din, dout, 3, 1, 1, 1, 1, KO_GROUP_DECODER, err, errlen)) return -1;
    snprintf(nm, sizeof nm, "%s.conv2", p);
    if (load_conv(m, &r->conv2, nm, dout, dout, 3, 1, 1, 1, 1, KO_GROUP_DECODER, err, errlen)) return -1;
    snprintf(nm, sizeof nm, "%s.norm1", p);
    if (load_adain(m, &r->n1, nm, din, err, errlen)) return -1;
    snprintf(nm, sizeof nm, "%s.norm2", p);
    if (load_adain(m, &r->n2, nm, dout, err, errlen)) return -1;
    r->has_1x1 = din != dout;
    if (r->has_1x1) {
        snprintf(nm, sizeof nm, "%s.conv1x1", p);
        if (load_conv(m, &r->conv1x1, nm, din, dout, 1, 1, 0, 1, 0, KO_GROUP_DECODER, err, errlen)) return -1;
    }
    r->pool_w = r->pool_b = NULL;
    if (up) {
        snprintf(nm, sizeof nm, "%s.pool.weight", p);
        NEED(r->pool_w, nm, (int64_t)din * 3);
        snprintf(nm, sizeof nm, "%s.pool.bias", p);
        NEED(r->pool_b, nm, din);
    }
    return 0;
}

static int load_convt(ko_model* m, convt_t* c, const char* p, int cin, int cout, int k, int stride, int pad, char* err,
                      size_t errlen) {
    char nm[256];
    c->cin = cin, c->cout = cout, c->k = k, c->stride = stride, c->pad = pad;
    snprintf(nm, sizeof nm, "%s.weight", p);
    NEED(c->w, nm, (int64_t)cin * cout * k);
    snprintf(nm, sizeof nm, "%s.bias", p);
    NEED(c->b, nm, cout);
    return 0;
}

void ko_model_free(ko_model* m) {
    if (!m) return;
    for (int i = 0; i < m->n; i++) {
        free(m->names[i]);
        free(m->data[i]);
    }
    free(m->names);
    free(m->data);
    free(m->numel);
    free(m);
}

/* Shapes: src/vocoder.rs:54-111 (Generator::load, Decoder::load). */
int ko_model_create(int n, const char* const* names, const float* const* data, const int64_t* numel, ko_model** out,
                    char* err, size_t errlen) {
    ko_model* m = (ko_model*)calloc(1, sizeof(ko_model));
    m->n = n;
    m->names = (char**)calloc(n, sizeof(char*));
    m->data = (float**)calloc(n, sizeof(float*));
    m->numel = (int64_t*)calloc(n, sizeof(int64_t));
    for (int i = 0; i < n; i++) {
        m->names[i] = strdup(names[i]);
        m->numel[i] = numel[i];
        m->data[i] = (float*)malloc((size_t)(numel[i] > 0 ? numel[i] : 1) * sizeof(float));
        memcpy(m->data[i], data[i], (size_t)numel[i] * sizeof(float));
    }
    char nm[256];
    int rc = 0;
    rc |= load_resblk(m, &m->encode, "decoder.encode", 514, 1024, 0, err, errlen);
    for (int i = 0; i < 4 && !rc; i++) {
        snprintf(nm, sizeof nm, "decoder.decode.%d", i);
        rc |= load_resblk(m, &m->decode[i], nm, 1090, i == 3 ? 512 : 1024, i == 3, err, errlen);
    }
    if (!rc) rc |= load_conv(m, &m->f0_conv, "decoder.F0_conv", 1, 1, 3, 2, 1, 1, 1, 0, err, errlen);
    if (!rc) rc |= load_conv(m, &m->n_conv, "decoder.N_conv", 1, 1, 3, 2, 1, 1, 1, 0, err, errlen);
    if (!rc) rc |= load_conv(m, &m->asr_res, "decoder.asr_res.0", 512, 64, 1, 1, 0, 1, 1, KO_GROUP_DECODER, err, errlen);
    const char* g = "decoder.generator";
    if (!rc) {
        const float* lb;
        snprintf(nm, sizeof nm, "%s.m_source.l_linear.weight", g);
        m->l_w = find(m, nm, HARMONICS, err, errlen);
        snprintf(nm, sizeof nm, "%s.m_source.l_linear.bias", g);
        lb = find(m, nm, 1, err, errlen);
        if (!m->l_w || !lb) rc = -1;
        else m->l_b = lb[0];
    }
    if (!rc) {
        snprintf(nm, sizeof nm, "%s.noise_convs.0", g);
        rc |= load_conv(m, &m->noise_convs[0], nm, 22, 256, 12, 6, 3, 1, 1, 0, err, errlen);
    }
    if (!rc) {
        snprintf(nm, sizeof nm, "%s.noise_convs.1", g);
        rc |= load_conv(m, &m->noise_convs[1], nm, 22, 128, 1, 1, 0, 1, 1, 0, err, errlen);
    }
    if (!rc) {
        snprintf(nm, sizeof nm, "%s.noise_res.0", g);
        rc |= load_snake(m, &m->noise_res[0], nm, 256, 7, err, errlen);
    }
    if (!rc) {
        snprintf(nm, sizeof nm, "%s.noise_res.1", g);
        rc |= load_snake(m, &m->noise_res[1], nm, 128, 11, err, errlen);
    }
    if (!rc) {
        snprintf(nm, sizeof nm, "%s.ups.0", g);
        rc |= load_convt(m, &m->ups[0], nm, 512, 256, 20, 10, 5, err, errlen);
    }
    if (!rc) {
        snprintf(nm, sizeof nm, "%s.ups.1", g);
        rc |= load_convt(m, &m->ups[1], nm, 256, 128, 12, 6, 3, err, errlen);
    }
    static const int ks[3] = {3, 7, 11};
    for (int i = 0; i < 6 && !rc; i++) {
        snprintf(nm, sizeof nm, "%s.resblocks.%d", g, i);
        rc |= load_snake(m, &m->resblocks[i], nm, i < 3 ? 256 : 128, ks[i % 3], err, errlen);
    }
    if (!rc) {
        snprintf(nm, sizeof nm, "%s.conv_post", g);
        rc |= load_conv(m, &m->conv_post, nm, 128, 22, 7, 1, 3, 1, 1, KO_GROUP_POST, err, errlen);
    }
    if (rc) {
        ko_model_free(m);
        *out = NULL;
        return -1;
    }
    *out = m;
    return 0;
}

/* A conv layer with the bf16 operand emulation applied to the layers the HIP path runs on MFMA. */
static void conv_layer(const conv_t* c, const float* x, int t, float* y, int tout) {
    if (g_bf16 && (c->mfma & g_groups)) {
        float* xr = round_copy(x, (size_t)c->cin * t, c->mfma);
        float* wr = round_copy(c->w, (size_t)c->cout * c->cin * c->k, c->mfma);
        conv1d_raw(xr, c->cin, t, wr, c->b, c->cout, c->k, c->stride, c->pad, c->dil, y, tout);
        free(xr);
        free(wr);
    } else {
        conv1d_raw(x, c->cin, t, c->w, c->b, c->cout, c->k, c->stride, c->pad, c->dil, y, tout);
    }
}

static void convt_layer(const convt_t* c, const float* x, int t, float* y, int tout) {
    if (g_bf16 && (g_groups & KO_GROUP_UPS)) {
        float* xr = round_copy(x, (size_t)c->cin * t, KO_GROUP_UPS);
        float* wr = round_copy(c->w, (size_t)c->cin * c->cout * c->k, KO_GROUP_UPS);
        ko_conv_transpose1d(xr, c->cin, t, wr, c->b, c->cout, c->k, c->stride, c->pad, y, tout);
        free(xr);
        free(wr);
    } else {
        ko_conv_transpose1d(x, c->cin, t, c->w, c->b, c->cout, c->k, c->stride, c->pad, y, tout);
    }
}

static void adain_act(const adain_t* a, const float* x, int t, const float* style, int mode, float slope,
                      const float* alpha, float* y) {
    int c = a->c;
    float* gb = (float*)malloc((size_t)2 * c * sizeof(float));
    float* mean = (float*)malloc((size_t)c * sizeof(float));
    float* rstd = (float*)malloc((size_t)c * sizeof(float));
    ko_style_fc(a->fw, a->fb, 2 * c, style, gb);
    ko_chan_stats(x, c, t, mean, rstd);
    ko_adain_apply(x, c, t, mean, rstd, a->nw, a->nb, gb, mode, slope, alpha, y);
    free(gb);
    free(mean);
    free(rstd);
}

/* snake_b (src/gpu_batch.rs:140-154).  res16 (emulation only): the running sum is an fp16 stream
 * on the HIP path -- rounded after each of the first `res16` steps (3 for a generator resblock
 * whose stream the stage's mean reads, 2 for the block whose last sum the mean takes unrounded;
 * 0: an f32 stream). */
static void snake_block(const snake_t* s, const float* x, int t, const float* style, float* out, int res16) {
    size_t n = (size_t)s->c * t;
    float* h = (float*)malloc(n * sizeof(float));
    float* u = (float*)malloc(n * sizeof(float));
    const int h16 = g_bf16 && (g_groups & KO_GROUP_H16);
    if (out != x) memcpy(out, x, n * sizeof(float));
    for (int i = 0; i < 3; i++) {
        adain_act(&s->a1[i], out, t, style, 1, 0.0f, s->al1[i], u);
        conv_layer(&s->c1[i], u, t, h, t);
        /* the HIP path stores conv1's output (the input of adain2) in fp16 */
        if (h16)
            for (size_t j = 0; j < n; j++) h[j] = ko_fp16_round(h[j]);
        adain_act(&s->a2[i], h, t, style, 1, 0.0f, s->al2[i], u);
        conv_layer(&s->c2[i], u, t, h, t);
        for (size_t j = 0; j < n; j++) out[j] = out[j] + h[j];
        if (h16 && i < res16)
            for (size_t j = 0; j < n; j++) out[j] = ko_fp16_round(out[j]);
    }
    free(h);
    free(u);
}

/* resblk_b (src/gpu_batch.rs:104-135): output [dout][up ? 2t : t]. */
static void resblk(const resblk_t* r, const float* x, int t, const float* style, float* out) {
    int t2 = r->up ? 2 * t : t;
    float* a = (float*)malloc((size_t)r->din * t * sizeof(float));
    adain_act(&r->n1, x, t, style, 0, 0.2f, NULL, a);
    float* p = a;
    if (r->up) {
        /* dw_convT_k3s2 (kernels/kokoro.cu:150-166): bias, then ascending contributing inputs. */
        p = (float*)malloc((size_t)r->din * t2 * sizeof(float));
#pragma omp parallel for schedule(static)
        for (int c = 0; c < r->din; c++) {
            for (int o = 0; o < t2; o++) {
                float acc = r->pool_b[c];
                for (int i = (o - 1) / 2 - 1; i <= (o + 1) / 2; i++) {
                    if (i < 0 || i >= t) continue;
                    int k = o + 1 - 2 * i;
                    if (k < 0 || k >= 3) continue;
                    acc = acc + r->pool_w[c * 3 + k] * a[(size_t)c * t + i];
                }
                p[(size_t)c * t2 + o] = acc;
            }
        }
    }
    float* h = (float*)malloc((size_t)r->dout * t2 * sizeof(float));
    conv_layer(&r->conv1, p, t2, h, t2);
    float* u = (float*)malloc((size_t)r->dout * t2 * sizeof(float));
    adain_act(&r->n2, h, t2, style, 0, 0.2f, NULL, u);
    conv_layer(&r->conv2, u, t2, h, t2);
    /* shortcut: nearest x2 (kernels/kokoro.cu:142-148) then conv1x1 */
    float* sc = (float*)malloc((size_t)r->din * t2 * sizeof(float));
    if (r->up) {
        for (int c = 0; c < r->din; c++)
            for (int o = 0; o < t2; o++) sc[(size_t)c * t2 + o] = x[(size_t)c * t + (o >> 1)];
    } else {
        memcpy(sc, x, (size_t)r->din * t * sizeof(float));
    }
    const float* scv = sc;
    float* sc2 = NULL;
    if (r->has_1x1) {
        sc2 = (float*)malloc((size_t)r->dout * t2 * sizeof(float));
        conv_layer(&r->conv1x1, sc, t2, sc2, t2);
        scv = sc2;
    }
    const float s2 = 1.0f / sqrtf(2.0f);
    size_t n = (size_t)r->dout * t2;
    for (size_t j = 0; j < n; j++) out[j] = (h[j] + scv[j]) * s2;
    if (p != a) free(p);
    free(a);
    free(h);
    free(u);
    free(sc);
    free(sc2);
}

int ko_resblk_forward(const ko_model* m, const char* prefix, const float* x, int t, const float* style, float* out) {
    const resblk_t* r = NULL;
    if (strcmp(prefix, "decoder.encode") == 0) r = &m->encode;
    for (int i = 0; i < 4; i++) {
        char nm[64];
        snprintf(nm, sizeof nm, "decoder.decode.%d", i);
        if (strcmp(prefix, nm) == 0) r = &m->decode[i];
    }
    if (!r || t <= 0) return -1;
    resblk(r, x, t, style, out);
    return 0;
}

int ko_snake_block_forward(const ko_model* m, const char* prefix, const float* x, int t, const float* style,
                           float* out) {
    const snake_t* s = NULL;
    char nm[96];
    for (int i = 0; i < 2; i++) {
        snprintf(nm, sizeof nm, "decoder.generator.noise_res.%d", i);
        if (strcmp(prefix, nm) == 0) s = &m->noise_res[i];
    }
    for (int i = 0; i < 6; i++) {
        snprintf(nm, sizeof nm, "decoder.generator.resblocks.%d", i);
        if (strcmp(prefix, nm) == 0) s = &m->resblocks[i];
    }
    if (!s || t <= 0) return -1;
    snake_block(s, x, t, style, out, 0);
    return 0;
}

/* Decoder glue (src/gpu_batch.rs:299-317). */
int ko_decoder_forward(const ko_model* m, const float* asr, const float* f0, const float* en, const float* style,
                       int n, float* x_out) {
    if (n <= 0) return -1;
    float* f0n = (float*)malloc((size_t)n * sizeof(float));
    float* nn = (float*)malloc((size_t)n * sizeof(float));
    conv_layer(&m->f0_conv, f0, 2 * n, f0n, n);
    conv_layer(&m->n_conv, en, 2 * n, nn, n);
    float* xcat = (float*)malloc((size_t)1090 * n * sizeof(float));
    memcpy(xcat, asr, (size_t)512 * n * sizeof(float));
    memcpy(xcat + (size_t)512 * n, f0n, (size_t)n * sizeof(float));
    memcpy(xcat + (size_t)513 * n, nn, (size_t)n * sizeof(float));
    float* x = (float*)malloc((size_t)1024 * n * sizeof(float));
    resblk(&m->encode, xcat, n, style, x);
    float* ar = (float*)malloc((size_t)64 * n * sizeof(float));
    conv_layer(&m->asr_res, asr, n, ar, n);
    for (int i = 0; i < 4; i++) {
        memcpy(xcat, x, (size_t)1024 * n * sizeof(float));
        memcpy(xcat + (size_t)1024 * n, ar, (size_t)64 * n * sizeof(float));
        memcpy(xcat + (size_t)1088 * n, f0n, (size_t)n * sizeof(float));
        memcpy(xcat + (size_t)1089 * n, nn, (size_t)n * sizeof(float));
        if (i < 3) {
            resblk(&m->decode[i], xcat, n, style, x);
        } else {
            resblk(&m->decode[i], xcat, n, style, x_out);
        }
    }
    free(f0n);
    free(nn);
    free(xcat);
    free(x);
    free(ar);
    return 0;
}

static void leaky_inplace(float* x, size_t n, float slope) {
    for (size_t i = 0; i < n; i++)
        if (x[i] < 0.0f) x[i] = x[i] * slope;
}

/* Mean of the three resblocks of a stage (src/gpu_batch.rs:395-401): acc = rb0; acc += rb_j; acc /= 3. */
static void resblock_mean(const ko_model* m, int first, const float* y, int t, const float* style, float* out) {
    int c = m->resblocks[first].c;
    size_t n = (size_t)c * t;
    float* r = (float*)malloc(n * sizeof(float));
    snake_block(&m->resblocks[first], y, t, style, out, 3);
    for (int j = 1; j < 3; j++) {
        snake_block(&m->resblocks[first + j], y, t, style, r, j < 2 ? 3 : 2);
        for (size_t i = 0; i < n; i++) out[i] = out[i] + r[i];
    }
    for (size_t i = 0; i < n; i++) out[i] = out[i] / 3.0f;
    free(r);
}

/* With the emulation of the fp16 streams (KO_GROUP_H16): x rounded to fp16 in place. */
static void round_h16(float* x, size_t n) {
    if (g_bf16 && (g_groups & KO_GROUP_H16))
        for (size_t i = 0; i < n; i++) x[i] = ko_fp16_round(x[i]);
}

/* Generator stages after the source (src/gpu_batch.rs:358-420), one item, from spec [22][120N+1].
 * The emulation rounds where the HIP path keeps fp16 streams: the noise branches (from the noise
 * conv's output on) and each stage's input (the ConvT's output plus the noise branch). */
int ko_generator_from_spec(const ko_model* m, const float* x_in, const float* spec, const float* style, int n,
                           float* audio, float* post_out) {
    if (n <= 0) return -1;
    const int l2 = 2 * n, f = 120 * n + 1, t0 = 20 * n, t1 = 120 * n + 1;
    /* stage 0 */
    float* x = (float*)malloc((size_t)512 * l2 * sizeof(float));
    memcpy(x, x_in, (size_t)512 * l2 * sizeof(float));
    leaky_inplace(x, (size_t)512 * l2, 0.1f);
    float* xs = (float*)malloc((size_t)256 * t0 * sizeof(float));
    conv_layer(&m->noise_convs[0], spec, f, xs, t0);
    round_h16(xs, (size_t)256 * t0);
    snake_block(&m->noise_res[0], xs, t0, style, xs, 3);
    float* y = (float*)malloc((size_t)256 * t0 * sizeof(float));
    convt_layer(&m->ups[0], x, l2, y, t0);
    for (size_t i = 0; i < (size_t)256 * t0; i++) y[i] = y[i] + xs[i];
    round_h16(y, (size_t)256 * t0);
    float* x1 = (float*)malloc((size_t)256 * t0 * sizeof(float));
    resblock_mean(m, 0, y, t0, style, x1);
    free(x);
    free(xs);
    free(y);

    /* stage 1 */
    leaky_inplace(x1, (size_t)256 * t0, 0.1f);
    float* xs1 = (float*)malloc((size_t)128 * t1 * sizeof(float));
    conv_layer(&m->noise_convs[1], spec, f, xs1, t1);
    round_h16(xs1, (size_t)128 * t1);
    snake_block(&m->noise_res[1], xs1, t1, style, xs1, 3);
    float* y0 = (float*)malloc((size_t)128 * (t1 - 1) * sizeof(float));
    convt_layer(&m->ups[1], x1, t0, y0, t1 - 1);
    float* y1 = (float*)malloc((size_t)128 * t1 * sizeof(float));
    /* ReflectionPad1d((1,0)) (kernels/kokoro.cu:452-467): out[0] = in[1], out[1+j] = in[j] */
    for (int c = 0; c < 128; c++) {
        const float* src = y0 + (size_t)c * (t1 - 1);
        float* dst = y1 + (size_t)c * t1;
        dst[0] = src[1];
        memcpy(dst + 1, src, (size_t)(t1 - 1) * sizeof(float));
    }
    for (size_t i = 0; i < (size_t)128 * t1; i++) y1[i] = y1[i] + xs1[i];
    round_h16(y1, (size_t)128 * t1);
    float* x2 = (float*)malloc((size_t)128 * t1 * sizeof(float));
    resblock_mean(m, 3, y1, t1, style, x2);
    free(x1);
    free(xs1);
    free(y0);
    free(y1);

    leaky_inplace(x2, (size_t)128 * t1, 0.01f);
    float* post = (float*)malloc((size_t)22 * t1 * sizeof(float));
    conv_layer(&m->conv_post, x2, t1, post, t1);
    if (post_out) memcpy(post_out, post, (size_t)22 * t1 * sizeof(float));
    ko_istft20(post, t1, audio);
    free(x2);
    free(post);
    return 0;
}

/* Generator (src/gpu_batch.rs:319-420), one item: source + STFT, then the stages above. */
int ko_generator_forward(const ko_model* m, const float* x_in, const float* f0, const float* style, int n,
                         const float* rand_ini, const float* noise, float* audio, float* spec_out, float* post_out) {
    if (n <= 0) return -1;
    const int l2 = 2 * n, s = 600 * n, f = 120 * n + 1;
    float* har = (float*)malloc((size_t)s * sizeof(float));
    ko_sine_source(f0, l2, rand_ini, noise, m->l_w, m->l_b, NULL, har);
    float* spec = (float*)malloc((size_t)22 * f * sizeof(float));
    ko_stft20(har, s, spec, f);
    free(har);
    if (spec_out) memcpy(spec_out, spec, (size_t)22 * f * sizeof(float));
    int rc = ko_generator_from_spec(m, x_in, spec, style, n, audio, post_out);
    free(spec);
    return rc;
}
