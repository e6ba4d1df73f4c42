// kk_misc.hip -- bandwidth-bound kernels of the decoder + generator path (gfx950).
//
// All activations are time-major [rows][ld] f32 with items packed along the rows (see
// kk_common.h).  Each kernel cites the reference kernel / host step whose semantics it restates.
#include "kk_common.h"
#include "kk_kernels.h"

namespace kk {

// Periodic Hann(20) window and DFT twiddles, computed in f64 on the host exactly as
// src/gpu.rs:93-101 does (uploaded once per context).
__constant__ double c_cos[11][20];
__constant__ double c_sin[11][20];
__constant__ float c_win[20];

namespace {

constexpr float kPiF = 3.14159274101257324f;  // (float)M_PI, kernels/kokoro.cu:9

// Four floats rounded to fp16 (to nearest even, v_cvt_pk_f16_f32), packed for one 8-byte store.
__device__ __forceinline__ uint2 pack_f16x4(float4 v) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t a = __builtin_convertvector((f32x2_t){v.x, v.y}, f16x2_t);
    const f16x2_t b = __builtin_convertvector((f32x2_t){v.z, v.w}, f16x2_t);
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

// ------------------------------------------------------------------ AdaIN statistics
// Statistics partials of x over item-aligned tiles: per (tile, channel) the sums of (v - shift) and
// (v - shift)^2 with shift = the tile's first value (the centring of chan_stats_seg,
// kernels/kokoro.cu:779-810, applied per tile).  One wave per 64 channels and row phase.
__global__ __launch_bounds__(256) void stats_tiles_kernel(const float* __restrict__ x, int64_t ld, int c, TilesDev t,
                                                          StatPart* __restrict__ part) {
    __shared__ float sa[4][64], sb[4][64];
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    const int ch = blockIdx.y * 64 + lane;
    const int64_t tile = blockIdx.x;
    const int64_t t0 = t.t0[tile];
    const int n = t.n[tile];
    float shift = 0.f, s1 = 0.f, s2 = 0.f;
    if (ch < c) {
        shift = x[t0 * ld + ch];
#pragma unroll 8
        for (int r = g; r < n; r += 4) {
            const float d = x[(t0 + r) * ld + ch] - shift;
            s1 += d;
            s2 = __builtin_fmaf(d, d, s2);
        }
    }
    sa[g][lane] = s1;
    sb[g][lane] = s2;
    __syncthreads();
    if (g == 0 && ch < c) {
        s1 = ((sa[0][lane] + sa[1][lane]) + sa[2][lane]) + sa[3][lane];
        s2 = ((sb[0][lane] + sb[1][lane]) + sb[2][lane]) + sb[3][lane];
        part[tile * c + ch] = StatPart{s1, s2, shift, (float)n};
    }
}

// Per (item, channel): combine the item's partials in a fixed order, then mean / rstd exactly as
// chan_stats_seg's epilogue (biased variance, eps 1e-5, rstd = 1 / sqrtf((float)var + eps)) and the
// AdaIN affine of adain_apply_seg (kernels/kokoro.cu:318-334) folded into v = x * sc + sh.
// Every partial is re-centred on one reference per (item, channel) -- the item's first partial's
// shift, a value of the data -- so the f64 sums need no division per partial and the final
// E[d^2] - E[d]^2 cancels only over a few standard deviations.  SUB threads per (item, channel)
// reduce in a fixed tree: deterministic, no atomics.  Each thread issues the loads of up to LOADS
// partials before it adds any, and the launcher picks the smallest SUB (16, 32 or 64) and LOADS
// (1, 4 or 8) that cover the largest item's partials in one such round: one memory latency per
// launch for most layers, and no idle threads for the decoder's few partials per item.  One launch
// serves every AdaIN layer that normalises the same tensor (outs: the three resblocks of a stage
// read the same input): the statistics once, then each layer's coefficients.
template <int SUB, int LOADS>
__global__ __launch_bounds__(16 * SUB) void finalize_kernel(const StatPart* __restrict__ part, int c, int wn, TilesDev t,
                                                            const float* __restrict__ gb, int64_t gb_ld, FinOuts outs,
                                                            const uint16_t* __restrict__ xrow, int64_t xrow_ld,
                                                            const int64_t* __restrict__ xrow_at) {
    constexpr int kFinSub = SUB;
    __shared__ double sa[kFinSub][16], sb[kFinSub][16], sn[kFinSub][16];
    const int cl = threadIdx.x & 15, sub = threadIdx.x >> 4;
    const int b = blockIdx.x;
    const int ch = blockIdx.y * 16 + cl;
    const int64_t lo = (int64_t)t.lo[b] * wn, hi = (int64_t)t.hi[b] * wn;
    double a1 = 0.0, a2 = 0.0, n = 0.0, ref = 0.0;
    auto add = [&](const StatPart& q) {
        if (q.n > 0.f) {
            const double dn = (double)q.n, d = (double)q.shift - ref, s1 = (double)q.s1;
            // sums of (v - ref) and (v - ref)^2 over the partial's columns
            a1 += s1 + dn * d;
            a2 += (double)q.s2 + 2.0 * d * s1 + dn * d * d;
            n += dn;
        }
    };
    if (ch < c && lo < hi) {
        ref = (double)part[lo * c + ch].shift;
        // partials lo + sub, lo + sub + SUB, ... in increasing order; past hi a record with n = 0
        for (int64_t base = lo + sub; base < hi; base += LOADS * kFinSub) {
            StatPart q[LOADS];
#pragma unroll
            for (int j = 0; j < LOADS; j++) {
                const int64_t pi = base + j * kFinSub;
                q[j] = pi < hi ? part[pi * c + ch] : StatPart{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int j = 0; j < LOADS; j++) add(q[j]);
        }
    }
    sa[sub][cl] = a1, sb[sub][cl] = a2, sn[sub][cl] = n;
    __syncthreads();
    for (int k = kFinSub / 2; k > 0; k >>= 1) {
        if (sub < k) {
            sa[sub][cl] += sa[sub + k][cl];
            sb[sub][cl] += sb[sub + k][cl];
            sn[sub][cl] += sn[sub + k][cl];
        }
        __syncthreads();
    }
    if (sub != 0 || ch >= c) return;
    a1 = sa[0][cl], a2 = sb[0][cl], n = sn[0][cl];
    if (xrow) {  // one more sample of the item, outside the partials: row xrow_at[b] of xrow (fp16)
        const double d = (double)(float)__builtin_bit_cast(_Float16, xrow[xrow_at[b] * xrow_ld + ch]) - ref;
        a1 += d, a2 += d * d, n += 1.0;
    }
    const int64_t i = (int64_t)b * c + ch;
    if (n <= 0.0) {
#pragma unroll
        for (int k = 0; k < kFinMaxOuts; k++)
            if (k < outs.n) outs.o[k].coef[i] = Coef{0.f, 0.f};
        return;
    }
    const double dm = a1 / n;
    double var = a2 / n - dm * dm;
    if (var < 0.0) var = 0.0;
    const float meanf = (float)(ref + dm);
    const float rstd = 1.0f / sqrtf((float)var + 1e-5f);
    // each AdaIN layer of this tensor: its own style offset, norm weight / bias and coefficients
#pragma unroll
    for (int k = 0; k < kFinMaxOuts; k++) {
        if (k >= outs.n) break;
        const FinOut& o = outs.o[k];
        const double g1 = 1.0 + (double)gb[b * gb_ld + o.gb_off + ch];
        const double beta = gb[b * gb_ld + o.gb_off + c + ch];
        const double a = (double)rstd * (double)o.nw[ch];
        o.coef[i] = Coef{(float)(a * g1), (float)(((double)o.nb[ch] - (double)meanf * a) * g1 + beta)};
    }
}

// ------------------------------------------------------------------ style projections
// GLinear of every AdaIN (src/gpu_batch.rs:84): gb[b][j] = bias[j] + sum_k W[j][k] style[b][k], summed
// in f64.  W is stored transposed [128][rows] so consecutive threads read consecutive rows.  A block
// covers 64 rows; its four waves take one quarter of k each (the loads of a quarter issued
// together), and the quarters' sums meet in LDS, 16 items per pass.
__global__ __launch_bounds__(256) void style_fc_kernel(const float* __restrict__ wt, const float* __restrict__ bias,
                                                       int rows, const float* __restrict__ style, int nb,
                                                       float* __restrict__ gb) {
    __shared__ float st[16][kStyleDim];
    __shared__ double part[3][16][64];
    const int r = threadIdx.x & 63, q = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + r;
    const int jc = j < rows ? j : rows - 1;
    float w[32];
#pragma unroll
    for (int i = 0; i < 32; i++) w[i] = wt[(int64_t)(32 * q + i) * rows + jc];
    for (int b0 = 0; b0 < nb; b0 += 16) {
        const int cnt = min(16, nb - b0);
        __syncthreads();
        for (int i = threadIdx.x; i < 16 * kStyleDim; i += 256)
            st[i / kStyleDim][i % kStyleDim] = i / kStyleDim < cnt ? style[(int64_t)b0 * kStyleDim + i] : 0.f;
        __syncthreads();
        double acc[16];
#pragma unroll
        for (int e = 0; e < 16; e++) acc[e] = 0.0;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const double wv = w[i];
#pragma unroll
            for (int e = 0; e < 16; e++) acc[e] += wv * (double)st[e][32 * q + i];
        }
        if (q > 0)
#pragma unroll
            for (int e = 0; e < 16; e++) part[q - 1][e][r] = acc[e];
        __syncthreads();
        if (q == 0 && j < rows)
            for (int e = 0; e < cnt; e++)
                gb[(int64_t)(b0 + e) * rows + j] =
                    (float)(((acc[e] + part[0][e][r]) + (part[1][e][r] + part[2][e][r])) + (double)bias[j]);
    }
}

// ------------------------------------------------------------------ duration expansion
// gather_cols (kernels/kokoro.cu:393-398; src/gpu_batch.rs:295-297): exact copies, gaps -> 0.
__global__ void expand_kernel(const float* __restrict__ t_en, int64_t t_rows, const int32_t* __restrict__ src_row,
                              int64_t l, float* __restrict__ asr, int64_t ld) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= l * 512) return;
    const int64_t t = i >> 9;
    const int ch = (int)(i & 511);
    const int32_t r = src_row[t];
    asr[t * ld + ch] = r < 0 ? 0.0f : t_en[(int64_t)r * 512 + ch];
}

// F0_conv / N_conv (src/vocoder.rs:106-107): Conv1d 1->1 k3 s2 p1, d2 -> dn, f32; gap rows -> 0.
__global__ void f0n_kernel(const float* __restrict__ f0, const float* __restrict__ en, int64_t l2,
                           const float* __restrict__ wf, const float* __restrict__ bf, const float* __restrict__ wn,
                           const float* __restrict__ bn, float* __restrict__ out, int64_t ld, int col_f0, int col_n,
                           const int32_t* __restrict__ col, int64_t ln) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= ln) return;
    float a = bf[0], b = bn[0];
    for (int k = 0; k < 3; k++) {
        const int64_t i = 2 * t - 1 + k;
        if (i < 0 || i >= l2) continue;
        a = a + wf[k] * f0[i];
        b = b + wn[k] * en[i];
    }
    const bool gap = col[t] < 0;
    out[t * ld + col_f0] = gap ? 0.f : a;
    out[t * ld + col_n] = gap ? 0.f : b;
}

__global__ __launch_bounds__(256) void copy_cols_kernel(const float* __restrict__ src, int64_t src_ld, int c,
                                                        float* __restrict__ dst, int64_t dst_ld, int dst_c0,
                                                        const int32_t* __restrict__ col, int64_t l) {
    const int64_t t = blockIdx.x;  // one row per block, threads over its channels
    const bool live = col[t] >= 0;
    for (int ch = threadIdx.x; ch < c; ch += 256) dst[t * dst_ld + dst_c0 + ch] = live ? src[t * src_ld + ch] : 0.f;
}

// Decoder upsample block (src/gpu_batch.rs:106-117): AdaIN + leaky 0.2 (adain_apply_seg, gaps -> 0)
// followed by the depthwise ConvTranspose1d k3 s2 p1 op1 (dw_convT_k3s2, kernels/kokoro.cu:150-166:
// bias, then ascending contributing inputs), masked on d2 and rounded to bf16 for conv1.
// One block per output row o of d2, threads over channel pairs: the row's item and contributing
// inputs are uniform, every load and store is coalesced across the row.
__global__ __launch_bounds__(256) void adain_pool_kernel(const float* __restrict__ x, int64_t ld, int c,
                                                         const Coef* __restrict__ coef,
                                                         const int32_t* __restrict__ col_n, int64_t ln,
                                                         const float* __restrict__ pw, const float* __restrict__ pb,
                                                         const int32_t* __restrict__ col_2, uint16_t* __restrict__ out,
                                                         int64_t out_ld) {
#pragma clang fp contract(off)
    const int64_t o = blockIdx.x;
    const bool live = col_2[o] >= 0;
    // contributing inputs t (ascending) and their taps k = o + 1 - 2 t in [0, 3), at most two
    int64_t tt[2];
    int kk[2], bb[2], nt = 0;
    for (int64_t t = (o - 1) / 2 - 1; t <= (o + 1) / 2; t++) {
        if (t < 0 || t >= ln) continue;
        const int64_t k = o + 1 - 2 * t;
        if (k < 0 || k >= 3 || nt == 2) continue;
        tt[nt] = t, kk[nt] = (int)k, bb[nt] = col_n[t], nt++;
    }
    for (int ch = 2 * threadIdx.x; ch < out_ld; ch += 512) {
        float v[2] = {0.f, 0.f};
        if (live && ch < c) {
            for (int e = 0; e < 2; e++) v[e] = pb[ch + e];
            for (int q = 0; q < nt; q++) {
                float a[2] = {0.f, 0.f};
                if (bb[q] >= 0) {
                    const float2 xv = *(const float2*)(x + tt[q] * ld + ch);
                    const float4 cf = *(const float4*)(coef + (int64_t)bb[q] * c + ch);  // (sc, sh) x 2
                    a[0] = __builtin_fmaf(xv.x, cf.x, cf.y);
                    a[1] = __builtin_fmaf(xv.y, cf.z, cf.w);
                    for (int e = 0; e < 2; e++) a[e] = a[e] < 0.f ? a[e] * 0.2f : a[e];
                }
                for (int e = 0; e < 2; e++) v[e] = v[e] + pw[(ch + e) * 3 + kk[q]] * a[e];
            }
        }
        *(uint32_t*)(out + o * out_ld + ch) = (uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
    }
}

// ------------------------------------------------------------------ noise convolutions (f32)
// conv1d_strided / conv_direct_tiled semantics (kernels/kokoro.cu:517-617): y = b + sum_k sum_ci
// w x with the spectrum's gap rows zeroed first (src/gpu_batch.rs:363-365).  A block computes
constexpr int kNcRows = kNoiseTile;

// noise_convs.1 (22 -> 128, k 1) on the bf16 matrix cores in split precision, as noise_convs.0
// (below): each value and weight split into its bf16 rounding and the rounding of the remainder,
// products accumulated in f32 as wh xh + wh xl + wl xh.  GEMM view per block: 128 output channels
// x the <= 128 rows of one item-aligned tile, K = 22 channels padded to 32 (two steps of 16, the
// pad zero in both operands).  Wave w owns rows 32 w .. 32 w + 31 (one 32-column tile) and all
// 128 channels (four 32-row tiles, taken two at a time).  A lane's B fragment of step s is 8
// consecutive channels of its row, loaded from the spectrum as two float4 and split in registers
// (no LDS staging); the weights are A fragments packed per lane ([32-row tile][step][rounding,
// remainder][lane] bf16x8).  The fp16 outputs go through LDS so that the tile's rows leave as
// contiguous 16-byte runs, and the tile's statistics partial (sums of v - b and (v - b)^2 over its
// rows, shift b: the bias is a value of the data's scale) is summed from the stored fp16 values.
constexpr int kNc1Ld = 128 + 8;  // LDS row stride of the output tile (fp16)
__device__ __forceinline__ bf16x8 bf16x8_of(const uint32_t (&u)[4]) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(bf16x8, (u32x4){u[0], u[1], u[2], u[3]});
}
__global__ __launch_bounds__(256) void noise_conv1_mfma_kernel(const float* __restrict__ spec, int64_t spec_ld,
                                                               const bf16x8* __restrict__ wq,
                                                               const float* __restrict__ b, uint16_t* __restrict__ y,
                                                               int64_t y_ld, TilesDev tl,
                                                               StatPart* __restrict__ part) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    __shared__ __align__(16) uint16_t ys[kNoiseTile1 * kNc1Ld];
    __shared__ float red[2][4][128];
    const int64_t t0 = tl.t0[blockIdx.x];
    const int nv = tl.n[blockIdx.x];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    // this lane's row (rows past the tile read its first row; their outputs are not stored)
    const int r = 32 * wave + l32;
    const float* xr = spec + (t0 + (r < nv ? r : 0)) * spec_ld + 8 * h;
    // B fragments: step 0 channels 8 h .. 8 h + 7, step 1 channels 16 + 8 h .. (22 and up zero)
    const float4 x0 = *(const float4*)xr, x1 = *(const float4*)(xr + 4);
    const float4 x2 = *(const float4*)(xr + 16), x3 = *(const float4*)(xr + 20);
    bf16x8 bh[2], bl[2];
    {
        const float v[2][8] = {{x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w},
                               {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, 0.f, 0.f}};  // 22, 23: the pad
#pragma unroll
        for (int s = 0; s < 2; s++) {
            uint32_t hi[4], lo[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float a = v[s][2 * e], c = v[s][2 * e + 1];
                if (s == 1 && h) a = 0.f, c = 0.f;  // channels 24-31: the pad
                const uint32_t ha = f32_to_bf16_bits(a), hc = f32_to_bf16_bits(c);
                const uint32_t la = f32_to_bf16_bits(a - __uint_as_float(ha << 16));
                const uint32_t lc = f32_to_bf16_bits(c - __uint_as_float(hc << 16));
                hi[e] = ha | hc << 16, lo[e] = la | lc << 16;
            }
            bh[s] = bf16x8_of(hi), bl[s] = bf16x8_of(lo);
        }
    }
    // the weights: tile mt, step s, part p at wq[((mt * 2 + s) * 2 + p) * 64 + lane]
    const bf16x8* wa = wq + lane;
#pragma unroll
    for (int mp = 0; mp < 2; mp++) {  // 32-row tiles 2 mp and 2 mp + 1
        __builtin_amdgcn_sched_barrier(0);  // one pair's weights live at a time (4 blocks per CU)
        bf16x8 a[2][2][2];  // [tile][step][part]
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int s = 0; s < 2; s++)
#pragma unroll
                for (int p = 0; p < 2; p++) a[t][s][p] = wa[(((2 * mp + t) * 2 + s) * 2 + p) * 64];
        f32x16 acc[2];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float4 bv = *(const float4*)(b + 32 * (2 * mp + t) + 8 * g + 4 * h);
                acc[t][4 * g] = bv.x, acc[t][4 * g + 1] = bv.y, acc[t][4 * g + 2] = bv.z, acc[t][4 * g + 3] = bv.w;
            }
#pragma unroll
        for (int s = 0; s < 2; s++)
#pragma unroll
            for (int t = 0; t < 2; t++) {
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[t][s][0], bh[s], acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[t][s][0], bl[s], acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[t][s][1], bh[s], acc[t], 0, 0, 0);
            }
        // D: element 4 g + e of tile t is channel 32 (2 mp + t) + 8 g + 4 h + e of row l32
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(uint2*)(ys + r * kNc1Ld + 32 * (2 * mp + t) + 8 * g + 4 * h) =
                    pack_f16x4(make_float4(acc[t][4 * g], acc[t][4 * g + 1], acc[t][4 * g + 2], acc[t][4 * g + 3]));
    }
    __builtin_amdgcn_wave_barrier();  // the wave's rows written before it reads them back
    // the wave's 32 rows, 16 bytes per lane: 4 rows per instruction, each 256 contiguous bytes
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int rr = 32 * wave + 4 * i + (lane >> 4);
        if (rr < nv) *(uint4*)(y + (t0 + rr) * y_ld + 8 * (lane & 15)) = *(const uint4*)(ys + rr * kNc1Ld + 8 * (lane & 15));
    }
    // statistics of the stored values: lane: channels 2 lane, 2 lane + 1 over the wave's rows
    {
        const float b0 = b[2 * lane], b1 = b[2 * lane + 1];
        float s1a = 0.f, s2a = 0.f, s1b = 0.f, s2b = 0.f;
        const int rn = min(max(nv - 32 * wave, 0), 32);
        for (int i = 0; i < rn; i++) {
            const uint32_t u = *(const uint32_t*)(ys + (32 * wave + i) * kNc1Ld + 2 * lane);
            const float va = (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu)) - b0;
            const float vb = (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16)) - b1;
            s1a += va, s2a = __builtin_fmaf(va, va, s2a);
            s1b += vb, s2b = __builtin_fmaf(vb, vb, s2b);
        }
        red[0][wave][2 * lane] = s1a, red[0][wave][2 * lane + 1] = s1b;
        red[1][wave][2 * lane] = s2a, red[1][wave][2 * lane + 1] = s2b;
    }
    __syncthreads();
    if (threadIdx.x < 128) {  // the waves' sums in order
        const int c = threadIdx.x;
        const float a1 = ((red[0][0][c] + red[0][1][c]) + red[0][2][c]) + red[0][3][c];
        const float a2 = ((red[1][0][c] + red[1][1][c]) + red[1][2][c]) + red[1][3][c];
        part[(int64_t)blockIdx.x * 128 + c] = StatPart{a1, a2, b[c], (float)nv};
    }
}

// noise_convs.0 (22 -> 256, k 12, stride 6) on the bf16 matrix cores in split precision
// (v_mfma_f32_32x32x16_bf16, f32 accumulation).  Every input value and weight is split into its
// bf16 rounding and the bf16 rounding of the remainder (v = vh + vl to within 2^-17 |v|), and each
// product is accumulated as wh xh + wh xl + wl xh: within ~2^-16 of the exact f32 product (the
// dropped wl xl and the two remainders' own roundings), far below the fp16 rounding of the stored
// output (2^-11).  GEMM view per block: 256 output channels x 64 output columns, K = 12 taps x 24
// channels (22 and two zeros) = 288 in 18 steps of 16.  The window is staged row-major, [row][24]
// bf16 in two planes (the roundings, then the remainders), so K index k = 24 tap + ci of output
// column n is window element 144 n + k (row 6 n + tap): a B fragment (8 consecutive k) is one
// 16-byte LDS read.  Wave w owns channels 64 w .. 64 w + 63 (2 x 2 tiles of 32 x 32).
//   A (weights) lane (i = l % 32, h = l / 32) of step c: W[row i][k = 16 c + 8 h + e], e < 8,
//     pre-packed as [32-row tile][step][rounding, remainder][lane] bf16x8;
//   B lane (j, h) of step c: window[144 j + 16 c + 8 h + e].
// Accumulators start at the bias; the epilogue stores each lane's 4 consecutive channels.
constexpr int kNc0Win = (kNcRows - 1) * 6 + 12;  // 390 input rows per 64 output columns
constexpr int kNc0Row = 24;                       // a window row: 22 channels and two zeros
constexpr int kNc0Plane = kNc0Win * kNc0Row;      // bf16 per plane
constexpr int kNc0Steps = 12 * kNc0Row / 16;      // K steps of 16
static_assert(144 * (kNcRows - 1) + 16 * kNc0Steps <= kNc0Plane, "the last column's last B fragment");
__device__ __forceinline__ void split_bf16x4(float4 v, uint2& hi, uint2& lo) {
    const float x[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        h[e] = f32_to_bf16_bits(x[e]);
        l[e] = f32_to_bf16_bits(x[e] - __uint_as_float(h[e] << 16));
    }
    hi = make_uint2(h[0] | h[1] << 16, h[2] | h[3] << 16);
    lo = make_uint2(l[0] | l[1] << 16, l[2] | l[3] << 16);
}
__global__ __launch_bounds__(256, 4) void noise_conv0_mfma_kernel(const float* __restrict__ spec, int64_t spec_ld,
                                                               int64_t l_in, const int64_t* __restrict__ in_start,
                                                               const int64_t* __restrict__ in_len,
                                                               const bf16x8* __restrict__ wq, const float* __restrict__ b,
                                                               int pad, uint16_t* __restrict__ y, int64_t y_ld,
                                                               TilesDev tl, StatPart* __restrict__ part) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    __shared__ __align__(16) uint16_t xs[2 * kNc0Plane];
    const int64_t t0 = tl.t0[blockIdx.x];
    const int nv = tl.n[blockIdx.x];
    const int64_t in0 = t0 * 6 - pad;
    // the tile's item: input rows outside its span are the zero padding (gap masking)
    const int item = tl.item[blockIdx.x];
    const int64_t i_lo = in_start[item], i_hi = i_lo + in_len[item];
    // the window: 6 float4 per row (channels 0-23 of the 32-float spectrum row; 22 and 23 set to 0),
    // every load in flight before the first conversion (rows clamped, the gap / range mask applied
    // afterwards)
    {
        constexpr int kQ = kNc0Win * 6, kPer = (kQ + 255) / 256;
        float4 sv[kPer];
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            const int i = min((int)threadIdx.x + k * 256, kQ - 1);
            const int r = i / 6, q = i - r * 6;
            const int64_t row = min(max(in0 + r, i_lo), i_hi - 1);
            sv[k] = *(const float4*)(spec + row * spec_ld + 4 * q);
        }
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            const int i = threadIdx.x + k * 256;
            if (i < kQ) {
                const int r = i / 6, q = i - r * 6;
                const int64_t row = in0 + r;
                const bool in = row >= i_lo && row < i_hi;
                float4 v = in ? sv[k] : make_float4(0.f, 0.f, 0.f, 0.f);
                if (q == 5) v.z = 0.f, v.w = 0.f;
                uint2 hi, lo;
                split_bf16x4(v, hi, lo);
                *(uint2*)(xs + r * kNc0Row + 4 * q) = hi;
                *(uint2*)(xs + kNc0Plane + r * kNc0Row + 4 * q) = lo;
            }
        }
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l32 = lane & 31, h = lane >> 5;
    f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const float4 bv = *(const float4*)(b + wave * 64 + mi * 32 + 8 * g + 4 * h);
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                acc[mi][ni][4 * g] = bv.x, acc[mi][ni][4 * g + 1] = bv.y;
                acc[mi][ni][4 * g + 2] = bv.z, acc[mi][ni][4 * g + 3] = bv.w;
            }
        }
    }
    // this lane's weights: tile 2 wave + mi, step c, part p at wa[((mi * steps + c) * 2 + p) * 64]
    const bf16x8* wa = wq + (int64_t)(2 * wave) * kNc0Steps * 2 * 64 + lane;
    const uint16_t* xb = xs + 144 * l32 + 8 * h;  // output column l32 (ni = 0); ni = 1 is 32 columns on
    // Step by step: the next step's weights are in flight while this step's 12 MFMAs run; two
    // register sets take turns (steps in pairs), so no copy waits for the loads.
    static_assert(kNc0Steps % 2 == 0, "steps in pairs");
    bf16x8 w0[2][2], w1[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int p = 0; p < 2; p++) w0[mi][p] = wa[(mi * kNc0Steps * 2 + p) * 64];
    auto step = [&](int c, bf16x8(&cur)[2][2], bf16x8(&nxt)[2][2]) {
        const int cn = min(c + 1, kNc0Steps - 1);
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int p = 0; p < 2; p++) nxt[mi][p] = wa[((mi * kNc0Steps + cn) * 2 + p) * 64];
        __builtin_amdgcn_sched_barrier(0);  // the loads stay ahead of this step's MFMAs
        bf16x8 bh[2], bl[2];
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
            bh[ni] = *(const bf16x8*)(xb + ni * 144 * 32 + 16 * c);
            bl[ni] = *(const bf16x8*)(xb + kNc0Plane + ni * 144 * 32 + 16 * c);
        }
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[mi][0], bh[ni], acc[mi][ni], 0, 0, 0);
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[mi][0], bl[ni], acc[mi][ni], 0, 0, 0);
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur[mi][1], bh[ni], acc[mi][ni], 0, 0, 0);
            }
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll 1
    for (int c = 0; c < kNc0Steps; c += 2) {
        step(c, w0, w1);
        step(c + 1, w1, w0);
    }
    // D layout: element 4 g + r of tile (mi, ni) is channel 64 wave + 32 mi + 8 g + 4 h + r of
    // output column t0 + 32 ni + l32.  The fp16 outputs go through the window's space (once every
    // wave is done with it) so that each output row leaves as 512 contiguous bytes, and the tile's
    // statistics partial (sums of v - b and (v - b)^2 over its rows, per channel) is summed from
    // the stored fp16 values.
    constexpr int kOutLd = 256 + 8;  // LDS row stride of the output tile (fp16)
    static_assert(kNcRows * kOutLd <= 2 * kNc0Plane, "the output tile fits the window's space");
    __syncthreads();
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(uint2*)(xs + (32 * ni + l32) * kOutLd + 64 * wave + 32 * mi + 8 * g + 4 * h) = pack_f16x4(
                    make_float4(acc[mi][ni][4 * g], acc[mi][ni][4 * g + 1], acc[mi][ni][4 * g + 2], acc[mi][ni][4 * g + 3]));
    __syncthreads();
    // rows of 512 bytes: 32 lanes of 16 bytes per row, 8 rows per pass of the block
#pragma unroll
    for (int i = 0; i < kNcRows / 8; i++) {
        const int r = 8 * i + (threadIdx.x >> 5), q = threadIdx.x & 31;
        if (r < nv) *(uint4*)(y + (t0 + r) * y_ld + 8 * q) = *(const uint4*)(xs + r * kOutLd + 8 * q);
    }
    // statistics: thread = channel, every row in order
    const float bc = b[threadIdx.x];
    float a1 = 0.f, a2 = 0.f;
    for (int r = 0; r < nv; r++) {
        const float d = (float)__builtin_bit_cast(_Float16, xs[r * kOutLd + threadIdx.x]) - bc;
        a1 += d, a2 = __builtin_fmaf(d, d, a2);
    }
    part[(int64_t)blockIdx.x * 256 + threadIdx.x] = StatPart{a1, a2, bc, (float)nv};
}

// ------------------------------------------------------------------ SineGen (kernels/kokoro.cu:188-254)
__device__ __forceinline__ float remainder1(float a) {
    float m = fmodf(a, 1.0f);
    if (m != 0.0f && m < 0.0f) m = m + 1.0f;
    return m;
}

__device__ __forceinline__ float sine_rad(const float* f0c, int l, float near_scale, int t, int h,
                                          const float* rand_ini) {
#pragma clang fp contract(off)
    int src = (int)floorf((float)t * near_scale);
    if (src > l - 1) src = l - 1;
    float r = remainder1(f0c[src] * (float)(h + 1) / 24000.0f);
    if (t == 0 && h > 0) r = r + rand_ini[h];
    return r;
}

// phase_pre[h][d] = (float(cumsum_f64(v)) * 2 * pi) * 300 where v is the ×1/300 linear downsample of
// rad (sine_phase_pre, kernels/kokoro.cu:206-226).  One block per (item, harmonic); the sequential
// f64 cumulative sum becomes a block scan in f64.
__global__ __launch_bounds__(256) void phase_pre_kernel(const float* __restrict__ f0, const int64_t* __restrict__ start2,
                                                        const int64_t* __restrict__ len2,
                                                        const float* __restrict__ rand_ini, float* __restrict__ pp,
                                                        int64_t pp_ld) {
#pragma clang fp contract(off)
    __shared__ double wsum[4];
    const int b = blockIdx.x / kHarmonics, h = blockIdx.x % kHarmonics;
    const int l = (int)len2[b];
    const float* f0c = f0 + start2[b];
    const float* ri = rand_ini + b * kHarmonics;
    const int s = l * 300;
    const int d_len = (int)floor((double)s * (1.0 / 300.0));
    const float near_scale = (float)(1.0 / 300.0);
    const float down_scale = (float)(1.0 / (1.0 / 300.0));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    double carry = 0.0;
    for (int d0 = 0; d0 < d_len; d0 += 256) {
        const int d = d0 + threadIdx.x;
        double v = 0.0;
        if (d < d_len) {
            float real = __builtin_fmaf(down_scale, (float)d + 0.5f, -0.5f);
            if (real < 0.0f) real = 0.0f;
            int i0 = (int)floorf(real);
            if (i0 > s - 1) i0 = s - 1;
            const float l1 = fminf(fmaxf(real - (float)i0, 0.0f), 1.0f);
            const int i1 = i0 < s - 1 ? i0 + 1 : i0;
            const float l0 = 1.0f - l1;
            v = (double)__builtin_fmaf(sine_rad(f0c, l, near_scale, i0, h, ri), l0,
                                       sine_rad(f0c, l, near_scale, i1, h, ri) * l1);
        }
        // inclusive wave scan in f64
        for (int off = 1; off < 64; off <<= 1) {
            const double u = __shfl_up(v, off, 64);
            if (lane >= off) v += u;
        }
        if (lane == 63) wsum[wave] = v;
        __syncthreads();
        double pre = carry;
        for (int w = 0; w < wave; w++) pre += wsum[w];
        const double tot = wsum[0] + wsum[1] + wsum[2] + wsum[3];
        __syncthreads();
        v += pre;
        if (d < d_len) pp[(int64_t)h * pp_ld + start2[b] + d] = (((float)v) * 2.0f * kPiF) * 300.0f;
        carry += tot;
    }
}

__device__ __forceinline__ uint64_t splitmix_at(uint64_t seed, uint64_t ctr) {
    uint64_t x = seed + (ctr + 1ull) * 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Box-Muller pair i of the counter stream (gen_noise, kernels/kokoro.cu:291-302).
__device__ __forceinline__ void noise_pair(uint64_t seed, uint64_t i, float& n0, float& n1) {
#pragma clang fp contract(off)
    const uint64_t x = splitmix_at(seed, 1024ull + i);
    const float u1 = (float)((x >> 40) + 1ull) * (1.0f / 16777216.0f);
    const float u2 = (float)((x >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);
    const float r = sqrtf(-2.0f * logf(u1));
    const float th = 6.2831855f * u2;
    float sn, cs;
    sincosf(th, &sn, &cs);
    n0 = r * cs;
    n1 = r * sn;
}

// har[t] of one item (sine_har_source, kernels/kokoro.cu:228-254).
__device__ float har_sample(const SourceParams& p, int b, int t) {
#pragma clang fp contract(off)
    const int l = (int)p.len2[b];
    const int d_len = l;
    const float* f0c = p.f0 + p.start2[b];
    const float near_scale = (float)(1.0 / 300.0);
    const float up_scale = (float)(1.0 / 300.0);
    int src = (int)floorf((float)t * near_scale);
    if (src > l - 1) src = l - 1;
    const float f0 = f0c[src];
    const float uv = f0 > 10.0f ? 1.0f : 0.0f;
    const float noise_amp = uv * 0.003f + (1.0f - uv) * 0.1f / 3.0f;
    float real = __builtin_fmaf(up_scale, (float)t + 0.5f, -0.5f);
    if (real < 0.0f) real = 0.0f;
    int i0 = (int)floorf(real);
    if (i0 > d_len - 1) i0 = d_len - 1;
    const float l1 = fminf(fmaxf(real - (float)i0, 0.0f), 1.0f);
    const int i1 = i0 < d_len - 1 ? i0 + 1 : i0;
    const float l0 = 1.0f - l1;
    float nz[kHarmonics + 1];
    const int64_t base = (int64_t)t * kHarmonics;
    if (p.noise_kind[b] == 0) {
        const uint64_t seed = p.seeds[b];
        const int64_t first = base >> 1;
#pragma unroll
        for (int q = 0; q < 5; q++) {
            float n0, n1;
            noise_pair(seed, (uint64_t)(first + q), n0, n1);
            const int64_t i0n = 2 * (first + q) - base;  // harmonic index of n0 (may be -1)
            if (i0n >= 0 && i0n < kHarmonics) nz[i0n] = n0;
            if (i0n + 1 >= 0 && i0n + 1 < kHarmonics) nz[i0n + 1] = n1;
        }
    } else {
        const float* fx = p.fixed_noise + (300 * p.start2[b]) * kHarmonics + base;
#pragma unroll
        for (int h = 0; h < kHarmonics; h++) nz[h] = fx[h];
    }
    const float* pp = p.pp + p.start2[b];
    float acc = 0.0f;
#pragma unroll
    for (int h = 0; h < kHarmonics; h++) {
        const float ph = __builtin_fmaf(pp[h * p.pp_ld + i0], l0, pp[h * p.pp_ld + i1] * l1);
        const float sine = sinf(ph) * 0.1f;
        const float v = sine * uv + noise_amp * nz[h];
        acc = acc + p.lw[h] * v;
    }
    return tanhf(acc + p.lb);
}

// Harmonic source + STFT (stft20_ld, kernels/kokoro.cu:470-490) over a run of frames of one item:
// the frames' reflect-padded samples are synthesized into LDS, then each wave takes 64 frames (one
// per lane) and one half of the 11 bins, so that every twiddle and window value a step reads is
// the same for the whole wave (a scalar load from constant memory) and the lane's 20 windowed
// samples stay in registers across its bins.  Each (frame, bin) is the reference's f64 DFT, term
// by term in the same order.  The magnitudes and phases go through an LDS tile so that the block
// writes its rows of the spectrum as contiguous runs.  One launch covers every item (work list
// blk_item / blk_f0).
constexpr int kSrcOutLd = 23;  // LDS row stride (floats) of the output tile: conflict-free per bin
__global__ __launch_bounds__(256) void source_stft_kernel(SourceParams p) {
#pragma clang fp contract(off)
    static_assert(kSourceFrames == 128, "two frame groups of 64 lanes, two bin halves each");
    __shared__ float har[kSourceFrames * 5 + 15];
    __shared__ float out[kSourceFrames * kSrcOutLd];
    const int64_t blk = blockIdx.x;
    const int b = (int)p.blk_item[blk];
    const int64_t f_begin = p.blk_f0[blk];
    const int64_t nf_item = p.f_len[b];
    const int nf = (int)min((int64_t)kSourceFrames, nf_item - f_begin);
    const int s_len = (int)(300 * p.len2[b]);
    const int64_t p0 = 5 * f_begin - 10;
    const int nsamp = 5 * (nf - 1) + 20;
    for (int i = threadIdx.x; i < nsamp; i += blockDim.x) {
        const int64_t pos = p0 + i;
        const int src = (int)(pos < 0 ? -pos : (pos >= s_len ? 2 * (int64_t)s_len - 2 - pos : pos));
        har[i] = har_sample(p, b, src);
        // test tap: the item's samples in place (blocks' windows overlap by 15 samples and store
        // the same values)
        if (p.har_tap && pos >= 0 && pos < s_len) p.har_tap[5 * p.start120[b] + pos] = har[i];
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int fl = (wave >> 1) * 64 + lane;  // this lane's frame within the block
    const int half = __builtin_amdgcn_readfirstlane(wave & 1);
    if (fl < nf) {
        double v[20];
#pragma unroll
        for (int n = 0; n < 20; n++) v[n] = (double)(har[fl * 5 + n] * c_win[n]);
        auto bin = [&](int k) {
            double re = 0.0, im = 0.0;
#pragma unroll
            for (int n = 0; n < 20; n++) {
                re += v[n] * c_cos[k][n];
                im -= v[n] * c_sin[k][n];
            }
            if (k == 0 || k == 10) im = 0.0;
            const float rf = (float)re, imf = (float)im;
            out[fl * kSrcOutLd + k] = hypotf(rf, imf);
            out[fl * kSrcOutLd + 11 + k] = atan2f(imf, rf);
        };
        if (half == 0) {
#pragma unroll
            for (int k = 0; k < 6; k++) bin(k);
        } else {
#pragma unroll
            for (int k = 6; k < 11; k++) bin(k);
        }
    }
    __syncthreads();
    float* dst = p.spec + (p.start120[b] + f_begin) * p.spec_ld;
    for (int i = threadIdx.x; i < nf * 22; i += blockDim.x) {
        const int f = i / 22, c = i - f * 22;
        dst[f * p.spec_ld + c] = out[f * kSrcOutLd + c];
    }
}

// ------------------------------------------------------------------ iSTFT (kernels/kokoro.cu:264-280, 492-508)
// One block per kIstftSamples output samples of one item.  The block's frames' spectra
// (m cos(sin p), m sin(sin p), computed in f32) are staged in LDS, widened to f64 once, and each
// output sample sums the inverse DFTs of its (up to four) frames at its own tap, in the reference's
// order -- no per-frame buffer, so a CU keeps more blocks (and their loads) in flight.  The f64
// arithmetic is the reference's, rounding for rounding, with three exact rewrites: the tables hold
// 2 cos / 2 sin (scaling by 2 is exact, so RN(re 2c - im 2s) = 2 RN(re c - im s)), the (-1)^n
// term is a sign flip, and v / 20 is q = RN(v r), q + RN((v - 20 q) r) with r = RN(1 / 20) -- the
// correctly rounded quotient (v / 5 of a double is never a binary tie, and the one FMA correction
// brings q within half an ulp; checked against IEEE division on 4e8 values over 200 binades).
// FP contraction is off: every other product and sum rounds as written.
constexpr int kIstftFrames = kIstftSamples / 5 + 5;
struct IdftLds {
    double cs2[20][10], sn2[20][10];  // row n: 2 cos / 2 sin(2 pi k n / 20), k = 1..9, one pad
    float win[20];
};
__device__ __forceinline__ double div20(double v) {
    constexpr double r = 1.0 / 20.0;
    const double q = v * r;
    return __builtin_fma(__builtin_fma(-q, 20.0, v), r, q);
}
__global__ __launch_bounds__(256) void istft_kernel(IstftParams p) {
#pragma clang fp contract(off)
    __shared__ __align__(16) double re[kIstftFrames][12];
    __shared__ __align__(16) double im[kIstftFrames][12];
    __shared__ __align__(16) IdftLds dft;
    for (int i = threadIdx.x; i < 200; i += blockDim.x) {
        const int n = i / 10, k = i - n * 10 + 1;
        (&dft.cs2[0][0])[i] = k < 10 ? 2.0 * c_cos[k][n] : 0.0;
        (&dft.sn2[0][0])[i] = k < 10 ? 2.0 * c_sin[k][n] : 0.0;
    }
    if (threadIdx.x < 20) dft.win[threadIdx.x] = c_win[threadIdx.x];
    const int64_t blk = blockIdx.x;
    const int b = (int)p.blk_item[blk];
    const int64_t s0 = p.blk_s0[blk];
    const int64_t nframes = p.f_len[b];
    const int64_t len = 5 * (nframes - 1);
    const int64_t s1 = min(s0 + kIstftSamples, len);
    // frames touched by samples [s0, s1): j = i + 10, f in [(j-19+4)/5, j/5]
    const int64_t jl = s0 + 10;
    const int64_t f_first = jl - 19 > 0 ? (jl - 19 + 4) / 5 : 0;
    const int64_t f_last = min((s1 - 1 + 10) / 5, nframes - 1);
    const int nfr = (int)(f_last - f_first + 1);
    const float* post = p.post + (p.start120[b] + f_first) * p.post_ld;
    // the block's frames of post, every load in flight before the first use (one memory latency)
    constexpr int kPer = (kIstftFrames * 11 + 255) / 256;
    float lm[kPer], lp[kPer];
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int i = min((int)threadIdx.x + j * 256, nfr * 11 - 1);
        const int q = i / 11, k = i - q * 11;
        lm[j] = post[q * p.post_ld + k];
        lp[j] = post[q * p.post_ld + 11 + k];
    }
#pragma unroll
    for (int j = 0; j < kPer; j++) {
        const int i = threadIdx.x + j * 256;
        if (i < nfr * 11) {
            const int q = i / 11, k = i - q * 11;
            const float m = expf(lm[j]);
            const float ph = sinf(lp[j]);
            float sn, cs;
            sincosf(ph, &sn, &cs);
            re[q][k] = (double)(m * cs);
            im[q][k] = (double)(m * sn);
        }
    }
    __syncthreads();
    // overlap-add in block-local coordinates: jr = j - 5 f_first lies in [10, 531) (f_first is the
    // first frame touching j = s0 + 10), so frame indices and taps are small 32-bit numbers.  Frame
    // f's sample at tap n: (re0 + (-1)^n re10 + sum_k 2 (re_k cos - im_k sin)) / 20 x window[n].
    float* out = p.audio + p.audio_start[b];
    const int jr0 = (int)(s0 + 10 - 5 * f_first);
    const int fmax = (int)(nframes - 1 - f_first);
    for (int ii = threadIdx.x; ii < (int)(s1 - s0); ii += blockDim.x) {
        const int jr = jr0 + ii;
        const int f_lo = f_first > 0 || jr > 19 ? (jr - 15) / 5 : 0;  // first frame with j - 5 f <= 19
        const int f_hi = min(jr / 5, fmax);
        double acc = 0.0, env = 0.0;
        for (int f = f_lo; f <= f_hi; f++) {
            const int n = jr - 5 * f;
            double rv[12], iv[12], cv[10], sv[10];
#pragma unroll
            for (int e = 0; e < 6; e++) {
                const double2 r2 = *(const double2*)&re[f][2 * e], i2 = *(const double2*)&im[f][2 * e];
                rv[2 * e] = r2.x, rv[2 * e + 1] = r2.y, iv[2 * e] = i2.x, iv[2 * e + 1] = i2.y;
            }
#pragma unroll
            for (int e = 0; e < 5; e++) {
                const double2 c2 = *(const double2*)&dft.cs2[n][2 * e], s2 = *(const double2*)&dft.sn2[n][2 * e];
                cv[2 * e] = c2.x, cv[2 * e + 1] = c2.y, sv[2 * e] = s2.x, sv[2 * e + 1] = s2.y;
            }
            double v = rv[0] + ((n & 1) ? -rv[10] : rv[10]);
#pragma unroll
            for (int k = 1; k < 10; k++) v += rv[k] * cv[k - 1] - iv[k] * sv[k - 1];
            v = div20(v);
            const double w = (double)dft.win[n];
            acc += v * w;
            env += w * w;
        }
        out[s0 + ii] = (float)(acc / env);
    }
}

// ------------------------------------------------------------------ PCM_16 (src/wav.rs:63-80)
// v = (s * 32767).round_ties_even() in f32; !(-32768 <= v <= 32767) counts as clipped (NaN
// included); the stored value is v clamped, and NaN casts to 0 as Rust's saturating `as i16`.
__global__ __launch_bounds__(256) void pcm16_kernel(const float* __restrict__ audio,
                                                    const int64_t* __restrict__ audio_start,
                                                    const int64_t* __restrict__ item_len,
                                                    const int64_t* __restrict__ blk_item,
                                                    const int64_t* __restrict__ blk_s0, int16_t* __restrict__ out,
                                                    unsigned long long* __restrict__ clipped) {
    const int64_t blk = blockIdx.x;
    const int b = blk_item ? (int)blk_item[blk] : 0;
    const int64_t s0 = blk_item ? blk_s0[blk] : blk * kIstftSamples;
    const int64_t base = audio_start ? audio_start[b] : 0;
    const int64_t end = min(s0 + kIstftSamples, item_len[b]);
    unsigned n_clip = 0;
    for (int64_t i = s0 + threadIdx.x; i < end; i += blockDim.x) {
        const float v = rintf(__fmul_rn(audio[base + i], 32767.0f));
        const bool in = v >= -32768.0f && v <= 32767.0f;
        n_clip += in ? 0u : 1u;
        out[base + i] = (int16_t)(v != v ? 0.0f : fminf(fmaxf(v, -32768.0f), 32767.0f));
    }
    // block total (integer: the result does not depend on the order), one atomic per block
    for (int o = 32; o > 0; o >>= 1) n_clip += __shfl_xor(n_clip, o, 64);
    __shared__ unsigned part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = n_clip;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned t = part[0] + part[1] + part[2] + part[3];
        if (t) atomicAdd(clipped + b, (unsigned long long)t);
    }
}

__global__ void fill_kernel(uint32_t* p, int64_t n, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

unsigned blocks_for(int64_t n, int per) { return (unsigned)ceil_div(n, per); }

}  // namespace

hipError_t upload_stft_tables(const double* cosv, const double* sinv, const float* win) {
    hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(c_cos), cosv, sizeof(double) * 220);
    if (e != hipSuccess) return e;
    e = hipMemcpyToSymbol(HIP_SYMBOL(c_sin), sinv, sizeof(double) * 220);
    if (e != hipSuccess) return e;
    return hipMemcpyToSymbol(HIP_SYMBOL(c_win), win, sizeof(float) * 20);
}

hipError_t launch_stats_tiles(const float* x, int64_t ld, int c, TilesDev t, StatPart* part, hipStream_t s) {
    if (t.count == 0) return hipSuccess;
    dim3 grid((unsigned)t.count, (unsigned)ceil_div(c, 64));
    hipLaunchKernelGGL(stats_tiles_kernel, grid, dim3(256), 0, s, x, ld, c, t, part);
    return hipGetLastError();
}

hipError_t launch_finalize(const StatPart* part, int c, int wn, TilesDev t, int nb, int64_t max_parts,
                           const float* gb, int64_t gb_ld, const FinOuts& outs, hipStream_t s, const uint16_t* xrow,
                           int64_t xrow_ld, const int64_t* xrow_at) {
    if (outs.n < 1 || outs.n > kFinMaxOuts) return hipErrorInvalidValue;
    dim3 grid((unsigned)nb, (unsigned)ceil_div(c, 16));
    auto go = [&](auto kern, int sub) {
        hipLaunchKernelGGL(kern, grid, dim3(16 * sub), 0, s, part, c, wn, t, gb, gb_ld, outs, xrow, xrow_ld,
                           xrow_at);
        return hipGetLastError();
    };
    if (max_parts <= 16) return go(finalize_kernel<16, 1>, 16);
    if (max_parts <= 64) return go(finalize_kernel<16, 4>, 16);
    if (max_parts <= 128) return go(finalize_kernel<16, 8>, 16);
    if (max_parts <= 256) return go(finalize_kernel<32, 8>, 32);
    return go(finalize_kernel<64, 8>, 64);
}

hipError_t launch_style_fc(const float* w, const float* bias, int rows, const float* style, int nb, float* gb,
                           hipStream_t s) {
    if (rows <= 0 || nb <= 0) return hipSuccess;
    hipLaunchKernelGGL(style_fc_kernel, dim3(blocks_for(rows, 64)), dim3(256), 0, s, w, bias, rows, style, nb, gb);
    return hipGetLastError();
}

hipError_t launch_expand(const float* t_en, int64_t t_rows, const int32_t* src_row, int64_t l, float* asr, int64_t ld,
                         hipStream_t s) {
    hipLaunchKernelGGL(expand_kernel, dim3(blocks_for(l * 512, 256)), dim3(256), 0, s, t_en, t_rows, src_row, l, asr,
                       ld);
    return hipGetLastError();
}

hipError_t launch_f0n_conv(const float* f0, const float* en, int64_t l2, const float* w_f0, const float* b_f0,
                           const float* w_n, const float* b_n, float* out, int64_t ld, int col_f0, int col_n,
                           const int32_t* col, int64_t ln, hipStream_t s) {
    hipLaunchKernelGGL(f0n_kernel, dim3(blocks_for(ln, 256)), dim3(256), 0, s, f0, en, l2, w_f0, b_f0, w_n, b_n, out,
                       ld, col_f0, col_n, col, ln);
    return hipGetLastError();
}

hipError_t launch_copy_cols(const float* src, int64_t src_ld, int c, float* dst, int64_t dst_ld, int dst_c0,
                            const int32_t* col, int64_t l, hipStream_t s) {
    if (l <= 0 || c <= 0) return hipSuccess;
    hipLaunchKernelGGL(copy_cols_kernel, dim3((unsigned)l), dim3(256), 0, s, src, src_ld, c, dst, dst_ld, dst_c0, col, l);
    return hipGetLastError();
}

hipError_t launch_adain_pool(const float* x, int64_t ld, int c, const Coef* coef, const int32_t* col_n, int64_t ln,
                             const float* pw, const float* pb, const int32_t* col_2, uint16_t* out, int64_t out_ld,
                             hipStream_t s) {
    if (ln <= 0) return hipSuccess;
    // channel pairs: float2 / two-Coef / bf16x2 accesses need even widths and leading dimensions
    if ((c | ld | out_ld) & 1 || c > out_ld) return hipErrorInvalidValue;
    hipLaunchKernelGGL(adain_pool_kernel, dim3((unsigned)(2 * ln)), dim3(256), 0, s, x, ld, c, coef, col_n, ln, pw, pb,
                       col_2, out, out_ld);
    return hipGetLastError();
}

hipError_t launch_noise_conv(const float* spec, int64_t spec_ld, int64_t l_in, const int64_t* in_start,
                             const int64_t* in_len, const uint16_t* wp, const float* b, int cout, int k, int stride,
                             int pad, uint16_t* y, int64_t y_ld, TilesDev t, int tile_rows, StatPart* part,
                             hipStream_t s) {
    if (!wp) return hipErrorInvalidValue;
    if (t.count == 0) return hipSuccess;
    const dim3 grid((unsigned)t.count);
    if (cout == 256 && k == 12 && stride == 6) {
        if (tile_rows != kNoiseTile) return hipErrorInvalidValue;
        hipLaunchKernelGGL(noise_conv0_mfma_kernel, grid, dim3(256), 0, s, spec, spec_ld, l_in, in_start, in_len,
                           (const bf16x8*)wp, b, pad, y, y_ld, t, part);
    } else if (cout == 128 && k == 1 && stride == 1 && pad == 0) {
        // output rows are input rows: every row of a tile lies inside its item
        if (tile_rows != kNoiseTile1 || y_ld != 128) return hipErrorInvalidValue;
        hipLaunchKernelGGL(noise_conv1_mfma_kernel, grid, dim3(256), 0, s, spec, spec_ld, (const bf16x8*)wp, b, y, y_ld,
                           t, part);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_phase_pre(const float* f0, const int64_t* start2, const int64_t* len2, int nb, const float* rand_ini,
                            float* pp, int64_t pp_ld, hipStream_t s) {
    hipLaunchKernelGGL(phase_pre_kernel, dim3(nb * kHarmonics), dim3(256), 0, s, f0, start2, len2, rand_ini, pp, pp_ld);
    return hipGetLastError();
}

hipError_t launch_source_stft(const SourceParams& p, hipStream_t s) {
    hipLaunchKernelGGL(source_stft_kernel, dim3((unsigned)p.n_blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_istft(const IstftParams& p, hipStream_t s) {
    hipLaunchKernelGGL(istft_kernel, dim3((unsigned)p.n_blocks), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_pcm16(const float* audio, const int64_t* audio_start, const int64_t* item_len,
                        const int64_t* blk_item, const int64_t* blk_s0, int64_t n_blocks, int16_t* out,
                        unsigned long long* clipped, hipStream_t s) {
    if (n_blocks <= 0) return hipSuccess;
    hipLaunchKernelGGL(pcm16_kernel, dim3((unsigned)n_blocks), dim3(256), 0, s, audio, audio_start, item_len,
                       blk_item, blk_s0, out, clipped);
    return hipGetLastError();
}

hipError_t launch_fill(void* p, int64_t bytes, uint32_t value, hipStream_t s) {
    const int64_t n = bytes / 4;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, (uint32_t*)p, n, value);
    return hipGetLastError();
}

hipError_t launch_zero(void* p, int64_t bytes, hipStream_t s) { return launch_fill(p, bytes, 0u, s); }

}  // namespace kk
