// kk_conv.hip -- bf16 implicit-GEMM convolution on CDNA4 MFMA (v_mfma_f32_16x16x32_bf16).
//
// One kernel family serves every MFMA layer of the path:
//   * stride-1 Conv1d with any K / dilation (decoder conv1/conv2/conv1x1/asr_res, the 48 Snake-block
//     convs, conv_post) -- the reference's conv1d_wmma_bf16[_snake[_res]] and per-tap cuBLAS
//     routes (src/gpu.rs:331-499, kernels/kokoro.cu:660-774);
//   * ConvTranspose1d with K = 2*stride as a polyphase 2-tap conv whose GEMM rows are
//     (phase, out-channel) pairs (replaces the f32 sgemm + convT_gather of src/gpu.rs:527-537).
//
// GEMM view: M = output channels (x phases), N = time columns, K = input channels x taps.
// * Blocks run over item-aligned tiles (kk_kernels.h TilesDev): a tile never mixes items, so the
//   per-item zero padding of the reference's gap masking (src/gpu_batch.rs:62-79) is a row-range
//   test and the AdaIN coefficients are constants of the block.
// * A (weights) is pre-packed as [tap][cin/32][M_pad][32] bf16: one A fragment (16 rows x 32
//   channels) is a contiguous 1 KB, loaded straight into registers one (tap, 32-channel) step
//   ahead of its use.
// * B (activations) is staged per 64-channel slab into LDS as [time][64 + 8 pad] bf16 (144-byte
//   rows: a 16-lane B-fragment read touches distinct banks); every tap reads the same slab at a
//   row offset.  The layer's prologue (AdaIN affine + Snake or leaky ReLU, f32 -> bf16 with the
//   hardware round-to-nearest-even convert) runs once per staged element.
// * Warp specialization: half of a block's waves are producers, half consumers.  Producers stage
//   (global loads + prologue VALU) the next 64-channel slab into one of two LDS buffers while the
//   consumers run the MFMAs of the current slab from the other, so VALU and MFMA co-execute on
//   every SIMD.  Blocks are persistent: each walks a strided list of (tile, M-block) units, and the
//   slab stream runs across unit boundaries, so the epilogue of one unit overlaps the staging of
//   the next.
// * Each consumer wave owns a 64 x 128 output tile (4 x 8 MFMA tiles, 128 accumulator registers);
//   A fragments are prefetched two (tap, 32-channel) steps ahead, across slab and unit boundaries.
// * The epilogue adds the bias, applies the layer's residual rule in f32 and, when asked, reduces
//   the instance-norm statistics of the values it stores: per (tile, wave, channel) sums of
//   (v - v_first), written to a partials buffer that finalize combines in a fixed order.
// * The Snake blocks' conv1 output (input of conv2's AdaIN) is stored as fp16 (PRO_*_H / EPI_STORE_H):
//   half the HBM traffic of f32, 8x the precision of bf16 operands; the residual stream stays f32.
#include "kk_common.h"
#include "kk_kernels.h"

#include <algorithm>

namespace kk {

namespace {

constexpr int kCK = 64;       // input channels staged per slab
constexpr int kRS = kCK + 8;  // LDS row stride (bf16 elements)
constexpr int kNJ = 8;        // 16-column MFMA tiles per wave (wave N = 128)

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const bf16x2_t v = __builtin_convertvector((f32x2_t){a, b}, bf16x2_t);  // v_cvt_pk_bf16_f32 (RNE)
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float snake(float v, float a_rev, float a_inv) {
    // v + sin^2(alpha v) / alpha; __builtin_amdgcn_sinf(x) = sin(2 pi x), so a_rev = alpha / (2 pi).
    const float s = __builtin_amdgcn_sinf(v * a_rev);
    return __builtin_fmaf(s * s, a_inv, v);
}

// Stage rows [in0, in0 + tw) x channels [c0, c0 + 64) of the input into LDS as bf16, applying the
// prologue.  Producer thread pt owns channel octet (pt % 8) of rows pt / 8, pt / 8 + NP / 8, ...;
// RB rows' global loads are issued before any of them is converted.
template <int PRO, bool IN_H, int NP>
__device__ __forceinline__ void stage_slab(const ConvParams& p, uint16_t* xs, int64_t in0, int tw, int c0,
                                           int64_t i_lo, int64_t i_hi, int item, int pt) {
    const int q = (pt & 7) * 8;
    const int c = c0 + q;
    constexpr int RP = NP / 8;  // rows per pass
    constexpr int RB = NP >= 256 ? 10 : 9;
    if constexpr (PRO == PRO_BF16) {
        const uint16_t* x = (const uint16_t*)p.x;
        for (int r = pt >> 3; r < tw; r += RP) {
            const int64_t row = in0 + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row >= i_lo && row < i_hi) v = *(const uint4*)(x + row * p.x_ld + c);
            *(uint4*)(xs + r * kRS + q) = v;
        }
        return;
    } else {
        // per-thread constants of this slab: AdaIN coefficients of the unit's item, Snake alphas
        float sc[8], sh[8], ar[8], ai[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const bool live = c + e < p.cin;
            sc[e] = 1.f, sh[e] = 0.f, ar[e] = 0.f, ai[e] = 0.f;
            if constexpr (PRO == PRO_ADAIN_LEAKY || PRO == PRO_ADAIN_SNAKE) {
                if (live) {
                    const Coef k = p.coef[(int64_t)item * p.cin + c + e];
                    sc[e] = k.sc, sh[e] = k.sh;
                }
            }
            if constexpr (PRO == PRO_ADAIN_SNAKE) {
                if (live) ar[e] = p.alpha_rev[c + e], ai[e] = p.alpha_inv[c + e];
            }
        }
        for (int rb = pt >> 3; rb < tw; rb += RB * RP) {
            float v[RB][8];
            bool ok[RB];
#pragma unroll
            for (int j = 0; j < RB; j++) {
                const int r = rb + j * RP;
                const int64_t row = in0 + r;
                ok[j] = r < tw && row >= i_lo && row < i_hi && c < p.cin;
                if constexpr (IN_H) {
                    uint4 h = make_uint4(0, 0, 0, 0);
                    if (ok[j]) h = *(const uint4*)((const uint16_t*)p.x + row * p.x_ld + c);
                    const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const _Float16 lo = __builtin_bit_cast(_Float16, (uint16_t)(hw[e] & 0xffffu));
                        const _Float16 hi = __builtin_bit_cast(_Float16, (uint16_t)(hw[e] >> 16));
                        v[j][2 * e] = (float)lo, v[j][2 * e + 1] = (float)hi;
                    }
                } else {
                    float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
                    if (ok[j]) {
                        const float* xp = (const float*)p.x + row * p.x_ld + c;
                        x0 = *(const float4*)xp;
                        x1 = *(const float4*)(xp + 4);
                    }
                    v[j][0] = x0.x, v[j][1] = x0.y, v[j][2] = x0.z, v[j][3] = x0.w;
                    v[j][4] = x1.x, v[j][5] = x1.y, v[j][6] = x1.z, v[j][7] = x1.w;
                }
            }
#pragma unroll
            for (int j = 0; j < RB; j++) {
                const int r = rb + j * RP;
                if (r >= tw) break;
                uint4 out = make_uint4(0, 0, 0, 0);
                if (ok[j]) {
                    float u[8];
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        float w = v[j][e];
                        if constexpr (PRO == PRO_LEAKY) {
                            w = w < 0.f ? w * p.slope : w;
                        } else if constexpr (PRO == PRO_ADAIN_LEAKY) {
                            w = __builtin_fmaf(w, sc[e], sh[e]);
                            w = w < 0.f ? w * p.slope : w;
                        } else if constexpr (PRO == PRO_ADAIN_SNAKE) {
                            w = snake(__builtin_fmaf(w, sc[e], sh[e]), ar[e], ai[e]);
                        }
                        u[e] = c + e < p.cin ? w : 0.f;
                    }
                    out.x = pack_bf16x2(u[0], u[1]);
                    out.y = pack_bf16x2(u[2], u[3]);
                    out.z = pack_bf16x2(u[4], u[5]);
                    out.w = pack_bf16x2(u[6], u[7]);
                }
                *(uint4*)(xs + r * kRS + q) = out;
            }
        }
    }
}

// Store 4 consecutive GEMM rows m..m+3 of GEMM column t; returns the stored values (statistics).
template <int EPI, bool OUT_H>
__device__ __forceinline__ float4 store4(const ConvParams& p, int item, int64_t t, int m, float4 v) {
    if constexpr (EPI == EPI_CONVT || EPI == EPI_CONVT_REFLECT) {
        const int ph = m / p.cout, co = m - ph * p.cout;
        const int64_t o = (int64_t)p.stride_t * t + ph - p.pad_t;  // ConvT output column
        const int64_t os = p.out_start[item];
        const int64_t ol = EPI == EPI_CONVT ? p.out_len[item] : p.out_len[item] - 1;
        if (o < os || o >= os + ol) return v;
        const float4 b = *(const float4*)(p.bias + co);
        v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
        // EPI_CONVT_REFLECT: ReflectionPad1d((1,0)) per item on the padded domain
        // (kernels/kokoro.cu:452-467): padded[s] = ups[s + 1], padded[s + 1 + j] = ups[s + j].
        const int64_t dest = EPI == EPI_CONVT ? o : o + 1;
        const float4 r = *(const float4*)(p.r0 + dest * p.r0_ld + co);
        *(float4*)(p.y + dest * p.y_ld + co) = make_float4(v.x + r.x, v.y + r.y, v.z + r.z, v.w + r.w);
        if (EPI == EPI_CONVT_REFLECT && o == os + 1) {
            const float4 r2 = *(const float4*)(p.r0 + os * p.r0_ld + co);
            *(float4*)(p.y + os * p.y_ld + co) = make_float4(v.x + r2.x, v.y + r2.y, v.z + r2.z, v.w + r2.w);
        }
        return v;
    } else {
        const float4 b = p.bias ? *(const float4*)(p.bias + m) : make_float4(0.f, 0.f, 0.f, 0.f);
        v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
        if constexpr (OUT_H) {
            // fp16 storage; the statistics describe the rounded values the next layer reads
            const _Float16 h0 = (_Float16)v.x, h1 = (_Float16)v.y, h2 = (_Float16)v.z, h3 = (_Float16)v.w;
            uint2 pk;
            pk.x = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            pk.y = (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16);
            *(uint2*)((uint16_t*)p.y + t * p.y_ld + m) = pk;
            return make_float4((float)h0, (float)h1, (float)h2, (float)h3);
        }
        float* dst = p.y + t * p.y_ld + m;
        float4 o = v;
        if constexpr (EPI == EPI_ACCUM) {
            const float4 y = *(const float4*)dst;
            o = make_float4(y.x + v.x, y.y + v.y, y.z + v.z, y.w + v.w);
        } else if constexpr (EPI == EPI_RESID) {
            const float4 y = *(const float4*)dst;
            const float s = p.scale;
            o = make_float4((v.x + y.x) * s, (v.y + y.y) * s, (v.z + y.z) * s, (v.w + y.w) * s);
        } else if constexpr (EPI == EPI_RESID_UP2) {
            const float4 y = *(const float4*)(p.r0 + (t >> 1) * p.r0_ld + m);
            const float s = p.scale;
            o = make_float4((v.x + y.x) * s, (v.y + y.y) * s, (v.z + y.z) * s, (v.w + y.w) * s);
        } else if constexpr (EPI == EPI_ADD_FROM) {
            const float4 y = *(const float4*)(p.r0 + t * p.r0_ld + m);
            o = make_float4(y.x + v.x, y.y + v.y, y.z + v.z, y.w + v.w);
        } else if constexpr (EPI == EPI_MEAN3) {
            // ((rb0 + rb1) + (rb2_resid + conv)) / 3   (src/gpu_batch.rs:395-401)
            const float4 a = *(const float4*)(p.r0 + t * p.r0_ld + m);
            const float4 b1 = *(const float4*)(p.r1 + t * p.r0_ld + m);
            const float4 c = *(const float4*)(p.r2 + t * p.r0_ld + m);
            o = make_float4(((a.x + b1.x) + (c.x + v.x)) / 3.0f, ((a.y + b1.y) + (c.y + v.y)) / 3.0f,
                            ((a.z + b1.z) + (c.z + v.z)) / 3.0f, ((a.w + b1.w) + (c.w + v.w)) / 3.0f);
        }
        *(float4*)dst = o;
        return o;
    }
}

// Sum over the 16 lanes of a DPP row (row_ror 1, 2, 4, 8): every lane of the row gets the total.
__device__ __forceinline__ float row_sum16(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
    return v;
}

template <int PRO, int EPI, int WM, int WN, bool STATS, bool IN_H, bool OUT_H>
__global__ __launch_bounds__(128 * WM * WN) void conv_mfma_kernel(ConvParams p) {
    constexpr int BM = 64 * WM, BN = 16 * kNJ * WN, NC = 64 * WM * WN;
    extern __shared__ __align__(16) uint16_t xs[];
    const int tw = BN + (p.k - 1) * p.dil;
    const int slab_elems = tw * kRS;
    const int nslab = p.cin_pad / kCK;
    const int mblocks = p.m_pad / BM;
    const int64_t units = p.tiles.count * mblocks;
    const int64_t my_units = units > blockIdx.x ? (units - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    const int64_t steps = my_units * nslab;
    auto unit_of = [&](int64_t g) { return (int64_t)blockIdx.x + (g / nslab) * gridDim.x; };

    if (threadIdx.x >= NC) {
        // ------------------------------------------------------------ producer waves
        const int pt = threadIdx.x - NC;
        auto stage = [&](int64_t g) {
            const int64_t u = unit_of(g);
            const int64_t tile = u / mblocks;
            const int item = p.tiles.item[tile];
            const int64_t i_lo = p.in_start[item], i_hi = i_lo + p.in_len[item];
            stage_slab<PRO, IN_H, NC>(p, xs + (g & 1) * slab_elems, p.tiles.t0[tile] - p.pad, tw,
                                      (int)(g % nslab) * kCK, i_lo, i_hi, item, pt);
        };
        if (steps > 0) stage(0);
        __syncthreads();
        for (int64_t g = 0; g < steps; g++) {
            if (g + 1 < steps) stage(g + 1);
            __syncthreads();
        }
        return;
    }

    // ---------------------------------------------------------------- consumer waves
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave % WM, wn = wave / WM;
    const int lr = lane & 15, lg = lane >> 4;
    const int ncc = p.cin_pad >> 5;
    const int64_t total = steps * p.k;  // flattened (slab step, tap) stream
    const int64_t a_step = (int64_t)p.m_pad * 4;
    // A fragments of flattened iteration f = g * k + tap: [half cs][i] for the unit's M block and slab
    bf16x8 a_cur[2][4], a_nxt[2][4];
    auto load_a = [&](bf16x8 (&dst)[2][4], int64_t f) {
        if (f >= total) return;
        const int64_t g = f / p.k;
        const int kk = (int)(f - g * p.k);
        const int mb = (int)(unit_of(g) % mblocks);
        const bf16x8* ap = (const bf16x8*)p.w + (int64_t)(mb * BM + wm * 64 + lr) * 4 + lg +
                           ((int64_t)kk * ncc + (g % nslab) * 2) * a_step;
#pragma unroll
        for (int cs = 0; cs < 2; cs++)
#pragma unroll
            for (int i = 0; i < 4; i++) dst[cs][i] = ap[cs * a_step + i * 64];
    };
    f32x4 acc[4][kNJ];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < kNJ; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    load_a(a_cur, 0);
    __syncthreads();  // slab 0 staged
    for (int64_t g = 0; g < steps; g++) {
        const uint16_t* buf = xs + (g & 1) * slab_elems;
        for (int kk = 0; kk < p.k; kk++) {
            load_a(a_nxt, g * p.k + kk + 1);  // one tap ahead, across slab and unit boundaries
            const int rb = wn * 128 + kk * p.dil + lr;
#pragma unroll
            for (int cs = 0; cs < 2; cs++) {
                const int col = cs * 32 + lg * 8;
#pragma unroll
                for (int j = 0; j < kNJ; j += 2) {
                    const bf16x8 b0 = *(const bf16x8*)(buf + (rb + j * 16) * kRS + col);
                    const bf16x8 b1 = *(const bf16x8*)(buf + (rb + j * 16 + 16) * kRS + col);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_cur[cs][i], b0, acc[i][j], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[i][j + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_cur[cs][i], b1, acc[i][j + 1], 0, 0, 0);
                }
            }
#pragma unroll
            for (int cs = 0; cs < 2; cs++)
#pragma unroll
                for (int i = 0; i < 4; i++) a_cur[cs][i] = a_nxt[cs][i];
        }
        if (g % nslab == nslab - 1) {
            // the unit's last slab: epilogue, then fresh accumulators for the next unit
            const int64_t u = unit_of(g);
            const int64_t tile = u / mblocks;
            const int m0 = (int)(u % mblocks) * BM;
            const int item = p.tiles.item[tile];
            const int64_t n0 = p.tiles.t0[tile];
            const int nv = p.tiles.n[tile];
            // D[i][j] lane layout: row (output channel) = 4 * (lane / 16) + r, column = lane % 16.
            const int wcol0 = wn * 128;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + wm * 64 + i * 16 + lg * 4;
                float s1[4] = {0.f, 0.f, 0.f, 0.f}, s2[4] = {0.f, 0.f, 0.f, 0.f}, sft[4];
#pragma unroll
                for (int j = 0; j < kNJ; j++) {
                    const int col = wcol0 + j * 16 + lr;
                    const bool valid = col < nv;
                    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (valid && m < p.m)
                        o = store4<EPI, OUT_H>(p, item, n0 + col, m,
                                               make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]));
                    acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
                    if constexpr (STATS) {
                        const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            if (j == 0) sft[r] = __shfl(ov[r], lane & 48, 64);  // the wave's first column
                            const float d = valid ? ov[r] - sft[r] : 0.f;
                            s1[r] += d;
                            s2[r] = __builtin_fmaf(d, d, s2[r]);
                        }
                    }
                }
                if constexpr (STATS) {
                    if (wcol0 < nv) {
                        StatPart* dst = p.part + (tile * WN + wn) * (int64_t)p.cout;
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const float sa = row_sum16(s1[r]);
                            const float sb = row_sum16(s2[r]);
                            if (lr == 0 && m + r < p.cout) dst[m + r] = StatPart{sa, sb, sft[r]};
                        }
                    }
                }
            }
        }
        __syncthreads();  // hand the slab buffer back to the producers
    }
}

template <int PRO, int EPI, int WM, int WN, bool STATS, bool IN_H, bool OUT_H>
hipError_t launch_t(const ConvParams& p, int n_cu, hipStream_t s) {
    constexpr int BM = 64 * WM, BN = 16 * kNJ * WN;
    const int tw = BN + (p.k - 1) * p.dil;
    const size_t smem = 2 * (size_t)tw * kRS * sizeof(uint16_t);
    if (p.m_pad % BM != 0 || p.cin_pad % kCK != 0 || smem > 160 * 1024) return hipErrorInvalidValue;
    auto kern = conv_mfma_kernel<PRO, EPI, WM, WN, STATS, IN_H, OUT_H>;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return e;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, 128 * WM * WN, smem);
    if (e != hipSuccess) return e;
    if (per_cu < 1) return hipErrorInvalidConfiguration;
    const int64_t units = p.tiles.count * (p.m_pad / BM);
    const int64_t grid = std::min<int64_t>(units, (int64_t)per_cu * n_cu);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(128 * WM * WN), smem, s, p);
    return hipGetLastError();
}

}  // namespace

// The (prologue, epilogue, block shape, statistics, fp16 in/out) combinations the engine uses;
// anything else is refused.
hipError_t launch_conv(const ConvParams& p, int pro, int epi, int shape, bool stats, bool in_h, bool out_h, int n_cu,
                       hipStream_t s) {
    if (p.tiles.count == 0) return hipSuccess;
#define KK_CONV(P, E, SH, WM, WN, ST, IH, OH)                                              \
    if (pro == P && epi == E && shape == SH && stats == ST && in_h == IH && out_h == OH) \
        return launch_t<P, E, WM, WN, ST, IH, OH>(p, n_cu, s);
    // Snake blocks, 256 ch (stage 0) and 128 ch (stage 1): conv1 X (f32) -> h (fp16) with statistics;
    // conv2 h -> X (ACCUM / ADD_FROM with statistics, last step without; MEAN3)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, SHAPE_256x128, 4, 1, true, false, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_256x128, 4, 1, true, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_256x128, 4, 1, false, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ADD_FROM, SHAPE_256x128, 4, 1, true, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_MEAN3, SHAPE_256x128, 4, 1, false, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, SHAPE_128x256, 2, 2, true, false, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_128x256, 2, 2, true, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_128x256, 2, 2, false, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ADD_FROM, SHAPE_128x256, 2, 2, true, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_MEAN3, SHAPE_128x256, 2, 2, false, true, false)
    // decoder
    KK_CONV(PRO_ADAIN_LEAKY, EPI_STORE, SHAPE_256x128, 4, 1, true, false, false)
    KK_CONV(PRO_ADAIN_LEAKY, EPI_RESID, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_ADAIN_LEAKY, EPI_RESID_UP2, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_F32, EPI_STORE, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_F32, EPI_STORE, SHAPE_64x256, 1, 2, false, false, false)
    KK_CONV(PRO_BF16, EPI_STORE, SHAPE_256x128, 4, 1, true, false, false)
    // ConvT ups and conv_post
    KK_CONV(PRO_LEAKY, EPI_CONVT, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_LEAKY, EPI_CONVT_REFLECT, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_LEAKY, EPI_STORE, SHAPE_64x256, 1, 2, false, false, false)
#undef KK_CONV
    return hipErrorInvalidValue;
}

}  // namespace kk
