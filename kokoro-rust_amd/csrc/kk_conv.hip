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
// A (weights) is pre-packed at upload as [tap][cin/32][M_pad][32] bf16 so one A fragment
// (16 rows x 32 channels) is a contiguous 1 KB; B (activations) is staged per 64-channel slab into
// LDS as [time][64 + 8 pad] bf16 (144-byte rows: a 16-lane B-fragment read touches 64 distinct
// banks), with the layer's prologue (AdaIN affine + Snake or leaky ReLU, gap masking, f32 -> bf16)
// applied once per staged element.  Each wave owns a 64 x 64 output tile (4 x 4 MFMA tiles, 64
// accumulator registers); a block is WM x WN waves.  Accumulation is f32; the epilogue adds the
// bias and applies the layer's residual rule in f32.
#include "kk_common.h"
#include "kk_kernels.h"

namespace kk {

namespace {

constexpr int kCK = 64;        // input channels staged per slab
constexpr int kRS = kCK + 8;   // LDS row stride (bf16 elements)

__device__ __forceinline__ float snake(float v, float a_rev, float a_inv) {
    // v + sin^2(alpha v) / alpha; __builtin_amdgcn_sinf(x) = sin(2 pi x), so a_rev = alpha / (2 pi).
    float s = __builtin_amdgcn_sinf(v * a_rev);
    return __builtin_fmaf(s * s, a_inv, v);
}

template <int PRO>
__device__ __forceinline__ void stage_slab(const ConvParams& p, uint16_t* xs, int64_t in0, int tw, int c0) {
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    if constexpr (PRO == PRO_BF16) {
        // 8 channels (16 B) per load; 8 loads per 64-channel row
        const uint16_t* x = (const uint16_t*)p.x;
        for (int i = tid; i < tw * 8; i += nthr) {
            int r = i >> 3, q = (i & 7) * 8;
            int64_t row = in0 + r;
            uint4 v = make_uint4(0, 0, 0, 0);
            bool ok = row >= 0 && row < p.l_in && c0 + q < p.cin_pad;
            if (ok && p.col_in) ok = p.col_in[row] >= 0;
            if (ok) v = *(const uint4*)(x + row * p.x_ld + c0 + q);
            *(uint4*)(xs + r * kRS + q) = v;
        }
    } else {
        // f32 input, 4 channels (16 B) per load; 16 loads per 64-channel row
        const float* x = (const float*)p.x;
        for (int i = tid; i < tw * 16; i += nthr) {
            int r = i >> 4, q = (i & 15) * 4;
            int64_t row = in0 + r;
            int c = c0 + q;
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            int item = 0;
            bool ok = row >= 0 && row < p.l_in;
            if (ok && p.col_in) {
                item = p.col_in[row];
                ok = item >= 0;
            }
            if (ok && c < p.cin) {
                float4 xv = *(const float4*)(x + row * p.x_ld + c);
                v[0] = xv.x, v[1] = xv.y, v[2] = xv.z, v[3] = xv.w;
                if constexpr (PRO == PRO_LEAKY) {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = v[e] < 0.f ? v[e] * p.slope : v[e];
                } else if constexpr (PRO == PRO_ADAIN_LEAKY || PRO == PRO_ADAIN_SNAKE) {
                    const Coef* cf = p.coef + (int64_t)item * p.cin + c;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        Coef k = cf[e];
                        float u = __builtin_fmaf(v[e], k.sc, k.sh);
                        if constexpr (PRO == PRO_ADAIN_LEAKY) {
                            u = u < 0.f ? u * p.slope : u;
                        } else {
                            u = snake(u, p.alpha_rev[c + e], p.alpha_inv[c + e]);
                        }
                        v[e] = u;
                    }
                }
                // channels beyond cin inside this float4 are zero
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (c + e >= p.cin) v[e] = 0.f;
            }
            uint2 packed;
            packed.x = (uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
            packed.y = (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
            *(uint2*)(xs + r * kRS + q) = packed;
        }
    }
}

template <int EPI>
__device__ __forceinline__ void store4(const ConvParams& p, int64_t t, int m, float4 v) {
    if constexpr (EPI == EPI_CONVT || EPI == EPI_CONVT_REFLECT) {
        const int ph = m / p.cout, co = m - ph * p.cout;
        const int64_t o = (int64_t)p.stride_t * t + ph - p.pad_t;  // ConvT output column
        if (o < 0 || o >= p.l_convt) return;
        float4 b = *(const float4*)(p.bias + co);
        v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
        if constexpr (EPI == EPI_CONVT) {
            float4 r = *(const float4*)(p.r0 + o * p.r0_ld + co);
            v.x += r.x, v.y += r.y, v.z += r.z, v.w += r.w;
            *(float4*)(p.y + o * p.y_ld + co) = v;
        } else {
            // ReflectionPad1d((1,0)) per item on the padded domain (kernels/kokoro.cu:452-467):
            // padded[s_b] = ups[s_b + 1], padded[s_b + 1 + j] = ups[s_b + j]; then += xs.
            const int64_t dest = o + 1;
            const int32_t bd = p.col_out[dest];
            if (bd < 0) {
                *(float4*)(p.y + dest * p.y_ld + co) = make_float4(0.f, 0.f, 0.f, 0.f);
            } else if (o >= p.start_out[bd]) {
                float4 r = *(const float4*)(p.r0 + dest * p.r0_ld + co);
                *(float4*)(p.y + dest * p.y_ld + co) = make_float4(v.x + r.x, v.y + r.y, v.z + r.z, v.w + r.w);
            }
            const int32_t bo = p.col_out[o];
            if (bo >= 0 && o == p.start_out[bo] + 1) {
                const int64_t s = p.start_out[bo];
                float4 r = *(const float4*)(p.r0 + s * p.r0_ld + co);
                *(float4*)(p.y + s * p.y_ld + co) = make_float4(v.x + r.x, v.y + r.y, v.z + r.z, v.w + r.w);
            }
        }
        return;
    } else {
        if (m >= p.cout) return;
        float4 b = p.bias ? *(const float4*)(p.bias + m) : make_float4(0.f, 0.f, 0.f, 0.f);
        v.x += b.x, v.y += b.y, v.z += b.z, v.w += b.w;
        float* dst = p.y + t * p.y_ld + m;
        if constexpr (EPI == EPI_STORE) {
            *(float4*)dst = v;
        } else if constexpr (EPI == EPI_ACCUM) {
            float4 y = *(const float4*)dst;
            *(float4*)dst = make_float4(y.x + v.x, y.y + v.y, y.z + v.z, y.w + v.w);
        } else if constexpr (EPI == EPI_RESID) {
            float4 y = *(const float4*)dst;
            const float s = p.scale;
            *(float4*)dst = make_float4((v.x + y.x) * s, (v.y + y.y) * s, (v.z + y.z) * s, (v.w + y.w) * s);
        } else if constexpr (EPI == EPI_RESID_UP2) {
            float4 y = *(const float4*)(p.r0 + (t >> 1) * p.r0_ld + m);
            const float s = p.scale;
            *(float4*)dst = make_float4((v.x + y.x) * s, (v.y + y.y) * s, (v.z + y.z) * s, (v.w + y.w) * s);
        } else if constexpr (EPI == EPI_ADD_FROM) {
            float4 y = *(const float4*)(p.r0 + t * p.r0_ld + m);
            *(float4*)dst = make_float4(y.x + v.x, y.y + v.y, y.z + v.z, y.w + v.w);
        } else if constexpr (EPI == EPI_MEAN3) {
            // ((rb0 + rb1) + (rb2_resid + conv)) / 3   (src/gpu_batch.rs:395-401)
            float4 a = *(const float4*)(p.r0 + t * p.r0_ld + m);
            float4 b1 = *(const float4*)(p.r1 + t * p.r0_ld + m);
            float4 c = *(const float4*)(p.r2 + t * p.r0_ld + m);
            *(float4*)dst = make_float4(((a.x + b1.x) + (c.x + v.x)) / 3.0f, ((a.y + b1.y) + (c.y + v.y)) / 3.0f,
                                        ((a.z + b1.z) + (c.z + v.z)) / 3.0f, ((a.w + b1.w) + (c.w + v.w)) / 3.0f);
        }
    }
}

template <int PRO, int EPI, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN) void conv_mfma_kernel(ConvParams p) {
    constexpr int BM = 64 * WM, BN = 64 * WN;
    extern __shared__ __align__(16) uint16_t xs[];
    const int tw = BN + (p.k - 1) * p.dil;
    const int64_t n0 = (int64_t)blockIdx.x * BN;
    const int m0 = blockIdx.y * BM;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave % WM, wn = wave / WM;
    const int lr = lane & 15, lg = lane >> 4;
    const int ncc = p.cin_pad >> 5;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    const int64_t in0 = n0 - p.pad;
    for (int c0 = 0; c0 < p.cin_pad; c0 += kCK) {
        __syncthreads();
        stage_slab<PRO>(p, xs, in0, tw, c0);
        __syncthreads();
        for (int kk = 0; kk < p.k; kk++) {
            const int rb = wn * 64 + kk * p.dil + lr;
#pragma unroll
            for (int cs = 0; cs < 2; cs++) {
                const int cc = (c0 >> 5) + cs;
                const bf16x8* wp =
                    (const bf16x8*)(p.w + (((int64_t)kk * ncc + cc) * p.m_pad + m0 + wm * 64) * 32);
                bf16x8 a[4], b[4];
#pragma unroll
                for (int i = 0; i < 4; i++) a[i] = wp[(i * 16 + lr) * 4 + lg];
#pragma unroll
                for (int j = 0; j < 4; j++) b[j] = *(const bf16x8*)(xs + (rb + j * 16) * kRS + cs * 32 + lg * 8);
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
        }
    }

    // D[i][j] lane layout: row (output channel) = 4 * (lane / 16) + r, column (time) = lane % 16.
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int64_t t = n0 + wn * 64 + j * 16 + lr;
        if (t >= p.n_out) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = m0 + wm * 64 + i * 16 + lg * 4;
            if (m >= p.m) continue;
            store4<EPI>(p, t, m, make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]));
        }
    }
}

template <int PRO, int EPI, int WM, int WN>
hipError_t launch_t(const ConvParams& p, hipStream_t s) {
    constexpr int BM = 64 * WM, BN = 64 * WN;
    const int tw = BN + (p.k - 1) * p.dil;
    const size_t smem = (size_t)tw * kRS * sizeof(uint16_t);
    dim3 grid((unsigned)ceil_div(p.n_out, BN), (unsigned)(p.m_pad / BM));
    hipLaunchKernelGGL((conv_mfma_kernel<PRO, EPI, WM, WN>), grid, dim3(64 * WM * WN), smem, s, p);
    return hipGetLastError();
}

}  // namespace

int conv_block_m(int shape) { return shape == SHAPE_W4x2 ? 256 : shape == SHAPE_W2x4 ? 128 : 64; }
int conv_block_n(int shape) { return shape == SHAPE_W4x2 ? 128 : 256; }

// The (prologue, epilogue, block shape) combinations the engine uses; anything else is refused.
hipError_t launch_conv(const ConvParams& p, int pro, int epi, int shape, hipStream_t s) {
#define KK_CONV(P, E, WM, WN)                                                                       \
    if (pro == P && epi == E && shape == (WM == 4 ? SHAPE_W4x2 : WM == 2 ? SHAPE_W2x4 : SHAPE_W1x4)) \
        return launch_t<P, E, WM, WN>(p, s);
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, 4, 2)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, 4, 2)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ADD_FROM, 4, 2)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_MEAN3, 4, 2)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, 2, 4)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, 2, 4)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ADD_FROM, 2, 4)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_MEAN3, 2, 4)
    KK_CONV(PRO_ADAIN_LEAKY, EPI_STORE, 4, 2)
    KK_CONV(PRO_ADAIN_LEAKY, EPI_RESID, 4, 2)
    KK_CONV(PRO_ADAIN_LEAKY, EPI_RESID_UP2, 4, 2)
    KK_CONV(PRO_F32, EPI_STORE, 4, 2)
    KK_CONV(PRO_F32, EPI_STORE, 1, 4)
    KK_CONV(PRO_BF16, EPI_STORE, 4, 2)
    KK_CONV(PRO_LEAKY, EPI_CONVT, 4, 2)
    KK_CONV(PRO_LEAKY, EPI_CONVT_REFLECT, 4, 2)
    KK_CONV(PRO_LEAKY, EPI_STORE, 1, 4)
#undef KK_CONV
    return hipErrorInvalidValue;
}

}  // namespace kk
