// kk_upstream.hip -- gfx950 kernels of the stages before the decoder (src/gpu_batch.rs:179-297):
// the ALBERT and text-encoder embeddings, LayerNorm / AdaLayerNorm over rows, ALBERT's per-item
// attention and the BiLSTM recurrence.  The linear layers and the text encoder's convolutions run
// on the MFMA conv kernel (kk_conv.hip) with bf16 operands and f32 accumulation, as the reference's
// GLinear / fused BF16 conv do (src/gpu.rs:280-301); everything here is f32.
//
// Token rows use the packed time-major layout of the decoder: items along the rows with gap rows
// between them, row_item[r] = owning item or -1.  Gap rows are never read by a consumer (the
// convolutions mask by item span, the attention and the recurrence read their item's rows only), so
// these kernels do not write them.
#include "kk_kernels.h"

#include <algorithm>
#include <atomic>
#include <functional>
#include <queue>
#include <utility>

namespace kk {
namespace {

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// Albert::embeddings (src/albert.rs:70-81): (word[id] + token_type[0]) + position[t], LayerNorm
// (eps 1e-12) over the 128 channels; one wave per row, two channels per lane.
__global__ void __launch_bounds__(256) albert_embed_kernel(const int32_t* ids, const int32_t* row_item,
                                                           const int64_t* start, int64_t rows, const float* word,
                                                           const float* pos, const float* tok0, const float* g,
                                                           const float* b, float* out) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int it = row_item[r];
    if (it < 0) return;
    const int64_t id = ids[r], t = r - start[it];
    float v[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int c = 2 * lane + e;
        v[e] = (word[id * 128 + c] + tok0[c]) + pos[t * 128 + c];
    }
    const float mean = wave_sum(v[0] + v[1]) * (1.0f / 128.0f);
    const float d0 = v[0] - mean, d1 = v[1] - mean;
    const float var = wave_sum(d0 * d0 + d1 * d1) * (1.0f / 128.0f);
    const float inv = 1.0f / sqrtf(var + 1e-12f);
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const int c = 2 * lane + e;
        out[r * 128 + c] = (v[e] - mean) * inv * g[c] + b[c];
    }
}

// text_encoder_b's embedding (src/gpu_batch.rs:461-469): out[r][0:512] = embedding[id]; one wave
// per row, two float4 per lane.
__global__ void __launch_bounds__(256) text_embed_kernel(const int32_t* ids, const int32_t* row_item, int64_t rows,
                                                         const float* emb, float* out) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows || row_item[r] < 0) return;
    const float4* src = (const float4*)(emb + (int64_t)ids[r] * 512);
    float4* dst = (float4*)(out + r * 512);
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
}

// LayerNorm over the first D channels of each item row of x [rows][ld], in place
// (layer_norm_rows / adaln_rows_seg, kernels/kokoro.cu:44-82, 337-373): mean, then the mean of
// squared deviations, inv = 1 / sqrt(var + eps); then either the affine g, b, or AdaLayerNorm's
// (1 + gamma[c]) o + beta[c] with gamma, beta = gb[item][gb_off + c], gb[item][gb_off + D + c];
// optionally leaky ReLU.  One wave per row, D / 256 float4 per lane.  The row is loaded together
// with its item index (a gap row is read and left alone), and the affine parameters as float4
// before the reductions: one or two memory latencies per row instead of three.
template <int D>
__global__ void __launch_bounds__(256) layernorm_kernel(float* x, int64_t ld, int64_t rows, const int32_t* row_item,
                                                        const float* g, const float* b, const float* gb, int64_t gb_ld,
                                                        int gb_off, float eps, int leaky, float slope) {
    constexpr int NV = D / 256;  // float4 per lane
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    const int it = row_item[r];
    float4* row = (float4*)(x + r * ld);
    float4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = row[lane + 64 * i];
    if (it < 0) return;
    float4 ga[NV], be[NV];  // the affine scale and shift of this lane's channels
    if (gb) {
        const float4* gam = (const float4*)(gb + (int64_t)it * gb_ld + gb_off);
#pragma unroll
        for (int i = 0; i < NV; i++) ga[i] = gam[lane + 64 * i], be[i] = gam[D / 4 + lane + 64 * i];
    } else {
#pragma unroll
        for (int i = 0; i < NV; i++) ga[i] = ((const float4*)g)[lane + 64 * i], be[i] = ((const float4*)b)[lane + 64 * i];
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    const float mean = wave_sum(s) * (1.0f / D);
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const float a = v[i].x - mean, bb = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
        q += (a * a + bb * bb) + (c * c + d * d);
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) * (1.0f / D) + eps);
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const float o[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        const float gv[4] = {ga[i].x, ga[i].y, ga[i].z, ga[i].w}, bv[4] = {be[i].x, be[i].y, be[i].z, be[i].w};
        float y4[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float y = (o[e] - mean) * inv;
            y = gb ? (1.0f + gv[e]) * y + bv[e] : y * gv[e] + bv[e];
            if (leaky) y = y < 0.f ? y * slope : y;
            y4[e] = y;
        }
        row[lane + 64 * i] = make_float4(y4[0], y4[1], y4[2], y4[3]);
    }
}

// Per-item multi-head attention of ALBERT (src/gpu_batch.rs:433-441; softmax_rows
// kernels/kokoro.cu:92-125): softmax over the item's keys of (q . k) / 8, times v, f32 throughout.
// qkv [rows][2304] (q | k | v, head h at columns 64 h), out [rows][768].  One block per (item, head,
// 64 queries); keys in chunks of 64 with the softmax carried across chunks (running row maximum and
// sum; the same exponentials as the reference's max-then-exp up to f32 rounding).  Thread (ty, tx)
// holds the scores of queries 4 ty..4 ty+3 x keys 4 tx..4 tx+3 and the output of those queries x
// dims 4 tx..4 tx+3: every LDS float4 read feeds 16 FMAs.
constexpr int kAttQ = 64, kAttLd = 68;  // queries per block; LDS row stride (floats)
__global__ void __launch_bounds__(256) attention_kernel(const float* qkv, const int64_t* start, const int64_t* len,
                                                        const int32_t* w_item, const int32_t* w_head,
                                                        const int32_t* w_q0, float* out, float scale) {
    __shared__ __align__(16) float Qt[64][kAttLd];  // [dim][query]
    __shared__ __align__(16) float Kt[64][kAttLd];  // [dim][key]
    __shared__ __align__(16) float Vs[64][kAttLd];  // [key][dim]
    __shared__ __align__(16) float Pt[64][kAttLd];  // [key][query]
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
    const int item = w_item[blockIdx.x], head = w_head[blockIdx.x], q0 = w_q0[blockIdx.x];
    const int64_t s0 = start[item];
    const int t = (int)len[item];
    const int nq = min(kAttQ, t - q0);
    constexpr int64_t LD = 3 * 768;
    // the query tile, transposed into LDS (rows past the item's queries as 0)
    for (int i = tid; i < kAttQ * 16; i += 256) {
        const int q = i >> 4, d4 = (i & 15) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (q < nq) v = *(const float4*)(qkv + (s0 + q0 + q) * LD + head * 64 + d4);
        Qt[d4][q] = v.x, Qt[d4 + 1][q] = v.y, Qt[d4 + 2][q] = v.z, Qt[d4 + 3][q] = v.w;
    }
    float m[4], l[4], o[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        m[i] = -INFINITY, l[i] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; j++) o[i][j] = 0.f;
    }
    for (int k0 = 0; k0 < t; k0 += 64) {
        const int nk = min(64, t - k0);
        __syncthreads();  // the previous chunk's Kt / Vs / Pt are consumed
        for (int i = tid; i < 64 * 16; i += 256) {
            const int k = i >> 4, d4 = (i & 15) * 4;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (k < nk) {
                const float* r = qkv + (s0 + k0 + k) * LD + head * 64 + d4;
                kv = *(const float4*)(r + 768), vv = *(const float4*)(r + 1536);
            }
            Kt[d4][k] = kv.x, Kt[d4 + 1][k] = kv.y, Kt[d4 + 2][k] = kv.z, Kt[d4 + 3][k] = kv.w;
            *(float4*)&Vs[k][d4] = vv;
        }
        __syncthreads();
        float sc[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) sc[i][j] = 0.f;
#pragma unroll 8
        for (int d = 0; d < 64; d++) {
            const float4 a = *(const float4*)&Qt[d][4 * ty], b = *(const float4*)&Kt[d][4 * tx];
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) sc[i][j] = fmaf(av[i], bv[j], sc[i][j]);
        }
        // scale, mask the keys past the item, carry the row maximum and sum (16 lanes per row)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                sc[i][j] = 4 * tx + j < nk ? sc[i][j] * scale : -INFINITY;
                mx = fmaxf(mx, sc[i][j]);
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
            const float mn = fmaxf(m[i], mx);
            const float corr = expf(m[i] - mn);  // 0 on the first chunk
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float e = expf(sc[i][j] - mn);
                Pt[4 * tx + j][4 * ty + i] = e;
                sum += e;
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
            l[i] = l[i] * corr + sum;
            m[i] = mn;
#pragma unroll
            for (int j = 0; j < 4; j++) o[i][j] *= corr;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < 64; k++) {
            const float4 p4 = *(const float4*)&Pt[k][4 * ty], v4 = *(const float4*)&Vs[k][4 * tx];
            const float pv[4] = {p4.x, p4.y, p4.z, p4.w}, vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) o[i][j] = fmaf(pv[i], vv[j], o[i][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int q = 4 * ty + i;
        if (q < nq) {
            const float inv = 1.0f / l[i];
            *(float4*)(out + (s0 + q0 + q) * 768 + head * 64 + 4 * tx) =
                make_float4(o[i][0] * inv, o[i][1] * inv, o[i][2] * inv, o[i][3] * inv);
        }
    }
}

// The same attention on the f32 matrix cores (v_mfma_f32_32x32x2_f32: f32 products, f32 sums, in
// another order than the VALU kernel above).  One block per (item, head, 64 queries), two waves of
// 32 queries each, keys in chunks of 64 staged in LDS ([key][dim]).  Everything is transposed so
// that a query stays in one lane pair: lane (l32, lh) owns query q0 + 32 w + l32, and
//  - S^T (keys x queries) = K Q^T: A = K[key][d], B = Q[query][d] with d = 32 lh + s at step s (the
//    lane's 32 dims of Q, pre-scaled by 1/8 -- exact, a power of two -- stay in registers), so the
//    lane ends with its query's scores for keys 8 (r / 4) + 4 lh + r % 4 (r < 16) of each 32-key
//    tile: the softmax's maximum and sum are lane-local plus one exchange with lane ^ 32;
//  - O^T (dims x queries) += V^T P^T: B = the lane's own P values (step s = r above), A =
//    V[key][dim] for the same keys, so P never leaves registers and the rescale by exp(m - m') is
//    per lane.
constexpr int kAmLd = 68;  // LDS row stride (floats) of the K and V chunks
__global__ void __launch_bounds__(128) attention_mfma_kernel(const float* qkv, const int64_t* start, const int64_t* len,
                                                             const int32_t* w_item, const int32_t* w_head,
                                                             const int32_t* w_q0, float* out) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    __shared__ __align__(16) float Ks[64][kAmLd];
    __shared__ __align__(16) float Vs[64][kAmLd];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, lh = lane >> 5;
    const int item = w_item[blockIdx.x], head = w_head[blockIdx.x], q0 = w_q0[blockIdx.x];
    const int64_t s0 = start[item];
    const int t = (int)len[item];
    constexpr int64_t LD = 3 * 768;
    const int q = q0 + 32 * wave + l32;  // this lane's query (rows past the item compute, unstored)
    float qr[32];
    {
        const float* qp = qkv + (s0 + (q < t ? q : 0)) * LD + head * 64 + 32 * lh;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 v = *(const float4*)(qp + 4 * j);
            const bool ok = q < t;
            qr[4 * j] = ok ? v.x * 0.125f : 0.f, qr[4 * j + 1] = ok ? v.y * 0.125f : 0.f;
            qr[4 * j + 2] = ok ? v.z * 0.125f : 0.f, qr[4 * j + 3] = ok ? v.w * 0.125f : 0.f;
        }
    }
    f32x16 o[2];
#pragma unroll
    for (int d = 0; d < 2; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[d][r] = 0.f;
    float m = -INFINITY, l = 0.f;
    for (int k0 = 0; k0 < t; k0 += 64) {
        const int nk = min(64, t - k0);
        __syncthreads();  // the previous chunk's K / V are consumed
        for (int i = tid; i < 64 * 16; i += 128) {
            const int k = i >> 4, d4 = (i & 15) * 4;
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (k < nk) {
                const float* r = qkv + (s0 + k0 + k) * LD + head * 64 + d4;
                kv = *(const float4*)(r + 768), vv = *(const float4*)(r + 1536);
            }
            *(float4*)&Ks[k][d4] = kv;
            *(float4*)&Vs[k][d4] = vv;
        }
        __syncthreads();
        // S^T for the chunk's two 32-key tiles
        f32x16 sc[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
#pragma unroll
            for (int r = 0; r < 16; r++) sc[kt][r] = 0.f;
            float kr[32];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float4 v = *(const float4*)&Ks[32 * kt + l32][32 * lh + 4 * j];
                kr[4 * j] = v.x, kr[4 * j + 1] = v.y, kr[4 * j + 2] = v.z, kr[4 * j + 3] = v.w;
            }
#pragma unroll
            for (int st = 0; st < 32; st++) sc[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[st], qr[st], sc[kt], 0, 0, 0);
        }
        // mask the keys past the item; the running maximum and sum of this lane's query
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = 32 * kt + 8 * (r >> 2) + 4 * lh + (r & 3);
                sc[kt][r] = key < nk ? sc[kt][r] : -INFINITY;
                mx = fmaxf(mx, sc[kt][r]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float mn = fmaxf(m, mx);
        const float corr = expf(m - mn);  // 0 on the first chunk
        float sum = 0.f;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                sc[kt][r] = expf(sc[kt][r] - mn);
                sum += sc[kt][r];
            }
        sum += __shfl_xor(sum, 32);
        l = l * corr + sum;
        m = mn;
#pragma unroll
        for (int d = 0; d < 2; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[d][r] *= corr;
        // O^T += V^T P^T: step st of tile kt pairs the keys 32 kt + 8 (st / 4) + 4 lh + st % 4
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int st = 0; st < 16; st++) {
                const int key = 32 * kt + 8 * (st >> 2) + 4 * lh + (st & 3);
#pragma unroll
                for (int d = 0; d < 2; d++)
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(Vs[key][32 * d + l32], sc[kt][st], o[d], 0, 0, 0);
            }
    }
    // lane (l32, lh) holds dims 32 d + 8 (r / 4) + 4 lh + r % 4 of query q: four float4 per tile
    if (q < t) {
        const float inv = 1.0f / l;
        float* op = out + (s0 + q) * 768 + head * 64;
#pragma unroll
        for (int d = 0; d < 2; d++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(float4*)(op + 32 * d + 8 * g + 4 * lh) =
                    make_float4(o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv, o[d][4 * g + 3] * inv);
    }
}

// BiLSTM recurrence (lstm_seq_batched semantics, kernels/kokoro.cu:400-455): one block per
// (item, direction), 512 threads.  Per step: gate_r = gx[row][dir 4H + r] + (W_hh[r] . h + b_hh[r])
// for the 4H = 1024 gate rows (gates i, f, g, o), then unit j: c_j = f c_j + i g, h_j = o tanh(c_j),
// written to out[row][dir H + j].  The forward direction walks the item's rows in order, the
// reverse one backwards.  gx rows come through gx_row (the frame -> token table: a repeated token
// row has the same gate pre-activations) or are the item's own rows.
//
// The step is bound by moving W_hh (1 MB of f32, k-major [H][4H]) into the CU, so as much of it as
// fits stays on the CU for the whole sequence: thread t owns gate rows 4c..4c+3 (c = t mod 256) over
// the k-half [128 q, 128 q + 128) (q = t / 256); of its 128 k, the first kLstmKR are held in
// registers (float4 per k), the next kLstmKL in LDS, the rest are read from L2 each step as one
// 16-byte load per k (384 KB in registers, 144 KB in LDS, 496 KB streamed per step).  The two
// k-halves' partial sums meet in LDS.  No block waits for another: every block ends after its
// item's steps.
constexpr int kH = 256, kLstmThreads = 512, kLstmKR = 48, kLstmKL = 18;
constexpr int kLstmKS = 128 - kLstmKR - kLstmKL;  // streamed k per half
constexpr size_t kLstmLds = ((size_t)2 * kLstmKL * 4 * kH + 2 * 4 * kH + kH) * sizeof(float);
__global__ void __launch_bounds__(kLstmThreads) lstm_kernel(const float* gx, int64_t gx_ld, const int32_t* gx_row,
                                                            const int64_t* start, const int64_t* len,
                                                            const float* whh_t, const float* bhh, float* out,
                                                            int64_t out_ld) {
    extern __shared__ __align__(16) float lsm[];
    float* Wl = lsm;                          // [2 halves][kLstmKL][1024]
    float* part = Wl + 2 * kLstmKL * 4 * kH;  // [2][1024] partial dot products
    float* hs = part + 2 * 4 * kH;            // [256] h of the previous step
    const int t = threadIdx.x, q = t >> 8, c = t & 255;
    const int item = blockIdx.x >> 1, dir = blockIdx.x & 1;
    const int64_t s0 = start[item], n = len[item];
    const float* W = whh_t + (int64_t)dir * kH * 4 * kH;
    const float* Wq = W + (int64_t)(128 * q) * 4 * kH + 4 * c;
    float4 wr[kLstmKR];
#pragma unroll
    for (int i = 0; i < kLstmKR; i++) wr[i] = *(const float4*)(Wq + (int64_t)i * 4 * kH);
    for (int i = t; i < 2 * kLstmKL * kH; i += kLstmThreads) {
        const int row = i >> 8, qq = row / kLstmKL, ii = row - qq * kLstmKL, c4 = i & 255;
        *(float4*)(Wl + (int64_t)row * 4 * kH + 4 * c4) =
            *(const float4*)(W + (int64_t)(128 * qq + kLstmKR + ii) * 4 * kH + 4 * c4);
    }
    float cst = 0.f, bh[4];
    if (t < kH) {
        hs[t] = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) bh[g] = bhh[dir * 4 * kH + g * kH + t];
    }
    __syncthreads();
    const float* Wlq = Wl + (int64_t)(q * kLstmKL) * 4 * kH + 4 * c;
    const float* Ws = Wq + (int64_t)(kLstmKR + kLstmKL) * 4 * kH;
    const float* hq = hs + 128 * q;
    for (int64_t step = 0; step < n; step++) {
        const int64_t row = s0 + (dir == 0 ? step : n - 1 - step);
        float gxv[4];
        if (t < kH) {
            const int64_t grow = gx_row ? (int64_t)gx_row[row] : row;
#pragma unroll
            for (int g = 0; g < 4; g++) gxv[g] = gx[grow * gx_ld + dir * 4 * kH + g * kH + t];
        }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < kLstmKR; i += 4) {
            const float4 h4 = *(const float4*)(hq + i);
            const float hv[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float4 w = wr[i + e];
                acc.x = fmaf(w.x, hv[e], acc.x), acc.y = fmaf(w.y, hv[e], acc.y);
                acc.z = fmaf(w.z, hv[e], acc.z), acc.w = fmaf(w.w, hv[e], acc.w);
            }
        }
#pragma unroll
        for (int i = 0; i < kLstmKL; i++) {
            const float hv = hq[kLstmKR + i];
            const float4 w = *(const float4*)(Wlq + (int64_t)i * 4 * kH);
            acc.x = fmaf(w.x, hv, acc.x), acc.y = fmaf(w.y, hv, acc.y);
            acc.z = fmaf(w.z, hv, acc.z), acc.w = fmaf(w.w, hv, acc.w);
        }
        // unrolled by 8: with 16 the compiler's schedule overlaps the streamed loads with the
        // register and LDS parts less well (measured 7.8 against 4.9 us per step)
#pragma unroll 8
        for (int i = 0; i < kLstmKS; i++) {
            const float hv = hq[kLstmKR + kLstmKL + i];
            const float4 w = *(const float4*)(Ws + (int64_t)i * 4 * kH);
            acc.x = fmaf(w.x, hv, acc.x), acc.y = fmaf(w.y, hv, acc.y);
            acc.z = fmaf(w.z, hv, acc.z), acc.w = fmaf(w.w, hv, acc.w);
        }
        *(float4*)(part + q * 4 * kH + 4 * c) = acc;
        __syncthreads();
        if (t < kH) {
            float gate[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int r = g * kH + t;
                gate[g] = gxv[g] + ((part[r] + part[4 * kH + r]) + bh[g]);
            }
            const float ig = sigmoid(gate[0]), fg = sigmoid(gate[1]), gg = tanhf(gate[2]), og = sigmoid(gate[3]);
            cst = fg * cst + ig * gg;
            const float h = og * tanhf(cst);
            hs[t] = h;
            out[row * out_ld + dir * kH + t] = h;
        }
        __syncthreads();
    }
}

// The same recurrence with each (item, direction) sequence split over a pair of blocks on two CUs:
// block half hf owns hidden units [128 hf, 128 hf + 128), i.e. the 512 gate rows g 256 + 128 hf + u,
// and all 512 KB of their W_hh stay on its CU (thread t: rows 4c..4c+3 of the half, c = t mod 128,
// over the k-quarter [64 q, 64 q + 64), q = t / 128; 48 of its k in registers, 16 in LDS).  Each
// step a block computes its 128 units of h and trades them with its partner through the exchange
// buffer: one 64-bit word per unit, (step + 1) << 32 | bits(h), written and polled with relaxed
// device-scope atomics -- a word carries its own step, so no fence orders data and flag.  Two
// parities of words per half: a block overwrites the words of step s at step s + 2 only after its
// partner has used them (the partner's step s + 1 needed them).  The buffer starts at zero each
// launch (lstm_exchange_clear_kernel), the first valid tag is 1.
// Pairing: block B = 16 grp + 8 hf + x is half hf of sequence 8 grp + x, so the two halves sit 8
// apart (the same XCD under round-robin dispatch, and consecutive on it).  Every wait is bounded:
// past wait_ticks of the 100 MHz clock (or once another block gave up) the block sets *abort and
// ends, and the host reports the run as failed.  silent_half (a test hook; -1 otherwise): the
// blocks of that half publish nothing, so that their partners' waits run out.
constexpr int kLpKR = 48, kLpKL = 16;  // per thread: k in registers, k in LDS (of 64)
constexpr size_t kLpLds = ((size_t)4 * kLpKL * 512 + 4 * 512 + kH) * sizeof(float);
__global__ void __launch_bounds__(kLstmThreads) lstm_pair_kernel(const float* gx, int64_t gx_ld, const int32_t* gx_row,
                                                                 const int64_t* start, const int64_t* len, int nseq,
                                                                 const float* whh_t, const float* bhh, float* out,
                                                                 int64_t out_ld, uint64_t* xbuf, int* abort,
                                                                 uint64_t wait_ticks, int silent_half) {
    extern __shared__ __align__(16) float lsm[];
    float* Wl = lsm;                       // [4 quarters][kLpKL][512 rows]
    float* part = Wl + 4 * kLpKL * 512;    // [4][512] partial dot products
    float* hs = part + 4 * 512;            // [256] h of the previous step
    __shared__ int gave_up;
    const int B = blockIdx.x, grp = B >> 4, hf = (B >> 3) & 1;
    const int seq = grp * 8 + (B & 7);
    if (seq >= nseq) return;  // the pair's other half returns too
    const int item = seq >> 1, dir = seq & 1;
    const int t = threadIdx.x, q = t >> 7, c = t & 127;
    const int64_t s0 = start[item], n = len[item];
    // this thread's four gate rows (one gate g = c / 32, units 4 (c mod 32) .. + 3 of the half)
    const int g0 = (c >> 5) * kH + 128 * hf + 4 * (c & 31);
    const float* W = whh_t + (int64_t)dir * kH * 4 * kH;
    float4 wr[kLpKR];
#pragma unroll
    for (int i = 0; i < kLpKR; i++) wr[i] = *(const float4*)(W + (int64_t)(64 * q + i) * 4 * kH + g0);
    for (int i = t; i < 4 * kLpKL * 128; i += kLstmThreads) {
        const int row = i >> 7, qq = row / kLpKL, ii = row - qq * kLpKL, cc = i & 127;
        const int gg = (cc >> 5) * kH + 128 * hf + 4 * (cc & 31);
        *(float4*)(Wl + (int64_t)row * 512 + 4 * cc) = *(const float4*)(W + (int64_t)(64 * qq + kLpKR + ii) * 4 * kH + gg);
    }
    float cst = 0.f, bh[4];
    if (t < 128) {
#pragma unroll
        for (int g = 0; g < 4; g++) bh[g] = bhh[dir * 4 * kH + g * kH + 128 * hf + t];
    }
    if (t < kH) hs[t] = 0.f;
    if (t == 0) gave_up = 0;
    __syncthreads();
    const float* Wlq = Wl + (int64_t)(q * kLpKL) * 512 + 4 * c;
    const float* hq = hs + 64 * q;
    uint64_t* xw = xbuf + (int64_t)seq * 512 + hf * 256;        // [parity][128] this half's words
    const uint64_t* xr = xbuf + (int64_t)seq * 512 + (1 - hf) * 256;  // the partner's
    for (int64_t step = 0; step < n; step++) {
        const int64_t row = s0 + (dir == 0 ? step : n - 1 - step);
        float gxv[4];
        if (t < 128) {
            const int64_t grow = gx_row ? (int64_t)gx_row[row] : row;
#pragma unroll
            for (int g = 0; g < 4; g++) gxv[g] = gx[grow * gx_ld + dir * 4 * kH + g * kH + 128 * hf + t];
        }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < kLpKR; i += 4) {
            const float4 h4 = *(const float4*)(hq + i);
            const float hv[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float4 w = wr[i + e];
                acc.x = fmaf(w.x, hv[e], acc.x), acc.y = fmaf(w.y, hv[e], acc.y);
                acc.z = fmaf(w.z, hv[e], acc.z), acc.w = fmaf(w.w, hv[e], acc.w);
            }
        }
#pragma unroll
        for (int i = 0; i < kLpKL; i++) {
            const float hv = hq[kLpKR + i];
            const float4 w = *(const float4*)(Wlq + (int64_t)i * 512);
            acc.x = fmaf(w.x, hv, acc.x), acc.y = fmaf(w.y, hv, acc.y);
            acc.z = fmaf(w.z, hv, acc.z), acc.w = fmaf(w.w, hv, acc.w);
        }
        *(float4*)(part + q * 512 + 4 * c) = acc;
        __syncthreads();
        if (t < 128) {
            float gate[4];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int r = g * 128 + t;
                gate[g] = gxv[g] + (((part[r] + part[512 + r]) + (part[1024 + r] + part[1536 + r])) + bh[g]);
            }
            const float ig = sigmoid(gate[0]), fg = sigmoid(gate[1]), gg = tanhf(gate[2]), og = sigmoid(gate[3]);
            cst = fg * cst + ig * gg;
            const float h = og * tanhf(cst);
            const uint64_t tag = (uint64_t)(step + 1) << 32;
            if (hf != silent_half)
                __hip_atomic_store(xw + (step & 1) * 128 + t, tag | __float_as_uint(h), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            hs[128 * hf + t] = h;
            out[row * out_ld + dir * kH + 128 * hf + t] = h;
            // the partner's unit t of this step
            const uint64_t* src = xr + (step & 1) * 128 + t;
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            uint64_t w;
            for (uint32_t spin = 1;; spin++) {
                w = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((w & 0xffffffff00000000ull) == tag) break;
                if ((spin & 255) == 0 && (__hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 ||
                                          __builtin_amdgcn_s_memrealtime() - t0 > wait_ticks)) {
                    gave_up = 1;
                    break;
                }
            }
            hs[128 * (1 - hf) + t] = __uint_as_float((uint32_t)w);
        }
        __syncthreads();
        if (gave_up) {
            if (t == 0) __hip_atomic_store(abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
    }
}

// The BiLSTM recurrence on FOUR CUs per (item, direction): block quarter qb owns the 64 hidden units
// [64 qb, 64 qb + 64), i.e. 256 gate rows, and keeps all of their W_hh in registers (thread t: the
// gate rows g 256 + 64 qb + 2 (c mod 32) + {0, 1} with g = c / 32, c = t mod 128, over the
// k-quarter q = t / 128: 64 k x 2 rows = 128 floats), so a step reads no weights from LDS and each
// CU does half the pair kernel's multiply-adds.  Each step the block computes its 64 units of h and
// trades them with its three partners through the same self-tagged 64-bit words as the pair kernel
// (one word per unit, two parities per quarter: a block rewrites step s's words at step s + 2 only
// after every partner has finished step s + 1, hence has read them); threads 0..63 compute and
// publish the block's units while threads 64..255 wait for the partners' 192.  Every row's dot
// product is summed in the pair kernel's order (the k-quarter's 64 terms in sequence, then the four
// quarters as ((q0 + q1) + (q2 + q3)) + b_hh): the outputs are bit-identical to it.
// The quarters of a quad are blocks 8 apart (the same XCD under round-robin dispatch) and 32
// consecutive blocks hold 8 complete quads; a launch has at most kLstmQuads quads (one block per
// CU), and each quad runs a list of sequences one after another, from a schedule the host computes
// at plan creation: longest first, each sequence to the quad with the least work so far -- the
// longest start at once, and the short ones follow on the quads that finish first, with no second
// wave of blocks waiting for CUs.  A quad reloads its W_hh rows only when the direction changes;
// every sequence starts from h = c = 0 and has its own exchange words.  A block whose partners
// are not resident yet waits for CUs that finishing quads release (nothing a quad waits for
// depends on a later one).  Every wait is bounded as in the pair kernel.
//   sched: [nq + 1] list offsets, then the sequence ids (2 item + direction) of the quads' lists.
__global__ void __launch_bounds__(kLstmThreads) lstm_quad_kernel(const float* gx, int64_t gx_ld, const int32_t* gx_row,
                                                                 const int64_t* start, const int64_t* len,
                                                                 const int32_t* sched, int nq, const float* whh_t,
                                                                 const float* bhh, float* out, int64_t out_ld,
                                                                 uint64_t* xbuf, int* abort, uint64_t wait_ticks,
                                                                 int silent_quarter) {
    __shared__ float part[4][256];  // partial dot products per k-quarter, local rows g 64 + u
    __shared__ float hs[kH];        // h of the previous step
    __shared__ int gave_up;
    const int B = blockIdx.x, qb = (B >> 3) & 3;
    const int quad = (B >> 5) * 8 + (B & 7);
    if (quad >= nq) return;  // the quad's other quarters return too
    const int t = threadIdx.x, q = t >> 7, c = t & 127;
    if (t == 0) gave_up = 0;
    const int g = c >> 5, u0 = 2 * (c & 31);  // this thread's rows: gate g, units u0, u0 + 1 of the quarter
    // threads 64..255: the partner quarter and unit they wait for
    const int tp = t - 64, pq = (qb + 1 + tp / 64) & 3, pu = tp & 63;
    const float* hq = hs + 64 * q;
    float2 wr[64];
    int wdir = -1;
    const int li_end = sched[quad + 1];
    for (int li = sched[quad]; li < li_end; li++) {
        const int seq = sched[nq + 1 + li];
        const int item = seq >> 1, dir = seq & 1;
        const int64_t s0 = start[item], n = len[item];
        if (dir != wdir) {
            const float* W = whh_t + (int64_t)dir * kH * 4 * kH + g * kH + 64 * qb + u0;
#pragma unroll
            for (int k = 0; k < 64; k++) wr[k] = *(const float2*)(W + (int64_t)(64 * q + k) * 4 * kH);
            wdir = dir;
        }
        float cst = 0.f, bh[4];
        if (t < 64) {
#pragma unroll
            for (int gg = 0; gg < 4; gg++) bh[gg] = bhh[dir * 4 * kH + gg * kH + 64 * qb + t];
        }
        if (t < kH) hs[t] = 0.f;  // every read of the previous sequence's h ended before its last barrier
        __syncthreads();
        uint64_t* xw = xbuf + (int64_t)seq * 512 + qb * 128;  // [parity][64] this quarter's words
        const uint64_t* xr = xbuf + (int64_t)seq * 512 + pq * 128 + pu;
        for (int64_t step = 0; step < n; step++) {
            const int64_t row = s0 + (dir == 0 ? step : n - 1 - step);
            float gxv[4];
            if (t < 64) {
                const int64_t grow = gx_row ? (int64_t)gx_row[row] : row;
#pragma unroll
                for (int gg = 0; gg < 4; gg++) gxv[gg] = gx[grow * gx_ld + dir * 4 * kH + gg * kH + 64 * qb + t];
            }
            float2 acc = make_float2(0.f, 0.f);
#pragma unroll
            for (int k = 0; k < 64; k += 4) {
                const float4 h4 = *(const float4*)(hq + k);
                const float hv[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    acc.x = fmaf(wr[k + e].x, hv[e], acc.x);
                    acc.y = fmaf(wr[k + e].y, hv[e], acc.y);
                }
            }
            *(float2*)(&part[q][g * 64 + u0]) = acc;
            __syncthreads();
            const uint64_t tag = (uint64_t)(step + 1) << 32;
            if (t < 64) {
                float gate[4];
#pragma unroll
                for (int gg = 0; gg < 4; gg++) {
                    const int r = gg * 64 + t;
                    gate[gg] = gxv[gg] + (((part[0][r] + part[1][r]) + (part[2][r] + part[3][r])) + bh[gg]);
                }
                const float ig = sigmoid(gate[0]), fg = sigmoid(gate[1]), gg2 = tanhf(gate[2]), og = sigmoid(gate[3]);
                cst = fg * cst + ig * gg2;
                const float h = og * tanhf(cst);
                if (qb != silent_quarter)
                    __hip_atomic_store(xw + (step & 1) * 64 + t, tag | __float_as_uint(h), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                hs[64 * qb + t] = h;
                out[row * out_ld + dir * kH + 64 * qb + t] = h;
            } else if (t < 256) {
                const uint64_t* src = xr + (step & 1) * 64;
                const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                uint64_t w;
                for (uint32_t spin = 1;; spin++) {
                    w = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((w & 0xffffffff00000000ull) == tag) break;
                    if ((spin & 255) == 0 &&
                        (__hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 ||
                         __builtin_amdgcn_s_memrealtime() - t0 > wait_ticks)) {
                        gave_up = 1;
                        break;
                    }
                }
                hs[64 * pq + pu] = __uint_as_float((uint32_t)w);
            }
            __syncthreads();
            if (gave_up) {
                if (t == 0) __hip_atomic_store(abort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                return;
            }
        }
    }
}

// Zeroes the pair recurrence's exchange words (n 64-bit words) before a launch.
__global__ void __launch_bounds__(256) lstm_exchange_clear_kernel(uint64_t* x, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = 0;
}

// out[r][col0 + c] = styles[row_item[r]][c] for the item rows (cat_style_rows_seg's style half,
// kernels/kokoro.cu:375-384; the other half is written in place by its producer).
__global__ void __launch_bounds__(256) style_cols_kernel(float* x, int64_t ld, int col0, int64_t rows,
                                                         const int32_t* row_item, const float* styles) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * 32) return;
    const int64_t r = i >> 5;
    const int c4 = (int)(i & 31) * 4;
    const int it = row_item[r];
    if (it < 0) return;
    *(float4*)(x + r * ld + col0 + c4) = *(const float4*)(styles + (int64_t)it * 128 + c4);
}

// F0_proj / N_proj, Conv1d k1 256 -> 1, over every row of the domain: y[r] = b + w . x[r] on item
// rows, 0 in the gaps (the reference masks F0 and N after the projection, src/gpu_batch.rs:291-292).
// One wave per row, four channels per lane.
__global__ void __launch_bounds__(256) proj1_kernel(const float* x, int64_t ld, const float* w, const float* b,
                                                    const int32_t* col, int64_t rows, float* y) {
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (r >= rows) return;
    if (col[r] < 0) {
        if (lane == 0) y[r] = 0.f;
        return;
    }
    const float4 v = *(const float4*)(x + r * ld + 4 * lane), ww = *(const float4*)(w + 4 * lane);
    const float d = wave_sum((v.x * ww.x + v.y * ww.y) + (v.z * ww.z + v.w * ww.w));
    if (lane == 0) y[r] = b[0] + d;
}

}  // namespace

hipError_t launch_proj1(const float* x, int64_t ld, int c, const float* w, const float* b, const int32_t* col,
                        int64_t rows, float* y, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (c != 256 || ld % 4 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(proj1_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s, x, ld, w, b, col, rows, y);
    return hipGetLastError();
}

hipError_t launch_albert_embed(const int32_t* ids, const int32_t* row_item, const int64_t* start, int64_t rows,
                               const float* word, const float* pos, const float* tok0, const float* g, const float* b,
                               float* out, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(albert_embed_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s, ids, row_item, start,
                       rows, word, pos, tok0, g, b, out);
    return hipGetLastError();
}

hipError_t launch_text_embed(const int32_t* ids, const int32_t* row_item, int64_t rows, const float* emb, float* out,
                             hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(text_embed_kernel, dim3((unsigned)ceil_div(rows, 4)), dim3(256), 0, s, ids, row_item, rows, emb,
                       out);
    return hipGetLastError();
}

hipError_t launch_layernorm(float* x, int64_t ld, int d, int64_t rows, const int32_t* row_item, const float* g,
                            const float* b, const float* gb, int64_t gb_ld, int gb_off, float eps, bool leaky,
                            float slope, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (ld % 4 != 0 || (gb == nullptr && (g == nullptr || b == nullptr))) return hipErrorInvalidValue;
    if (gb && (gb_ld % 4 != 0 || gb_off % 4 != 0)) return hipErrorInvalidValue;  // float4 parameter loads
    const dim3 grid((unsigned)ceil_div(rows, 4));
    if (d == 768)
        hipLaunchKernelGGL(layernorm_kernel<768>, grid, dim3(256), 0, s, x, ld, rows, row_item, g, b, gb, gb_ld, gb_off,
                           eps, (int)leaky, slope);
    else if (d == 512)
        hipLaunchKernelGGL(layernorm_kernel<512>, grid, dim3(256), 0, s, x, ld, rows, row_item, g, b, gb, gb_ld, gb_off,
                           eps, (int)leaky, slope);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_attention(const float* qkv, const int64_t* start, const int64_t* len, const int32_t* w_item,
                            const int32_t* w_head, const int32_t* w_q0, int64_t n_blocks, float* out, hipStream_t s,
                            bool valu) {
    if (n_blocks <= 0) return hipSuccess;
    if (valu)
        hipLaunchKernelGGL(attention_kernel, dim3((unsigned)n_blocks), dim3(256), 0, s, qkv, start, len, w_item,
                           w_head, w_q0, out, 0.125f);
    else
        hipLaunchKernelGGL(attention_mfma_kernel, dim3((unsigned)n_blocks), dim3(128), 0, s, qkv, start, len, w_item,
                           w_head, w_q0, out);
    return hipGetLastError();
}

hipError_t launch_lstm(const float* gx, int64_t gx_ld, const int32_t* gx_row, const int64_t* start, const int64_t* len,
                       int nb, const float* whh_t, const float* bhh, float* out, int64_t out_ld, hipStream_t s) {
    if (nb <= 0) return hipSuccess;
    // the dynamic LDS limit is a per-device attribute of the kernel: set once per device
    static std::atomic<uint64_t> attr_set{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!((attr_set.load() >> dev) & 1u)) {
        e = hipFuncSetAttribute((const void*)lstm_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLstmLds);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(1ull << dev);
    }
    hipLaunchKernelGGL(lstm_kernel, dim3((unsigned)(2 * nb)), dim3(kLstmThreads), kLstmLds, s, gx, gx_ld, gx_row, start,
                       len, whh_t, bhh, out, out_ld);
    return hipGetLastError();
}

hipError_t launch_lstm_pair(const float* gx, int64_t gx_ld, const int32_t* gx_row, const int64_t* start,
                            const int64_t* len, int nb, const float* whh_t, const float* bhh, float* out, int64_t out_ld,
                            uint64_t* xbuf, int* abort, hipStream_t s, uint64_t wait_ticks, int silent_half) {
    if (nb <= 0) return hipSuccess;
    if (!xbuf || !abort || wait_ticks == 0) return hipErrorInvalidValue;
    static std::atomic<uint64_t> attr_set{0};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    if (!((attr_set.load() >> dev) & 1u)) {
        e = hipFuncSetAttribute((const void*)lstm_pair_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLpLds);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(1ull << dev);
    }
    const int nseq = 2 * nb;
    const int64_t words = (int64_t)nseq * 512;
    hipLaunchKernelGGL(lstm_exchange_clear_kernel, dim3((unsigned)ceil_div(words, 256)), dim3(256), 0, s, xbuf, words);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(lstm_pair_kernel, dim3((unsigned)(ceil_div(nseq, 8) * 16)), dim3(kLstmThreads), kLpLds, s, gx,
                       gx_ld, gx_row, start, len, nseq, whh_t, bhh, out, out_ld, xbuf, abort, wait_ticks, silent_half);
    return hipGetLastError();
}

hipError_t launch_lstm_quad(const float* gx, int64_t gx_ld, const int32_t* gx_row, const int64_t* start,
                            const int64_t* len, int nb, const int32_t* sched, const float* whh_t, const float* bhh,
                            float* out, int64_t out_ld, uint64_t* xbuf, int* abort, hipStream_t s, uint64_t wait_ticks,
                            int silent_quarter) {
    if (nb <= 0) return hipSuccess;
    if (!xbuf || !abort || !sched || wait_ticks == 0) return hipErrorInvalidValue;
    const int nseq = 2 * nb, nq = lstm_quads(nb);
    const int64_t words = (int64_t)nseq * 512;
    hipLaunchKernelGGL(lstm_exchange_clear_kernel, dim3((unsigned)ceil_div(words, 256)), dim3(256), 0, s, xbuf, words);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(lstm_quad_kernel, dim3((unsigned)(ceil_div(nq, 8) * 32)), dim3(kLstmThreads), 0, s, gx, gx_ld,
                       gx_row, start, len, sched, nq, whh_t, bhh, out, out_ld, xbuf, abort, wait_ticks, silent_quarter);
    return hipGetLastError();
}

std::vector<int32_t> lstm_schedule(const int64_t* len, int nb) {
    const int nq = lstm_quads(nb);
    std::vector<int32_t> items(nb);
    for (int i = 0; i < nb; i++) items[i] = i;
    std::stable_sort(items.begin(), items.end(), [&](int a, int b) { return len[a] > len[b]; });
    typedef std::pair<int64_t, int> Load;  // (total length, quad): the least first, ties by quad
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> free_q;
    for (int q = 0; q < nq; q++) free_q.push(Load{0, q});
    std::vector<std::vector<int32_t>> lists(nq);
    for (int i : items)
        for (int d = 0; d < 2; d++) {
            const Load l = free_q.top();
            free_q.pop();
            lists[l.second].push_back(2 * i + d);
            free_q.push(Load{l.first + len[i], l.second});
        }
    std::vector<int32_t> out(nq + 1 + 2 * nb);
    int o = 0;
    for (int q = 0; q < nq; q++) {
        out[q] = o;
        for (int32_t sq : lists[q]) out[nq + 1 + o++] = sq;
    }
    out[nq] = o;
    return out;
}

hipError_t launch_clear_u64(uint64_t* x, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(lstm_exchange_clear_kernel, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, s, x, n);
    return hipGetLastError();
}

hipError_t launch_style_cols(float* x, int64_t ld, int col0, int64_t rows, const int32_t* row_item,
                             const float* styles, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if ((ld | col0) % 4 != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(style_cols_kernel, dim3((unsigned)ceil_div(rows * 32, 256)), dim3(256), 0, s, x, ld, col0, rows,
                       row_item, styles);
    return hipGetLastError();
}

}  // namespace kk
