// kk_conv.hip -- bf16 implicit-GEMM convolution on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// One kernel family serves every MFMA layer of the path:
//   * stride-1 Conv1d with any K / dilation (decoder conv1/conv2/conv1x1/asr_res, the 48 Snake-block
//     convs, conv_post) -- the reference's conv1d_wmma_bf16[_snake[_res]] and per-tap cuBLAS
//     routes (src/gpu.rs:331-499, kernels/kokoro.cu:660-774);
//   * ConvTranspose1d with K = 2*stride as a polyphase 2-tap conv whose GEMM rows are
//     (phase, out-channel) pairs (replaces the f32 sgemm + convT_gather of src/gpu.rs:527-537).
//
// GEMM view: M = output channels (x phases), N = time columns, K = input channels x taps.
// * Work units are (tile, M-block) pairs.  Tiles are item-aligned (kk_kernels.h TilesDev): a tile
//   never mixes items, so the per-item zero padding of the reference's gap masking
//   (src/gpu_batch.rs:62-79) is a row-range test and the AdaIN coefficients are constants of the
//   unit.  One persistent block per CU walks a strided list of units; the M-blocks of one tile run
//   side by side on one XCD and share its L2 copy of the tile's input.
// * Warp specialization.  Producer waves stream the input through LDS in 64-channel slabs
//   ([time][64 + 8 pad] bf16, 144-byte rows: the 16 rows of a B-fragment read fall on distinct
//   banks): global loads of slab g + 2 are in flight while slab g + 1 is converted, and the layer's
//   prologue (AdaIN affine + Snake or leaky ReLU, f32 -> bf16 with the hardware round-to-nearest-
//   even convert) runs once per staged element.  Consumer waves run the MFMAs of slab g from the
//   other LDS buffer; one barrier per slab hands the buffers over.  Vector-memory counters complete
//   in issue order, so keeping the HBM stream in the producer waves keeps the consumers' waits to
//   their own weight loads (L2 hits), and the producers' VALU work co-issues with the MFMAs.
// * The consumers issue v_mfma_f32_32x32x16_bf16: one wave per SIMD sustains the matrix core's
//   rate with the 32x32 shape (the 16x16x32 shape needs two).  Each consumer wave owns a 64 x 128
//   output tile (2 x 4 MFMA tiles, 128 accumulator registers); layers of at most 32 output rows
//   (conv_post) use 32 x 128 tiles (1 x 4).
// * A (weights) is pre-packed as [tap][cin/16][M_pad][16] bf16: one A fragment (32 rows x 16
//   channels) is a contiguous 1 KB, loaded into registers a full tap ahead of its use; B fragments
//   are read from LDS one 16-channel step ahead.
// * The epilogue adds the bias, applies the layer's residual rule in f32 and, when asked, reduces
//   the instance-norm statistics of the values it stores: per (tile, wave, channel) sums of
//   (v - v_first), written to a partials buffer that finalize combines in a fixed order.
// * The Snake blocks' conv1 output (input of conv2's AdaIN) is stored as fp16: half the HBM
//   traffic of f32, 8x the precision of the bf16 operands.  So is the generator resblocks' residual
//   stream (each block's running sum: conv2 adds into it in place as fp16, the next conv1 reads
//   it, the stage's mean reads all three); the stage input it starts from stays f32.
#include "kk_common.h"
#include "kk_kernels.h"
#include "kk_walk.h"

#include <algorithm>
#include <type_traits>
#include <atomic>

namespace kk {

namespace {

constexpr int kCK = 64;       // input channels per LDS slab
constexpr int kRS = kCK + 8;  // LDS row stride (bf16 elements, 144 bytes)
constexpr int kNJ = 8;        // 16-column MFMA tiles per wave (wave N = 128)
constexpr int kMaxHalo = 64;    // largest (k - 1) * dil the staging covers
constexpr int kSmallHalo = 16;  // layers with (k - 1) * dil up to this run fewer producer passes
constexpr int kNP = 256;      // producer threads per block

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    const bf16x2_t v = __builtin_convertvector((f32x2_t){a, b}, bf16x2_t);  // v_cvt_pk_bf16_f32 (RNE)
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    const f16x2_t v = __builtin_convertvector((f32x2_t){a, b}, f16x2_t);  // v_cvt_pk_f16_f32 (RNE)
    return __builtin_bit_cast(uint32_t, v);
}

// Read-only tables (tiles, item spans) through the constant address space: uniform indices become
// scalar loads, which leave the vector-memory counter -- and the producers' prefetch -- alone.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p, int64_t i) {
    return ((const __attribute__((address_space(4))) T*)p)[i];
}

// Per-device flags (device ordinals below 64), safe to set from several host threads.
struct DeviceFlags {
    std::atomic<uint64_t> bits{0};
    bool test(int dev) const { return dev >= 0 && dev < 64 && ((bits.load() >> dev) & 1u); }
    void set(int dev) {
        if (dev >= 0 && dev < 64) bits.fetch_or(1ull << dev);
    }
};

// One (tile, M-block) unit of work.  Rows fit in 32 bits (checked on the host).
struct Unit {
    int tile, n0, in0, i_lo, i_hi, m0, item, nv;
};

// An empty asm that reads its operands: whatever produces them (e.g. their loads) completes here,
// once and outside any branch.  Without it, a first use inside a branch that may be skipped makes
// the wait-count pass (whose state merges conservatively at join points) wait for every later load.
__device__ __forceinline__ void ready(const float4& v) { asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w)); }
__device__ __forceinline__ void ready(uint32_t v) { asm volatile("" ::"v"(v)); }
// Copy a (uniform) value into a VGPR, so it is not rematerialized from memory inside a loop.
__device__ __forceinline__ int vgpr(int x) {
    int v;
    asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "s"(x));
    return v;
}
__device__ __forceinline__ float vgpr_f(float x) { return __int_as_float(vgpr(__float_as_int(x))); }

// Producer side: one slab = rows [in0, in0 + tw) x channels [c0, c0 + 64) of the input.  Producer
// thread pt owns channel quad q = (pt % 16) * 4 of rows pt / 16 + j * RP (j < RB).  A Slot holds one
// slab's raw input and the per-channel prologue constants in registers; load() issues every global
// load of the slab (addresses outside the unit's item are clamped to a row of the item, so the
// number of loads is fixed and the producers' wait counts are static), convert() applies the
// prologue and writes bf16 rows into an LDS buffer.  Rows outside the item, and channels >= cin,
// are staged as 0 (the conv's zero padding of the activated signal).
template <int PRO, bool IN_H, int BN, int MAXH>
struct Slot {
    static constexpr int RP = kNP / 16;                   // rows per pass
    static constexpr int RB = (BN + MAXH + RP - 1) / RP;  // passes (MAXH: the largest halo served)
    static constexpr bool WIDE = PRO != PRO_BF16 && !IN_H;    // f32 source: 4 dwords per quad
    static constexpr int NW = WIDE ? 4 : 2;
    static constexpr bool ADAIN = PRO == PRO_ADAIN_LEAKY || PRO == PRO_ADAIN_SNAKE;
    static constexpr bool SNAKE = PRO == PRO_ADAIN_SNAKE;
    uint32_t raw[RB][NW];
    float4 k01, k23;  // AdaIN coefficients (sc, sh) of channels c..c+1 and c+2..c+3
    float4 ar, ai;    // Snake alpha / (2 pi) and 1 / alpha

    // Slab (u, c0): row in0 + r (r = rr + j RP < tw) is read clamped into the item's rows and
    // channel c0 + q as channel 0 past cin (the conversion zeroes both).  Addresses are 32-bit byte
    // offsets from the item's first row (a uniform base), one clamp and one 24-bit multiply-add per
    // row.
    __device__ __forceinline__ void load(const ConvParams& p, const Unit& u, int c0, int tw, int q, int rr) {
        const int c = c0 + q;
        const int cl = c < p.cin ? c : 0;
        constexpr int ES = WIDE ? 4 : 2;  // bytes per element
        const char* base = (const char*)p.x + (int64_t)u.i_lo * p.x_ld * ES;
        const uint32_t ld = (uint32_t)p.x_ld;
        const int r0 = u.in0 - u.i_lo, rmax = u.i_hi - 1 - u.i_lo;  // row offsets from the item start
#pragma unroll
        for (int j = 0; j < RB; j++) {
            // rows past the slab's window re-read its first row (a cache hit, no HBM traffic); the
            // first BN / RP passes lie inside every window (tw >= BN), with no test
            const int r = ((j + 1) * RP <= BN || rr + j * RP < tw) ? rr + j * RP : 0;
            const uint32_t row = (uint32_t)max(min(r0 + r, rmax), 0);
            const uint32_t off = (__umul24(row, ld) + (uint32_t)cl) * ES;
            if constexpr (WIDE) {
                const uint4 x = *(const uint4*)(base + off);
                raw[j][0] = x.x, raw[j][1] = x.y, raw[j][2] = x.z, raw[j][3] = x.w;
            } else {
                const uint2 h = *(const uint2*)(base + off);
                raw[j][0] = h.x, raw[j][1] = h.y;
            }
        }
        if constexpr (ADAIN) {
            const float4* kp = (const float4*)(p.coef + (int64_t)u.item * p.cin + cl);
            k01 = kp[0], k23 = kp[1];
        }
        if constexpr (SNAKE) {
            ar = *(const float4*)(p.alpha_rev + cl);
            ai = *(const float4*)(p.alpha_inv + cl);
        }
    }

    // Converts the slab into LDS rows [r][kRS]: the layer's prologue once per element, rows outside
    // the item (gap masking) and channels past cin as zero, branch-free per row.
    __device__ __forceinline__ void convert(const ConvParams& p, uint16_t* xs, const Unit& u, int c0, int tw, int q,
                                            int rr) const {
        const int c = c0 + q;
#pragma unroll
        for (int j = 0; j < RB; j++)
#pragma unroll
            for (int e = 0; e < NW; e++) ready(raw[j][e]);
        if constexpr (ADAIN) ready(k01), ready(k23);
        if constexpr (SNAKE) ready(ar), ready(ai);
        const float sc[4] = {k01.x, k01.z, k23.x, k23.z}, sh[4] = {k01.y, k01.w, k23.y, k23.w};
        // Snake in its cosine form, with the AdaIN affine folded into both operands (four channel
        // constants per slab, three VALU operations and one cosine per element):
        //   v + sin^2(a v) / a = (v + h) - h cos(2 a v),  h = 1 / (2 a),
        //   2 a v / (2 pi) = x (sc a / pi) + sh a / pi   (__builtin_amdgcn_cosf(t) = cos(2 pi t)).
        float tsc[4], tsh[4], vsh[4], nh[4];
        if constexpr (SNAKE) {
            const float arv[4] = {ar.x, ar.y, ar.z, ar.w}, aiv[4] = {ai.x, ai.y, ai.z, ai.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float a_pi = 2.0f * arv[e], h = 0.5f * aiv[e];  // a / pi, 1 / (2 a)
                tsc[e] = sc[e] * a_pi, tsh[e] = sh[e] * a_pi, vsh[e] = sh[e] + h, nh[e] = -h;
            }
        }
        // Per-slab limits, held in VGPRs for the whole loop (the kernel is short of SGPRs, and a
        // limit rematerialized from the kernel arguments costs a scalar load and a wait per row):
        // live rows r in [r_lo, r_hi), live channels e < n_ch of this quad.
        const int r_lo = vgpr(u.i_lo - u.in0), r_hi = vgpr(min(tw, u.i_hi - u.in0)), n_ch = p.cin - c;
        const uint32_t r_n = (uint32_t)(r_hi - r_lo);
        const float slope = vgpr_f(p.slope);
        uint16_t* xrow = xs + rr * kRS + q;
#pragma unroll
        for (int j = 0; j < RB; j++) {
            const int r = rr + j * RP;
            const bool live = (uint32_t)(r - r_lo) < r_n;
            uint2 out;
            if constexpr (PRO == PRO_BF16) {
                out = make_uint2(raw[j][0], raw[j][1]);  // bf16 input: channels >= cin hold 0
            } else {
                float v[4];
                if constexpr (WIDE) {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = __uint_as_float(raw[j][e]);
                } else {
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        v[2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(raw[j][e] & 0xffffu));
                        v[2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(raw[j][e] >> 16));
                    }
                }
                float w[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    float x = v[e];
                    if constexpr (PRO == PRO_LEAKY) {
                        x = x < 0.f ? x * slope : x;
                    } else if constexpr (PRO == PRO_ADAIN_LEAKY) {
                        x = __builtin_fmaf(x, sc[e], sh[e]);
                        x = x < 0.f ? x * slope : x;
                    } else if constexpr (PRO == PRO_ADAIN_SNAKE) {
                        const float c = __builtin_amdgcn_cosf(__builtin_fmaf(x, tsc[e], tsh[e]));
                        x = __builtin_fmaf(c, nh[e], __builtin_fmaf(x, sc[e], vsh[e]));
                    }
                    // the Snake layers' cin is a multiple of the slab width (checked on the host)
                    if constexpr (!SNAKE) x = e < n_ch ? x : 0.f;
                    w[e] = x;
                }
                out = make_uint2(pack_bf16x2(w[0], w[1]), pack_bf16x2(w[2], w[3]));
            }
            if constexpr (PRO == PRO_BF16) {
                if (!live) out = make_uint2(0, 0);
            } else {
                if (!live || n_ch <= 0) out = make_uint2(0, 0);
            }
            // (a branch per row would keep the compiler from scheduling across rows)
            if ((j + 1) * RP <= BN || r < tw) *(uint2*)(xrow + j * RP * kRS) = out;
        }
    }
};

// ConvT epilogue geometry (kernels/kokoro.cu:452-467 for the reflection pad).  GEMM row m = phase
// ph x cout + co of input column t is output column o = stride t + ph - pad; the wave's 64 rows lie in
// one phase (cout is a multiple of 64).  EPI_CONVT writes y[o] = conv + b + r0[o] for o in the
// item's output span; EPI_CONVT_REFLECT applies ReflectionPad1d((1,0)) per item on the padded
// domain (padded[s] = ups[s + 1], padded[s + 1 + j] = ups[s + j]): it writes row o + 1 for
// o < len - 1, and the item's first row again from o = 1.
struct ConvTGeo {
    int64_t os, ol;  // the item's output span (rows written from ups: [os, os + ol))
    int ph, co;      // this lane's phase and first output channel
};

// Residual operands a stride-1 epilogue reads per 4 output rows.
template <int EPI>
constexpr int kNumRes = EPI == EPI_MEAN3_LEAKY_BF16 ? 3
                        : (EPI == EPI_ACCUM || EPI == EPI_RESID || EPI == EPI_RESID_UP2 || EPI == EPI_ADD_FROM) ? 1
                                                                                                                 : 0;

// Row pointers of one unit: every tensor the epilogue touches, advanced to the unit's first row
// (uniform), so a lane's element offset within the unit fits 32 bits.
struct EpiBase {
    void* y;
    const float *r0, *r1, *r2;
    __amdgpu_buffer_rsrc_t ry;   // y from the unit's first row, as a buffer resource (see store4)
    __amdgpu_buffer_rsrc_t rr0, rr1, rr2;  // EPI_ADD_FROM, EPI_MEAN3_LEAKY_BF16: r0..r2 likewise
};

// fp16 residual operands travel as their raw bits (4 halves in .x and .y) from the load to
// finish4, which widens them: converting at the load would wait for it there.
__device__ __forceinline__ float4 raw_h4(uint2 v) { return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), 0.f, 0.f); }
__device__ __forceinline__ float4 widen_h4(float4 raw) {
    const f16x2_t a = __builtin_bit_cast(f16x2_t, __float_as_uint(raw.x));
    const f16x2_t b = __builtin_bit_cast(f16x2_t, __float_as_uint(raw.y));
    return make_float4((float)a.x, (float)a.y, (float)b.x, (float)b.y);
}

// h + v for the four fp16 values of a raw residual (halves 0, 1 in .x, 2, 3 in .y): one
// v_fma_mix_f32 each, h widened in the instruction, h * one + v with one rounding -- the value that
// widening h and adding it in f32 gives.  `one` is 1.0 held in a VGPR (a literal 1.0 would turn
// the fma back into a widen and an add).
__device__ __forceinline__ float4 add_h4(float4 raw, float4 v, float one) {
    const f16x2_t a = __builtin_bit_cast(f16x2_t, __float_as_uint(raw.x));
    const f16x2_t b = __builtin_bit_cast(f16x2_t, __float_as_uint(raw.y));
    return make_float4(__builtin_fmaf((float)a.x, one, v.x), __builtin_fmaf((float)a.y, one, v.y),
                       __builtin_fmaf((float)b.x, one, v.z), __builtin_fmaf((float)b.y, one, v.w));
}
// The same with both operands raw fp16 residuals.
__device__ __forceinline__ float4 add_hh4(float4 raw_a, float4 raw_b, float one) {
    const f16x2_t b0 = __builtin_bit_cast(f16x2_t, __float_as_uint(raw_b.x));
    const f16x2_t b1 = __builtin_bit_cast(f16x2_t, __float_as_uint(raw_b.y));
    return add_h4(raw_a, make_float4((float)b0.x, (float)b0.y, (float)b1.x, (float)b1.y), one);
}

// x / 3 rounded to nearest, equal to the division x / 3.0f for every finite x (checked over all of
// them, tests/test_div3.py): q = x RN(1/3), the exact remainder as n = 3 q - x (one FMA), then
// Markstein's correction q - n RN(1/3) (one FMA).  The remainder is taken negated so that a zero
// x keeps its sign: x = -0 gives q = -0, n = +0 and -0 + -0 = -0 (with r = x - 3 q, r = +0 and
// the correction would give +0).  Three FMA-unit operations instead of the ~10 of a correctly
// rounded division.
__device__ __forceinline__ float div3(float x) {
    constexpr float kThird = 1.0f / 3.0f;
    const float q = __fmul_rn(x, kThird);
    const float n = __builtin_fmaf(3.0f, q, -x);
    return __builtin_fmaf(-n, kThird, q);
}

// Raw buffer resources (stride 0) of the epilogue's rows: byte offsets are 32-bit, and an offset
// past the range drops a store (see store4)
constexpr int kBufRecords = 0x7fffffff;         // the resource's range in bytes
constexpr uint32_t kDropOffset = 0x80000000u;   // past it: the store is dropped
constexpr int kCpolNT = 2;                      // cache policy: nontemporal
constexpr int kBufFormat = 0x00020000;          // descriptor word 3: 32-bit data format, no swizzle

// Residual operands of output row t, channels m..m+3 (`yo`, `ro`: element offsets from the unit's
// first row in y and r0..r2).
template <int EPI, bool OUT_H>
__device__ __forceinline__ void load_res(const ConvParams& p, const EpiBase& eb, uint32_t yo, uint32_t ro, int64_t t,
                                         int m, float4* r) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    if constexpr (EPI == EPI_ACCUM && OUT_H) {
        // the fp16 rows this epilogue overwrites, streamed like its stores (a buffer load: 32-bit
        // offsets, no 64-bit address arithmetic)
        const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(eb.ry, (int)(yo * 2u), 0, kCpolNT);
        r[0] = raw_h4(make_uint2(v.x, v.y));
    } else if constexpr (EPI == EPI_MEAN3_LEAKY_BF16) {
        const u32x2_t v0 = __builtin_amdgcn_raw_buffer_load_b64(eb.rr0, (int)(ro * 2u), 0, 0);
        const u32x2_t v1 = __builtin_amdgcn_raw_buffer_load_b64(eb.rr1, (int)(ro * 2u), 0, 0);
        const u32x2_t v2 = __builtin_amdgcn_raw_buffer_load_b64(eb.rr2, (int)(ro * 2u), 0, 0);
        r[0] = raw_h4(make_uint2(v0.x, v0.y));
        r[1] = raw_h4(make_uint2(v1.x, v1.y));
        r[2] = raw_h4(make_uint2(v2.x, v2.y));
    } else if constexpr (EPI == EPI_ACCUM || EPI == EPI_RESID) {
        // the rows this epilogue overwrites: streamed (nontemporal), like its stores
        const f32x4 v = __builtin_nontemporal_load((const f32x4*)((const float*)eb.y + yo));
        r[0] = make_float4(v.x, v.y, v.z, v.w);
    } else if constexpr (EPI == EPI_RESID_UP2) {
        r[0] = *(const float4*)(p.r0 + (t >> 1) * p.r0_ld + m);
    } else if constexpr (EPI == EPI_ADD_FROM && OUT_H) {
        const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(eb.rr0, (int)(ro * 2u), 0, 0);
        r[0] = raw_h4(make_uint2(v.x, v.y));
    } else if constexpr (EPI == EPI_ADD_FROM) {
        r[0] = *(const float4*)(eb.r0 + ro);
    }
}

// The residual rule applied to v (conv + bias) of 4 channels of one output row: the values to
// store (the statistics describe these: what the next layer reads).  With fp16 output, `pk` gets
// the fp16 bits.
template <int EPI, bool OUT_H>
__device__ __forceinline__ float4 finish4(const ConvParams& p, float4 v, const float4* r, uint2& pk, float one) {
    if constexpr (EPI == EPI_GELU_BF16) {
        // gelu_new x (1 + tanh u) / 2, u = sqrt(2 / pi) (x + 0.044715 x^3), once per element, as
        // x sigmoid(2 u) = x / (1 + 2^(-2 u log2 e)): one exp2 and one reciprocal (~1 ulp each, far
        // below the bf16 rounding that follows), no cancellation for negative x, and the limits
        // come out exact (2^(+inf) = inf -> -0, 2^(-inf) = 0 -> x).  Stored as the bf16 operand
        // the next linear's MFMA reads (round to nearest even, as its f32 prologue would do).
        constexpr float k2ul = 2.0f * 0.797884560802865355f * 1.44269504088896341f;
        float g[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float x = g[e];
            const float t = __builtin_amdgcn_exp2f(-k2ul * __builtin_fmaf(0.044715f * x, x * x, x));
            g[e] = x * __builtin_amdgcn_rcpf(1.0f + t);
        }
        pk = make_uint2(pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3]));
        return v;
    } else if constexpr (EPI == EPI_MEAN3_LEAKY_BF16) {
        // ((rb0 + rb1) + (rb2_resid + conv)) / 3 (src/gpu_batch.rs:395-401) from the three fp16
        // residual streams, then the next layer's prologue (leaky ReLU, round to nearest even bf16):
        // the same operand bits that layer's PRO_LEAKY staging would produce
        const float4 ab = add_hh4(r[0], r[1], one), cv = add_h4(r[2], v, one);
        const float o[4] = {div3(ab.x + cv.x), div3(ab.y + cv.y), div3(ab.z + cv.z), div3(ab.w + cv.w)};
        // leaky ReLU as max(o, slope o): equal to o < 0 ? slope o : o for 0 < slope <= 1 (the
        // launch refuses other slopes), zeros' signs included
        const float slope = p.slope;
        float w[4];
#pragma unroll
        for (int e = 0; e < 4; e++) w[e] = __builtin_fmaxf(o[e], o[e] * slope);
        pk = make_uint2(pack_bf16x2(w[0], w[1]), pack_bf16x2(w[2], w[3]));
        return make_float4(o[0], o[1], o[2], o[3]);
    } else if constexpr (OUT_H && EPI == EPI_STORE) {
        // fp16 storage; the statistics describe the stored fp16 values (what the next layer reads;
        // ~2^-12 relative from the f32 values the reference's f32 h would give, far below the next
        // layer's bf16 operand rounding)
        pk = make_uint2(pack_f16x2(v.x, v.y), pack_f16x2(v.z, v.w));
        return v;
    }
    float4 o = v;
    if constexpr (EPI == EPI_ACCUM || EPI == EPI_ADD_FROM) {
        // an fp16 residual stream: the sum in f32, stored rounded to fp16 (statistics as above)
        if constexpr (OUT_H) {
            o = add_h4(r[0], v, one);
            pk = make_uint2(pack_f16x2(o.x, o.y), pack_f16x2(o.z, o.w));
        } else {
            const float4 y = r[0];
            o = make_float4(y.x + v.x, y.y + v.y, y.z + v.z, y.w + v.w);
        }
    } else if constexpr (EPI == EPI_RESID || EPI == EPI_RESID_UP2) {
        const float4 y = r[0];
        const float s = p.scale;
        o = make_float4((v.x + y.x) * s, (v.y + y.y) * s, (v.z + y.z) * s, (v.w + y.w) * s);
    }
    return o;
}

// Stores one row's result at element offset `yo` from the unit's first row of y, if `ok`.
// Buffer stores: a store of a lane that must not write gets a byte offset past the resource's
// range and is dropped by the hardware's range check, so no branch surrounds the store.  (Branches
// around stores make the compiler's vector-memory wait counts assume the store was skipped and
// wait for it on the other path: a residual load issued after a store would be waited for together
// with that store.)  Nontemporal: the layer's output is read again only by the next launch, so it
// streams through L2 instead of evicting the weights the A fragments reload every tap (1.4% of the
// Snake convs' time on the benchmark configuration).
template <bool OUT_H>
__device__ __forceinline__ void store4(const EpiBase& eb, uint32_t yo, bool ok, float4 o, uint2 pk) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const uint32_t off = ok ? yo * (OUT_H ? 2u : 4u) : kDropOffset;
    if constexpr (OUT_H) {
        __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){pk.x, pk.y}, eb.ry, (int)off, 0, kCpolNT);
    } else {
        __builtin_amdgcn_raw_buffer_store_b128(
            (u32x4_t){__float_as_uint(o.x), __float_as_uint(o.y), __float_as_uint(o.z), __float_as_uint(o.w)}, eb.ry,
            (int)off, 0, kCpolNT);
    }
}

// store4 with the byte offset given (kDropOffset: no store)
template <bool OUT_H>
__device__ __forceinline__ void store4b(const EpiBase& eb, uint32_t off, float4 o, uint2 pk) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    if constexpr (OUT_H) {
        __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){pk.x, pk.y}, eb.ry, (int)off, 0, kCpolNT);
    } else {
        __builtin_amdgcn_raw_buffer_store_b128(
            (u32x4_t){__float_as_uint(o.x), __float_as_uint(o.y), __float_as_uint(o.z), __float_as_uint(o.w)}, eb.ry,
            (int)off, 0, kCpolNT);
    }
}

constexpr int kScrLd = 64 + 4;  // epilogue LDS scratch row stride (f32): one time column, 64 channels
constexpr int kScrLd16 = 32 + 2;  // the same in 32-bit words for fp16 values (two buffers fit one f32 one)
constexpr int kMaxBias = 1152;  // bias vector staged in LDS (output rows, M_pad)

// Starts a unit's accumulators at its bias (stride-1 layers): element 4 g + r of MFMA tile (i, j)
// is output row i 32 + 8 g + 4 lh + r of the wave's 32 MI rows, for every column.  ConvT layers
// (bias per output channel of a phase, added in their scatter) start from zero.
template <bool BIAS, int MI = 2>
__device__ __forceinline__ void init_acc(f32x16 (&acc)[MI][4], const float* bias_s, int m0, int wm, int lane) {
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float4 bv = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (BIAS) bv = *(const float4*)(bias_s + m0 + wm * 32 * MI + i * 32 + 8 * g + 4 * (lane >> 5));
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc[i][j][4 * g] = bv.x, acc[i][j][4 * g + 1] = bv.y;
                acc[i][j][4 * g + 2] = bv.z, acc[i][j][4 * g + 3] = bv.w;
            }
        }
}

// Epilogue of one unit: residual rule, stores, statistics partials; then starts the accumulators of
// the block's next unit (at its bias, or zero for ConvT).
// The MFMA layout gives each lane 4 channels of one column (D of tile (i, j): rows i*32 + 8 g + 4 lh
// + r of column j*32 + l32), so stores straight from it would scatter 8-16 byte pieces over 32
// rows.  Instead the wave transposes each 32-column slice through its LDS scratch ([32][kScrLd]
// f32): afterwards 16 lanes hold one column's 64 channels (lane group cg = column, cq = channel
// quad), so every store and residual load covers whole 256-byte column rows, and the statistics
// accumulate per lane over columns with one cross-group reduction at the end.
// FULL: every column of the wave and every row of the unit is valid (no masks).
template <int EPI, int WM, int WN, bool STATS, bool OUT_H, bool FULL>
__device__ __forceinline__ void epilogue(const ConvParams& p, const Unit& u, f32x16 (&acc)[2][4], int wm, int wn,
                                         int lane, float* scr, const float* bias_s, int next_m0) {
    constexpr bool CONVT = EPI == EPI_CONVT || EPI == EPI_CONVT_REFLECT;
    constexpr int NR = CONVT ? 1 : kNumRes<EPI>;
    constexpr int NRA = NR > 0 ? NR : 1;
    // fp16 residuals: the streams of the fp16 accumulations, the means and the ConvTs' noise branch
    constexpr bool RES_H = ((EPI == EPI_ACCUM || EPI == EPI_ADD_FROM || CONVT) && OUT_H) || EPI == EPI_MEAN3_LEAKY_BF16;
    constexpr int QB = NR > 1 && !RES_H ? 2 : (NR >= 1 ? 4 : 8);  // column groups per batch
    const int l32 = lane & 31, lh = lane >> 5;
    const int cq = lane & 15, cg = lane >> 4;
    const int wcol0 = wn * 128;                // this wave's first column within the tile
    const int m = u.m0 + wm * 64 + 4 * cq;     // this lane's 4 output rows after the transpose
    const bool mok = FULL || m < p.m;
    // ConvT: the item's output span (uniform, scalar loads), the lane's phase / channel and bias,
    // all once per unit
    ConvTGeo cg_ = {0, 0, 0, 0};
    float4 cb = make_float4(0.f, 0.f, 0.f, 0.f), rfl = cb;
    int64_t ubase = 0;  // ConvT: the first output row the unit can write (its stores' base)
    if constexpr (CONVT) {
        cg_.os = ld_const(p.out_start, u.item);
        cg_.ol = ld_const(p.out_len, u.item) - (EPI == EPI_CONVT_REFLECT ? 1 : 0);
        const int mm = mok ? m : u.m0;
        cg_.ph = mm / p.cout, cg_.co = mm - cg_.ph * p.cout;
        cb = *(const float4*)(p.bias + cg_.co);
        // rows o >= stride n0 - pad (o + 1 with the reflection pad), and the item's first row when
        // the unit writes o = os + 1 (then stride n0 - pad - 1 <= os); as convt_cols computes it
        ubase = max(cg_.os, (int64_t)p.stride_t * u.n0 - p.pad_t - 1);
        // the reflected row's residual: r0 at the item's first row
        if constexpr (EPI == EPI_CONVT_REFLECT) {
            if constexpr (OUT_H)
                rfl = widen_h4(raw_h4(*(const uint2*)((const uint16_t*)p.r0 + cg_.os * p.r0_ld + cg_.co)));
            else
                rfl = *(const float4*)(p.r0 + cg_.os * p.r0_ld + cg_.co);
        }
        ready(cb);
    }
    // ConvT: the columns this lane writes, [lo, hi), and each one's row relative to ubase,
    // rel0 + stride col (kk_walk.h convt_cols, checked on the CPU).  The lane's columns are
    // wcol0 + cg + 4 k for k = 8 j + q < 32, so the valid ones are k in [ct_klo, ct_klo + ct_kn)
    // (one subtract and one unsigned compare per column), and column k's element offsets in y and
    // r0 are ct_y0 + k ct_dy and ct_q0 + k ct_dq (ct_dy, ct_dq uniform: one add per column).
    // Other columns store nothing and read the residual at the unit's first row.
    // ct_krefl: the k whose column also fills the item's first row (the reflection pad), or -1.
    int ct_klo = 0, ct_kn = 0, ct_krefl = -1;
    uint32_t ct_y0 = 0, ct_q0 = 0, ct_dy = 0, ct_dq = 0;
    if constexpr (CONVT) {
        const ConvTCols cc = convt_cols(u.n0, u.nv, p.stride_t, p.pad_t, cg_.ph, cg_.os, cg_.ol,
                                        EPI == EPI_CONVT_REFLECT, mok);
        const int bcol = wcol0 + cg;
        const int klo = min(max((cc.lo - bcol + 3) >> 2, 0), 32);  // ceil((lo - bcol) / 4), clamped
        const int khi = min(max((cc.hi - bcol + 3) >> 2, 0), 32);
        ct_klo = klo, ct_kn = max(khi - klo, 0);
        if (cc.refl >= bcol && cc.refl - bcol < 128 && ((cc.refl - bcol) & 3) == 0) ct_krefl = (cc.refl - bcol) >> 2;
        const uint32_t row0 = (uint32_t)(cc.rel0 + p.stride_t * bcol);  // column k = 0 (wraps when invalid)
        ct_y0 = row0 * (uint32_t)p.y_ld + (uint32_t)cg_.co, ct_q0 = row0 * (uint32_t)p.r0_ld + (uint32_t)cg_.co;
        ct_dy = 4u * (uint32_t)p.stride_t * (uint32_t)p.y_ld, ct_dq = 4u * (uint32_t)p.stride_t * (uint32_t)p.r0_ld;
    }
    // (FULL ConvT units lie inside their item's span with every row valid: all 32 columns write)
    auto ct_ok = [&](int k) { return FULL || (uint32_t)(k - ct_klo) < (uint32_t)ct_kn; };
    // Row pointers at the unit's first row (uniform) and this lane's 32-bit element offsets of its
    // first output row (column wcol0 + cg); row wcol0 + cg + c adds c * ld, one 24-bit multiply
    // with ld held in a VGPR (uniform products of every c would occupy scalar registers).
    EpiBase eb;
    const int64_t n0 = u.n0;
    eb.y = OUT_H ? (void*)((uint16_t*)p.y + n0 * p.y_ld) : (void*)(p.y + n0 * p.y_ld);
    if constexpr (CONVT) eb.y = OUT_H ? (void*)((uint16_t*)p.y + ubase * p.y_ld) : (void*)(p.y + ubase * p.y_ld);
    eb.ry = __builtin_amdgcn_make_buffer_rsrc(eb.y, 0, kBufRecords, kBufFormat);  // raw (stride 0) buffer
    eb.r0 = eb.r1 = eb.r2 = nullptr;
    if constexpr (EPI == EPI_ADD_FROM) {
        eb.r0 = OUT_H ? (const float*)((const uint16_t*)p.r0 + n0 * p.r0_ld) : p.r0 + n0 * p.r0_ld;
        eb.rr0 = __builtin_amdgcn_make_buffer_rsrc((void*)eb.r0, 0, kBufRecords, kBufFormat);
    }
    if constexpr (EPI == EPI_MEAN3_LEAKY_BF16) {  // fp16 rows, addressed as such in load_res
        eb.r0 = (const float*)((const uint16_t*)p.r0 + n0 * p.r0_ld);
        eb.r1 = (const float*)((const uint16_t*)p.r1 + n0 * p.r0_ld);
        eb.r2 = (const float*)((const uint16_t*)p.r2 + n0 * p.r0_ld);
        eb.rr0 = __builtin_amdgcn_make_buffer_rsrc((void*)eb.r0, 0, kBufRecords, kBufFormat);
        eb.rr1 = __builtin_amdgcn_make_buffer_rsrc((void*)eb.r1, 0, kBufRecords, kBufFormat);
        eb.rr2 = __builtin_amdgcn_make_buffer_rsrc((void*)eb.r2, 0, kBufRecords, kBufFormat);
    }
    const uint32_t yld = (uint32_t)vgpr((int)p.y_ld), rld = (uint32_t)vgpr((int)p.r0_ld);
    const uint32_t yo0 = (uint32_t)(wcol0 + cg) * yld + m, ro0 = (uint32_t)(wcol0 + cg) * rld + m;
    const uint32_t yz = u.m0, rz = u.m0;  // clamped operand of an invalid row: row 0 of the unit
    float s1[4] = {0.f, 0.f, 0.f, 0.f}, s2[4] = {0.f, 0.f, 0.f, 0.f}, sft[4] = {0.f, 0.f, 0.f, 0.f};
    // fp16 outputs (h and the generator's streams): the statistics of the stored fp16 values, two
    // columns of a channel per instruction -- the pair's shifted values d (v_pk_add_f16; exact
    // when a value is within a factor 2 of the shift, else rounded to fp16), then sum d and sum d^2
    // accumulated in f32 by v_dot2c_f32_f16 (products exact) -- 2 instructions per value instead of
    // 3 in f32
    constexpr bool HSTATS = STATS && OUT_H && !CONVT;
    // fp16 transpose (below) for plain fp16 stores.  (Not for the fp16 accumulations: rounding their
    // conv + bias to fp16 before the residual is added measured -0.07 ms and moved the audio by
    // -46 dB, too much of the parity margin.)
    constexpr bool H16T = OUT_H && EPI == EPI_STORE && (HSTATS || !STATS);
    f16x2_t sftp[4] = {};  // the shift of channel r, in both halves
    float cnt = 0.f;  // ConvT: rows this lane group wrote (the statistics' count)
    // Batches of QB column groups, BPS per 32-column slice.  The residual loads of batch b + LEAD are
    // issued before batch b's stores: vector-memory counters complete in issue order (stores
    // included), so a load issued after a store could only be waited for together with that store.
    constexpr int BPS = 8 / QB, NB = 4 * BPS;
    // Two batches ahead for the one-residual fp16 epilogues (the ConvTs' noise stream, the
    // resblocks' fp16 streams: rows read from HBM; the stage-1 ConvT 397 -> 373 us, kernel-only
    // -0.13 ms on the benchmark configuration), but for the 256-channel accumulate with statistics,
    // which would spill.
    constexpr int LEAD = NR > 0 ? ((CONVT || (RES_H && NR == 1 && !(WM == 4 && EPI == EPI_ACCUM && STATS))) ? 2 : 1) : 0;
    constexpr int RING = LEAD + 1;
    float4 res[RING][QB][NRA];
    const float one = vgpr_f(1.0f);  // the fp16 residuals' fma_mix multiplier (add_h4)
    // ConvT: the residual from the unit's first writable row (its element type as y's), as a raw
    // buffer
    const __amdgpu_buffer_rsrc_t ct_r0 = __builtin_amdgcn_make_buffer_rsrc(
        !CONVT ? nullptr
        : OUT_H ? (void*)((const uint16_t*)p.r0 + ubase * p.r0_ld)
                : (void*)(p.r0 + ubase * p.r0_ld),
        0, kBufRecords, kBufFormat);
    float4 ct_rsv = make_float4(0.f, 0.f, 0.f, 0.f);  // REFLECT: conv + bias of column ct_krefl
    // unconditional loads (invalid columns / rows read column 0 / row 0 of the tile)
    auto issue = [&](int b) {
        const int j = b / BPS, q0 = (b % BPS) * QB;
#pragma unroll
        for (int qq = 0; qq < QB; qq++) {
            const int c = j * 32 + 4 * (q0 + qq);
            if constexpr (CONVT) {
                typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
                typedef float f32x4_t __attribute__((ext_vector_type(4)));
                const int k = c / 4;
                // (an invalid column reads the unit's first row: its value can still be the
                // statistics' shift, which should be near the data)
                const uint32_t off = (ct_ok(k) ? ct_q0 + (uint32_t)k * ct_dq : (uint32_t)cg_.co) * (OUT_H ? 2u : 4u);
                if constexpr (OUT_H) {
                    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(ct_r0, (int)off, 0, 0);
                    res[b % RING][qq][0] = raw_h4(make_uint2(v.x, v.y));
                } else {
                    const f32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(ct_r0, (int)off, 0, 0);
                    res[b % RING][qq][0] = make_float4(v.x, v.y, v.z, v.w);
                }
            } else {
                const bool ok = FULL || (wcol0 + c + cg < u.nv && mok);
                load_res<EPI, OUT_H>(p, eb, ok ? yo0 + __umul24(c, yld) : yz, ok ? ro0 + __umul24(c, rld) : rz,
                              ok ? n0 + wcol0 + cg + c : n0, ok ? m : u.m0, res[b % RING][qq]);
            }
        }
    };
    if constexpr (NR > 0) {
#pragma unroll
        for (int b = 0; b < LEAD; b++) issue(b);
    }
    // Plain fp16 stores (conv1 of the Snake steps: h): the values are rounded to fp16 before the
    // transpose (what is stored, and what the statistics describe), so a slice takes half the LDS
    // traffic and two slices fit the scratch: slice j + 1 is written while slice j is read.
    uint32_t* scr16 = (uint32_t*)scr;
    auto put16 = [&](int jj) {
        uint32_t* d = scr16 + (jj & 1) * 32 * kScrLd16 + l32 * kScrLd16 + 2 * lh;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(uint2*)(d + 16 * i + 4 * g) = make_uint2(pack_f16x2(acc[i][jj][4 * g], acc[i][jj][4 * g + 1]),
                                                           pack_f16x2(acc[i][jj][4 * g + 2], acc[i][jj][4 * g + 3]));
    };
    if constexpr (H16T) {
        put16(0);
        __builtin_amdgcn_wave_barrier();  // LDS operations of one wave execute in order
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int j = b / BPS, q0 = (b % BPS) * QB;
        if (!H16T && b % BPS == 0) {
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    *(float4*)(scr + l32 * kScrLd + i * 32 + 8 * g + 4 * lh) = make_float4(
                        acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]);
            __builtin_amdgcn_wave_barrier();  // LDS operations of one wave execute in order
        }
        {
            if constexpr (NR > 0) {
                if (b + LEAD < NB) issue(b + LEAD);
            }
            // all LDS reads of the batch first, one wait, then the arithmetic and the stores
            float4 v[QB];
            uint2 v16[QB];
            if constexpr (H16T) {
                // this slice's reads, then the next slice's writes into the other buffer (issued
                // after the reads, so the wait below covers only the reads)
#pragma unroll
                for (int qq = 0; qq < QB; qq++)
                    v16[qq] = *(const uint2*)(scr16 + (j & 1) * 32 * kScrLd16 + (4 * (q0 + qq) + cg) * kScrLd16 + 2 * cq);
                __builtin_amdgcn_wave_barrier();
                if (j + 1 < 4 && b % BPS == BPS - 1) put16(j + 1);
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int qq = 0; qq < QB; qq++) ready(v16[qq].x), ready(v16[qq].y);
            } else {
#pragma unroll
                for (int qq = 0; qq < QB; qq++) v[qq] = *(const float4*)(scr + (4 * (q0 + qq) + cg) * kScrLd + 4 * cq);
#pragma unroll
                for (int qq = 0; qq < QB; qq++) ready(v[qq]);
            }
            float4(&rc)[QB][NRA] = res[b % RING];
            if constexpr (NR > 0) {
#pragma unroll
                for (int qq = 0; qq < QB; qq++)
#pragma unroll
                    for (int e = 0; e < NRA; e++) {
                        if constexpr (RES_H) {  // raw fp16 bits in .x and .y only
                            ready(__float_as_uint(rc[qq][e].x));
                            ready(__float_as_uint(rc[qq][e].y));
                        } else {
                            ready(rc[qq][e]);
                        }
                    }
            }
            uint2 pkq[QB];  // HSTATS: each column group's stored fp16 values
            bool vq[QB];
#pragma unroll
            for (int qq = 0; qq < QB; qq++) {
                const int q = q0 + qq;
                const int col = wcol0 + j * 32 + 4 * q + cg;
                bool valid = FULL || col < u.nv;
                // the values are computed for every row (they feed the statistics, masked there);
                // only the store is conditional
                float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
                if constexpr (CONVT) {
                    const int k = 8 * j + q;
                    const bool ok = ct_ok(k);
                    const float4 w = make_float4(v[qq].x + cb.x, v[qq].y + cb.y, v[qq].z + cb.z, v[qq].w + cb.w);
                    if constexpr (OUT_H) {
                        o = add_h4(rc[qq][0], w, one);  // + the fp16 noise stream
                    } else {
                        const float4 r = rc[qq][0];
                        o = make_float4(w.x + r.x, w.y + r.y, w.z + r.z, w.w + r.w);
                    }
                    valid = ok;
                    // fp16 output: the stage input of the resblocks' fp16 streams
                    const uint2 pk = OUT_H ? make_uint2(pack_f16x2(o.x, o.y), pack_f16x2(o.z, o.w)) : make_uint2(0u, 0u);
                    store4b<OUT_H>(eb, ok ? (ct_y0 + (uint32_t)k * ct_dy) * (OUT_H ? 2u : 4u) : kDropOffset, o, pk);
                    if constexpr (EPI == EPI_CONVT_REFLECT && !FULL) {
                        if (k == ct_krefl) ct_rsv = w;  // stored after the last column
                    }
                    if constexpr (STATS) cnt += ok ? 1.f : 0.f;
                } else {
                    uint2 pk;  // v = conv + bias (the accumulators started at the bias)
                    if constexpr (H16T)
                        pk = v16[qq];  // rounded before the transpose (finish4's rule for this case)
                    else
                        o = finish4<EPI, OUT_H>(p, v[qq], rc[qq], pk, one);
                    store4<OUT_H>(eb, yo0 + __umul24(j * 32 + 4 * q, yld), valid && mok, o, pk);
                    pkq[qq] = pk, vq[qq] = valid;
                    if constexpr (HSTATS) {
                        if (j == 0 && q == 0) {  // the wave's first column: lanes cq of lane group 0
                            const f16x2_t h01 = __builtin_bit_cast(f16x2_t, (uint32_t)__shfl((int)pk.x, cq, 64));
                            const f16x2_t h23 = __builtin_bit_cast(f16x2_t, (uint32_t)__shfl((int)pk.y, cq, 64));
                            sftp[0] = __builtin_shufflevector(h01, h01, 0, 0);
                            sftp[1] = __builtin_shufflevector(h01, h01, 1, 1);
                            sftp[2] = __builtin_shufflevector(h23, h23, 0, 0);
                            sftp[3] = __builtin_shufflevector(h23, h23, 1, 1);
#pragma unroll
                            for (int r = 0; r < 4; r++) sft[r] = (float)sftp[r].x;
                        }
                        if (qq % 2 == 1) {  // the pair (qq - 1, qq): channel r of the two columns
                            const f16x2_t a01 = __builtin_bit_cast(f16x2_t, pkq[qq - 1].x);
                            const f16x2_t a23 = __builtin_bit_cast(f16x2_t, pkq[qq - 1].y);
                            const f16x2_t b01 = __builtin_bit_cast(f16x2_t, pk.x), b23 = __builtin_bit_cast(f16x2_t, pk.y);
                            f16x2_t d[4] = {__builtin_shufflevector(a01, b01, 0, 2), __builtin_shufflevector(a01, b01, 1, 3),
                                            __builtin_shufflevector(a23, b23, 0, 2), __builtin_shufflevector(a23, b23, 1, 3)};
                            const uint32_t keep = (vq[qq - 1] ? 0x0000ffffu : 0u) | (valid ? 0xffff0000u : 0u);
                            const f16x2_t one2 = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
                            for (int r = 0; r < 4; r++) {
                                d[r] = d[r] - sftp[r];
                                if constexpr (!FULL)
                                    d[r] = __builtin_bit_cast(f16x2_t, __builtin_bit_cast(uint32_t, d[r]) & keep);
                                s1[r] = __builtin_amdgcn_fdot2(d[r], one2, s1[r], false);
                                s2[r] = __builtin_amdgcn_fdot2(d[r], d[r], s2[r], false);
                            }
                        }
                    }
                }
                if constexpr (STATS && !HSTATS) {
                    const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        if (j == 0 && q == 0) sft[r] = __shfl(ov[r], cq, 64);  // the wave's first column
                        const float d = valid ? ov[r] - sft[r] : 0.f;
                        s1[r] += d;
                        s2[r] = __builtin_fmaf(d, d, s2[r]);
                    }
                }
            }
        }
        if (b % BPS == BPS - 1) __builtin_amdgcn_wave_barrier();  // the slice's LDS reads before the next writes
    }
    if constexpr (EPI == EPI_CONVT_REFLECT && !FULL) {
        // column ct_krefl (o = os + 1) also fills the item's first row (the reflected sample): its
        // conv + bias plus r0 at that row; ct_krefl >= 0 only in the unit whose first row is os
        // (ubase = os there).  The statistics leave this row to finalize, which reads it back.
        const float4 f = make_float4(ct_rsv.x + rfl.x, ct_rsv.y + rfl.y, ct_rsv.z + rfl.z, ct_rsv.w + rfl.w);
        const uint2 fk = OUT_H ? make_uint2(pack_f16x2(f.x, f.y), pack_f16x2(f.z, f.w)) : make_uint2(0u, 0u);
        store4b<OUT_H>(eb, ct_krefl >= 0 ? (uint32_t)cg_.co * (OUT_H ? 2u : 4u) : kDropOffset, f, fk);
    }
    if constexpr (STATS) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            s1[r] += __shfl_xor(s1[r], 16, 64);
            s2[r] += __shfl_xor(s2[r], 16, 64);
            s1[r] += __shfl_xor(s1[r], 32, 64);
            s2[r] += __shfl_xor(s2[r], 32, 64);
        }
        if constexpr (CONVT) {
            cnt += __shfl_xor(cnt, 16, 64);
            cnt += __shfl_xor(cnt, 32, 64);
        }
        // every wave writes its record, an empty one (n = 0) when the tile ends before its columns;
        // ConvT: one record per (tile, phase, wave column), over the rows the wave wrote
        if (cg == 0) {
            StatPart* dst = CONVT ? p.part + (((int64_t)u.tile * p.stride_t + cg_.ph) * WN + wn) * p.cout + cg_.co
                                  : p.part + ((int64_t)u.tile * WN + wn) * p.cout + m;
            const float nc = CONVT ? cnt : (float)max(min(u.nv - wcol0, 128), 0);
#pragma unroll
            for (int r = 0; r < 4; r++)
                if (mok && (CONVT ? cg_.co : m) + r < p.cout)
                    dst[r] = nc > 0.f ? StatPart{s1[r], s2[r], sft[r], nc} : StatPart{0.f, 0.f, 0.f, 0.f};
        }
    }
    init_acc<!CONVT>(acc, bias_s, next_m0, wm, lane);  // the next unit starts at its bias
}

// Epilogue of a wave with one 32-row MFMA tile per column tile (layers of at most 32 output rows:
// conv_post): plain stores of conv + bias.  Each 32-column slice goes through the wave's LDS scratch
// ([32 columns][kScrLd32] f32), after which 8 lanes hold one column's 32 rows (lane group cg = lane /
// 8 of 8 columns, cq = lane % 8 a quad of rows), so a store covers 8 columns' 128-byte row pieces.
constexpr int kScrLd32 = 32 + 4;
template <int WN>
__device__ __forceinline__ void epilogue_m32(const ConvParams& p, const Unit& u, f32x16 (&acc)[1][4], int wm, int wn,
                                             int lane, float* scr, const float* bias_s, int next_m0) {
    const int l32 = lane & 31, lh = lane >> 5;
    const int cq = lane & 7, cg = lane >> 3;
    const int wcol0 = wn * 128;
    const int m = u.m0 + wm * 32 + 4 * cq;  // this lane's 4 output rows after the transpose
    const bool mok = m < p.m;
    EpiBase eb;
    eb.y = p.y + (int64_t)u.n0 * p.y_ld;
    eb.ry = __builtin_amdgcn_make_buffer_rsrc(eb.y, 0, kBufRecords, kBufFormat);
    eb.r0 = eb.r1 = eb.r2 = nullptr;
    const uint32_t yld = (uint32_t)vgpr((int)p.y_ld);
    const uint32_t yo0 = (uint32_t)(wcol0 + cg) * yld + m;
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int g = 0; g < 4; g++)
            *(float4*)(scr + l32 * kScrLd32 + 8 * g + 4 * lh) =
                make_float4(acc[0][j][4 * g], acc[0][j][4 * g + 1], acc[0][j][4 * g + 2], acc[0][j][4 * g + 3]);
        __builtin_amdgcn_wave_barrier();  // LDS operations of one wave execute in order
        float4 v[4];
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = *(const float4*)(scr + (8 * q + cg) * kScrLd32 + 4 * cq);
#pragma unroll
        for (int q = 0; q < 4; q++) ready(v[q]);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int c = j * 32 + 8 * q;  // column of lane group 0 within the wave
            const uint2 nopk = make_uint2(0u, 0u);
            store4<false>(eb, yo0 + __umul24(c, yld), wcol0 + c + cg < u.nv && mok, v[q], nopk);
        }
        __builtin_amdgcn_wave_barrier();  // the slice's LDS reads before the next writes
    }
    init_acc<true, 1>(acc, bias_s, next_m0, wm, lane);  // the next unit starts at its bias
}

// MI: 32-row MFMA tiles per wave (2: 64 x 128 outputs per wave; 1: 32 x 128, layers of at most 32
// output rows, plain stores).
template <int PRO, int EPI, int WM, int WN, bool STATS, bool IN_H, bool OUT_H, int MAXH, int MI = 2>
__global__ __launch_bounds__(64 * WM * WN + kNP) void conv_mfma_kernel(ConvParams p) {
    constexpr int BM = 32 * MI * WM, BN = 16 * kNJ * WN, NC = 64 * WM * WN;
    static_assert(MI == 2 || (EPI == EPI_STORE && !STATS && !OUT_H), "32-row waves: plain f32 stores only");
    extern __shared__ __align__(16) uint16_t xs[];
    const int mblocks = p.m_pad / BM;
    const int tw = BN + (p.k - 1) * p.dil;
    const int slab_elems = tw * kRS;
    const int nsl = p.cin_pad / kCK;

    // Units: U = g * 8 * mblocks + w * 8 + x is M-block w of tile g * 8 + x.  Block b runs units
    // b, b + G, b + 2G, ... (G = gridDim.x, a multiple of 8 * mblocks, so b keeps its w and x).
    // Workgroup slots go to the 8 XCDs round-robin: block b stays on XCD x.
    auto unit_at = [&](int U, Unit& u) -> bool {
        if (!walk_unit(U, mblocks, BM, p.tiles.count, u.tile, u.m0)) return false;
        u.item = ld_const(p.tiles.item, u.tile);
        u.n0 = (int)ld_const(p.tiles.t0, u.tile);
        u.nv = ld_const(p.tiles.n, u.tile);
        u.i_lo = (int)ld_const(p.in_start, u.item);
        u.i_hi = u.i_lo + (int)ld_const(p.in_len, u.item);
        u.in0 = u.n0 - p.pad;
        return true;
    };
    // slabs this block runs: units b + i G with tile g_i * 8 + x < count, g_i = g_0 + i * (G / grp)
    const int n_units = walk_n_units(blockIdx.x, gridDim.x, mblocks, p.tiles.count);
    const int G = n_units * nsl;
    if (G == 0) return;

    if (threadIdx.x >= NC) {
        // ------------------------------------------------------------ producer waves
        // Two register slots: the loads of step n + 2 are in flight while step n + 1 is converted.
        // Every load is issued unconditionally (past the last step the load iterator repeats its
        // last unit), so the number of loads in flight is the same at every wait.
        const int pt = threadIdx.x - NC;
        const int q = (pt & 15) * 4, rr = pt >> 4;
        Slot<PRO, IN_H, BN, MAXH> s0, s1;
        // iterators over (unit, slab) steps: load and convert
        int lU = blockIdx.x, ls = 0, cU = blockIdx.x, cs = 0;
        Unit lu, cuv;
        unit_at(lU, lu);
        cuv = lu;
        auto adv_l = [&]() {
            if (++ls == nsl) {
                Unit t;
                ls = 0;
                lU += gridDim.x;
                if (unit_at(lU, t)) lu = t;
            }
        };
        auto adv_c = [&]() {
            if (++cs == nsl) {
                cs = 0;
                cU += gridDim.x;
                unit_at(cU, cuv);
            }
        };
        s0.load(p, lu, ls * kCK, tw, q, rr);
        adv_l();
        s1.load(p, lu, ls * kCK, tw, q, rr);
        adv_l();
        s0.convert(p, xs, cuv, cs * kCK, tw, q, rr);
        adv_c();
        s0.load(p, lu, ls * kCK, tw, q, rr);
        adv_l();
        __syncthreads();
        for (int g = 0; g < G; g += 2) {
            // step g: convert step g + 1 (slot 1), then load step g + 3 into slot 1
            if (g + 1 < G) {
                s1.convert(p, xs + slab_elems, cuv, cs * kCK, tw, q, rr);
                adv_c();
            }
            s1.load(p, lu, ls * kCK, tw, q, rr);
            adv_l();
            __syncthreads();
            if (g + 1 >= G) break;
            // step g + 1: convert step g + 2 (slot 0), then load step g + 4 into slot 0
            if (g + 2 < G) {
                s0.convert(p, xs, cuv, cs * kCK, tw, q, rr);
                adv_c();
            }
            s0.load(p, lu, ls * kCK, tw, q, rr);
            adv_l();
            __syncthreads();
        }
        return;
    }

    // ---------------------------------------------------------------- consumer waves
    // v_mfma_f32_32x32x16_bf16 lane layouts (l32 = lane % 32, lh = lane / 32): A[l32][8 lh + e],
    // B[8 lh + e][l32], D[8 (r / 4) + 4 lh + r % 4][l32] for r < 16.  One wave issuing 32x32 MFMAs
    // back to back keeps the matrix core busy; the 16x16 shape needs two waves per SIMD.
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = wave % WM, wn = wave / WM;
    const int l32 = lane & 31, lh = lane >> 5;
    // this wave's epilogue scratch, after the two slab buffers
    float* scr = (float*)(xs + 2 * slab_elems) + wave * 32 * kScrLd;
    const int n16 = p.cin_pad / 16;               // 16-channel groups
    const int64_t a_step = (int64_t)p.m_pad * 2;  // one 16-channel group of A, in bf16x8
    const bf16x8* w_lane = (const bf16x8*)p.w + (int64_t)(wm * 32 * MI + l32) * 2 + lh;
    // A fragments of tap kk, 16-channel group c16: rows m0 + wm*32*MI + i*32 + l32 (i < MI)
    auto load_a = [&](bf16x8 (&dst)[MI], int m0, int kk, int c16) {
        const bf16x8* ap = w_lane + (int64_t)m0 * 2 + ((int64_t)kk * n16 + c16) * a_step;
#pragma unroll
        for (int i = 0; i < MI; i++) dst[i] = ap[64 * i];
    };
    // B fragments of tap kk, 16-channel step kc of the slab: columns wn*128 + j*32 + l32 (j < 4)
    auto read_b = [&](bf16x8 (&dst)[4], const uint16_t* buf, int kk, int kc) {
        const uint16_t* bp = buf + (wn * 128 + kk * p.dil + l32) * kRS + kc * 16 + lh * 8;
#pragma unroll
        for (int j = 0; j < 4; j++) dst[j] = *(const bf16x8*)(bp + j * 32 * kRS);
    };
    // the layer's bias in LDS (after the scratch), read when each unit's accumulators start
    constexpr bool CONVT = EPI == EPI_CONVT || EPI == EPI_CONVT_REFLECT;
    float* bias_s = (float*)(xs + 2 * slab_elems) + NC / 64 * 32 * kScrLd;
    if constexpr (!CONVT) {
        for (int i = threadIdx.x; i < p.m_pad; i += NC) bias_s[i] = i < p.m ? p.bias[i] : 0.f;
    }
    f32x16 acc[MI][4];

    int U = blockIdx.x, sl = 0;
    Unit cu{}, nu{};
    unit_at(U, cu);
    bool has_next = unit_at(U + gridDim.x, nu);
    // A of the current tap, one register set per 16-channel step; each set is refilled with the
    // next tap's fragments right after its MFMAs issue (a full tap of lead time for the L2 loads).
    bf16x8 A[4][MI], B0[4], B1[4];
#pragma unroll
    for (int kc = 0; kc < 4; kc++) load_a(A[kc], cu.m0, 0, kc);
    __syncthreads();  // slab 0 and the bias staged
    init_acc<!CONVT, MI>(acc, bias_s, cu.m0, wm, lane);
    read_b(B0, xs, 0, 0);  // slab 0's first step
    for (int g = 0; g < G; g++) {
        const uint16_t* buf = xs + (g & 1) * slab_elems;
        const uint16_t* nbuf = xs + ((g + 1) & 1) * slab_elems;  // the next slab's buffer
        const bool last = sl + 1 == nsl;
        // One tap: 4 steps of 16 channels.  Each step reads the next step's B fragments, four reads
        // on every path, so that the LDS wait counts of its MFMAs are static (with a skippable
        // read the compiler waits for all of them before the step's last MFMAs, i.e. for the reads
        // it has just issued).  The slab's last tap is a copy of its own (FINAL): at its last step
        // every read of the slab's buffer has been issued, and the barrier (after they complete:
        // nothing is left outstanding, on either path) hands the buffer back to the producers; the
        // next slab's first step is then read from the other buffer, which the producers filled
        // before the barrier, under this step's MFMAs -- or after the epilogue when one follows
        // (those registers live through it would spill).  Past the last slab that read is of a
        // stale buffer, in bounds and unused.
        auto tap = [&](int kk, auto final_tap) {
            constexpr bool FINAL = decltype(final_tap)::value;
            // the tap after this one: same slab, first tap of the next slab, or of the next unit
            // (the very last tap reloads tap 0 of this slab: a harmless load keeps the count static)
            int n_m0, n_kk, n_c16;
            walk_next_a(kk, p.k, sl, nsl, has_next, cu.m0, nu.m0, n_m0, n_kk, n_c16);
#pragma unroll
            for (int kc = 0; kc < 4; kc++) {
                bf16x8(&bc)[4] = (kc & 1) ? B1 : B0;
                bf16x8(&bn)[4] = (kc & 1) ? B0 : B1;
                if (FINAL && kc == 3) {
                    __syncthreads();
                    if (!last) read_b(bn, nbuf, 0, 0);
                }
                // The MFMAs fragment-major (fragment i's four, then i + 1's), each A fragment
                // reloaded right after its last MFMA, and the loads and LDS reads issued between
                // the MFMAs: a wave issues in order, so a load or read that waits for the memory
                // pipeline to accept it stalls the MFMAs behind it -- issued after all of the step's
                // MFMAs, those stalls left the matrix core idle.  (Every accumulator's sum is the
                // same sequence of MFMAs: the outputs do not change.)
                __builtin_amdgcn_sched_barrier(0);
                if (kc < 3)
                    read_b(bn, buf, kk, kc + 1);
                else if (!FINAL)
                    read_b(bn, buf, kk + 1, 0);
#pragma unroll
                for (int i = 0; i < MI; i++) {
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[kc][i], bc[j], acc[i][j], 0, 0, 0);
                    A[kc][i] = w_lane[(int64_t)n_m0 * 2 + ((int64_t)n_kk * n16 + n_c16 + kc) * a_step + 64 * i];
                }
                // issue order: (MFMA, LDS read) x 4, A reload, (MFMA x MI*4 - 4 ... ), A reload
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
                }
#pragma unroll
                for (int i = 0; i < MI; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // global load (A fragment i)
                    if (i + 1 < MI) __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        for (int kk = 0; kk + 1 < p.k; kk++) tap(kk, std::false_type{});
        tap(p.k - 1, std::true_type{});
        if (last) {
            const int next_m0 = has_next ? nu.m0 : cu.m0;
            // (not for the 256-channel f32 accumulate-with-statistics variant: a second epilogue copy
            // makes it spill)
            constexpr bool kFullPath = !(EPI == EPI_ACCUM && !OUT_H && WM == 4 && STATS);
            // ConvT: full when every phase's rows of the unit lie inside the item's output span,
            // at least two rows past its first (so no column writes the reflected row either)
            bool interior = true;
            if constexpr (CONVT) {
                const int64_t os = ld_const(p.out_start, cu.item);
                const int64_t oe = os + ld_const(p.out_len, cu.item) - (EPI == EPI_CONVT_REFLECT ? 1 : 0);
                const int64_t o_first = (int64_t)p.stride_t * cu.n0 - p.pad_t;
                interior = o_first >= os + 2 && o_first + (int64_t)p.stride_t * cu.nv <= oe;
            }
            if constexpr (MI == 1)
                epilogue_m32<WN>(p, cu, acc, wm, wn, lane, scr, bias_s, next_m0);
            else if (kFullPath && cu.nv >= wn * 128 + 128 && cu.m0 + BM <= p.m && interior)  // uniform: the common case
                epilogue<EPI, WM, WN, STATS, OUT_H, true>(p, cu, acc, wm, wn, lane, scr, bias_s, next_m0);
            else
                epilogue<EPI, WM, WN, STATS, OUT_H, false>(p, cu, acc, wm, wn, lane, scr, bias_s, next_m0);
            read_b(B0, nbuf, 0, 0);
        }
        if (last) {
            sl = 0;
            U += gridDim.x;
            cu = nu;
            has_next = unit_at(U + gridDim.x, nu);
        } else {
            sl++;
        }
    }
}

template <int PRO, int EPI, int WM, int WN, bool STATS, bool IN_H, bool OUT_H, int MI = 2>
hipError_t launch_t(const ConvParams& p, int n_cu, hipStream_t s, bool validate_only) {
    constexpr int BM = 32 * MI * WM, BN = 16 * kNJ * WN, NT = 64 * WM * WN + kNP;
    const int halo = (p.k - 1) * p.dil;
    constexpr size_t scr_bytes = (size_t)WM * WN * 32 * kScrLd * sizeof(float) + kMaxBias * sizeof(float);
    const size_t smem = 2 * (size_t)(BN + halo) * kRS * sizeof(uint16_t) + scr_bytes;
    constexpr size_t smem_max = 2 * (size_t)(BN + kMaxHalo) * kRS * sizeof(uint16_t) + scr_bytes;
    static_assert(smem_max <= 160 * 1024, "LDS budget");
    constexpr bool CONVT = EPI == EPI_CONVT || EPI == EPI_CONVT_REFLECT;
    if (p.m_pad % BM != 0 || p.cin_pad % kCK != 0 || halo < 0 || halo > kMaxHalo || !p.bias) return hipErrorInvalidValue;
    if (!CONVT && p.m_pad > kMaxBias) return hipErrorInvalidValue;  // the bias staged in LDS
    if (PRO == PRO_ADAIN_SNAKE && p.cin % kCK != 0) return hipErrorInvalidValue;  // no channel mask there
    if (EPI == EPI_MEAN3_LEAKY_BF16 && !(p.slope > 0.f && p.slope <= 1.f)) return hipErrorInvalidValue;  // max form
    if (p.l_in >= (int64_t)1 << 30 || p.tiles.count >= (int64_t)1 << 28) return hipErrorInvalidValue;  // 32-bit rows
    // epilogue stores: byte offsets within one unit's rows inside the buffer resource's range
    if (!CONVT && ((int64_t)BN * max(p.y_ld, p.r0_ld) + p.m_pad) * 4 >= kBufRecords) return hipErrorInvalidValue;
    if (CONVT && ((int64_t)p.stride_t * (BN + 1) + p.pad_t + 2) * max(p.y_ld, p.r0_ld) * 4 >= kBufRecords)
        return hipErrorInvalidValue;
    // producer loads: 32-bit byte offsets within one item's rows, rows and channels within the
    // 24-bit multiplier
    if (p.in_max_len * p.x_ld * (PRO != PRO_BF16 && !IN_H ? 4 : 2) >= (int64_t)1 << 32) return hipErrorInvalidValue;
    if (p.in_max_len >= (int64_t)1 << 24 || p.x_ld >= (int64_t)1 << 24 || p.y_ld >= (int64_t)1 << 24 ||
        p.r0_ld >= (int64_t)1 << 24)
        return hipErrorInvalidValue;
    if (validate_only) return hipSuccess;
    // one persistent block per CU; the grid is a multiple of 8 * mblocks
    const int64_t grid = walk_grid(p.tiles.count, p.m_pad / BM, n_cu);
    // the dynamic LDS limit is a per-device attribute of each kernel: set once per device
    auto go = [&](auto kern, DeviceFlags& attr) -> hipError_t {
        int dev = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e != hipSuccess) return e;
        if (!attr.test(dev)) {
            e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem_max);
            if (e != hipSuccess) return e;
            attr.set(dev);
        }
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(NT), smem, s, p);
        return hipGetLastError();
    };
    // small halos (every k3 layer, k7 at dilation 1, the ConvTs, 1x1 convs): the producers stage
    // BN + 16 rows instead of BN + 64 (3 of 20 row passes fewer at BN 256, 3 of 12 at BN 128)
    static DeviceFlags attr_small, attr_max;
    if (halo <= kSmallHalo)
        return go(conv_mfma_kernel<PRO, EPI, WM, WN, STATS, IN_H, OUT_H, kSmallHalo, MI>, attr_small);
    return go(conv_mfma_kernel<PRO, EPI, WM, WN, STATS, IN_H, OUT_H, kMaxHalo, MI>, attr_max);
}

}  // namespace

// The (prologue, epilogue, block shape, statistics, fp16 in/out) combinations the engine uses;
// anything else is refused.
hipError_t launch_conv(const ConvParams& p, int pro, int epi, int shape, bool stats, bool in_h, bool out_h, int n_cu,
                       hipStream_t s, bool validate_only) {
    if (p.tiles.count == 0) return hipSuccess;
#define KK_CONV(P, E, SH, WM, WN, ST, IH, OH)                                              \
    if (pro == P && epi == E && shape == SH && stats == ST && in_h == IH && out_h == OH) \
        return launch_t<P, E, WM, WN, ST, IH, OH>(p, n_cu, s, validate_only);
    // Snake blocks in place on an f32 stream (the noise branches, the one-block plans), 256 ch
    // (stage 0) and 128 ch (stage 1): conv1 X (f32) -> h (fp16) with statistics; conv2 h -> X
    // (ACCUM with statistics, last step without)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, SHAPE_256x128, 4, 1, true, false, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_256x128, 4, 1, true, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_256x128, 4, 1, false, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, SHAPE_128x256, 2, 2, true, false, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_128x256, 2, 2, true, true, false)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_128x256, 2, 2, false, true, false)
    // the generator's fp16 residual streams: conv1 X (fp16) -> h; conv2 h -> X as ADD_FROM (the
    // resblocks' first step, from the stage input) and ACCUM, with statistics but for the last
    // step; each stage's mean of its resblocks' three streams stored as the next layer's bf16
    // operand (ups.1, conv_post)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, SHAPE_256x128, 4, 1, true, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ADD_FROM, SHAPE_256x128, 4, 1, true, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_256x128, 4, 1, true, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_256x128, 4, 1, false, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_MEAN3_LEAKY_BF16, SHAPE_256x128, 4, 1, false, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_STORE, SHAPE_128x256, 2, 2, true, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ADD_FROM, SHAPE_128x256, 2, 2, true, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_128x256, 2, 2, true, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_ACCUM, SHAPE_128x256, 2, 2, false, true, true)
    KK_CONV(PRO_ADAIN_SNAKE, EPI_MEAN3_LEAKY_BF16, SHAPE_128x256, 2, 2, false, true, true)
    // decoder
    KK_CONV(PRO_ADAIN_LEAKY, EPI_STORE, SHAPE_256x128, 4, 1, true, false, false)
    KK_CONV(PRO_ADAIN_LEAKY, EPI_RESID, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_ADAIN_LEAKY, EPI_RESID_UP2, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_F32, EPI_STORE, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_F32, EPI_STORE, SHAPE_64x256, 1, 2, false, false, false)
    KK_CONV(PRO_BF16, EPI_STORE, SHAPE_256x128, 4, 1, true, false, false)
    // stages before the decoder: residual linears (ALBERT attention output; FFN output from the
    // FFN's bf16 gelu_new output) and the FFN itself
    KK_CONV(PRO_F32, EPI_RESID, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_BF16, EPI_RESID, SHAPE_256x128, 4, 1, false, false, false)
    KK_CONV(PRO_F32, EPI_GELU_BF16, SHAPE_256x128, 4, 1, false, false, true)
    // ConvT ups (the stage input in fp16, plus the noise branch's fp16 stream) and conv_post
    KK_CONV(PRO_LEAKY, EPI_CONVT, SHAPE_256x128, 4, 1, true, false, true)
    KK_CONV(PRO_BF16, EPI_CONVT_REFLECT, SHAPE_256x128, 4, 1, true, false, true)
    KK_CONV(PRO_LEAKY, EPI_STORE, SHAPE_64x256, 1, 2, false, false, false)
    // conv_post (22 output rows) on 32-row waves, from its bf16 operand (or f32 through leaky ReLU)
    if (pro == PRO_BF16 && epi == EPI_STORE && shape == SHAPE_32x256 && !stats && !in_h && !out_h)
        return launch_t<PRO_BF16, EPI_STORE, 1, 2, false, false, false, 1>(p, n_cu, s, validate_only);
    if (pro == PRO_LEAKY && epi == EPI_STORE && shape == SHAPE_32x256 && !stats && !in_h && !out_h)
        return launch_t<PRO_LEAKY, EPI_STORE, 1, 2, false, false, false, 1>(p, n_cu, s, validate_only);
#undef KK_CONV
    return hipErrorInvalidValue;
}

}  // namespace kk
