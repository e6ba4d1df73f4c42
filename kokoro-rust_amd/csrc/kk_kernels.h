// kk_kernels.h -- launch interface of the gfx950 kernels (host side of kk_conv.hip / kk_misc.hip).
#pragma once
#include "kk_common.h"

namespace kk {

// ---------------------------------------------------------------- MFMA convolution
enum Prologue {
    PRO_BF16 = 0,         // input already bf16 [L][ld], gap rows -> 0
    PRO_F32 = 1,          // f32 input -> bf16, gap rows -> 0
    PRO_LEAKY = 2,        // leaky ReLU(slope), gap rows -> 0
    PRO_ADAIN_LEAKY = 3,  // AdaIN (per item, per channel affine) + leaky ReLU(slope)
    PRO_ADAIN_SNAKE = 4,  // AdaIN + Snake x + sin^2(a x)/a
};
enum Epilogue {
    EPI_STORE = 0,          // y = conv + b
    EPI_ACCUM = 1,          // y += conv + b
    EPI_RESID = 2,          // y = (conv + b + y) * scale
    EPI_RESID_UP2 = 3,      // y = (conv + b + r0[t/2]) * scale
    EPI_ADD_FROM = 4,       // y = r0 + (conv + b)
    EPI_MEAN3 = 5,          // y = ((r0 + r1) + (r2 + conv + b)) / 3
    EPI_CONVT = 6,          // polyphase ConvT scatter, y[o] = conv + b + r0[o]
    EPI_CONVT_REFLECT = 7,  // ConvT scatter with per-item ReflectionPad1d((1,0)), + r0
};
enum BlockShape {
    SHAPE_W4x2 = 0,  // 256 (M) x 128 (N), 8 waves
    SHAPE_W2x4 = 1,  // 128 x 256, 8 waves
    SHAPE_W1x4 = 2,  // 64 x 256, 4 waves
};

struct ConvParams {
    const void* x;           // input [l_in][x_ld] (f32 or bf16)
    int64_t x_ld;
    int64_t l_in;
    int cin, cin_pad;        // real and padded (multiple of 64) input channels
    const int32_t* col_in;   // input domain col_item (null: no gap masking)
    const Coef* coef;        // [nb][cin]
    const float* alpha_rev;  // [cin] alpha / 2 pi
    const float* alpha_inv;  // [cin] 1 / alpha
    float slope;
    const uint16_t* w;       // packed bf16 [k][cin_pad/32][m_pad][32]
    const float* bias;       // [cout] or null
    int m, m_pad;            // GEMM rows (cout, or stride * cout for ConvT), padded to the block
    int k, dil, pad;
    float* y;                // output [rows][y_ld]
    int64_t y_ld;
    int cout;
    int64_t n_out;           // GEMM columns
    const float* r0;         // epilogue operands
    const float* r1;
    const float* r2;
    int64_t r0_ld;
    float scale;
    int stride_t, pad_t;     // ConvT stride / padding
    int64_t l_convt;         // ConvT output length (before the reflect pad)
    const int32_t* col_out;  // padded output domain (reflect epilogue)
    const int64_t* start_out;
};

int conv_block_m(int shape);
int conv_block_n(int shape);
hipError_t launch_conv(const ConvParams& p, int pro, int epi, int shape, hipStream_t s);

// ---------------------------------------------------------------- bandwidth kernels (kk_misc.hip)
// AdaIN statistics: per-(item, channel) shifted sums accumulated in f64 (sums [nb][C][2]).
hipError_t launch_stats(const float* x, int64_t ld, int c, DomDev d, double* sums, hipStream_t s);
// sums -> AdaIN coefficients (and sums reset to zero for the next use).
hipError_t launch_finalize(const float* x, int64_t ld, int c, DomDev d, double* sums, const float* gb,
                           int64_t gb_ld, int gb_off, const float* nw, const float* nb, Coef* coef, int reset,
                           hipStream_t s);
// gb[b][j] = W[j] . style[b] + bias[j] for every AdaIN layer at once.
hipError_t launch_style_fc(const float* w, const float* bias, int rows, const float* style, int nb, float* gb,
                           hipStream_t s);
// asr[t][c] = t_en[c][src_row[t]] (0 in gaps), time-major [l][ld] with channels [0, 512).
hipError_t launch_expand(const float* t_en, int64_t t_rows, const int32_t* src_row, int64_t l, float* asr,
                         int64_t ld, hipStream_t s);
// F0_conv / N_conv: 1 -> 1 channel, k3 s2 p1 on d2 -> dn; out at column `col` of [ln][ld].
hipError_t launch_f0n_conv(const float* f0, const float* en, int64_t l2, const float* w_f0, const float* b_f0,
                           const float* w_n, const float* b_n, float* out, int64_t ld, int col_f0, int col_n,
                           const int32_t* col, int64_t ln, hipStream_t s);
// Copy channels [0, c) of src [l][src_ld] into dst [l][dst_ld] at channel offset dst_c0; gap rows -> 0.
hipError_t launch_copy_cols(const float* src, int64_t src_ld, int c, float* dst, int64_t dst_ld, int dst_c0,
                            const int32_t* col, int64_t l, hipStream_t s);
// AdaIN + leaky(0.2) then depthwise ConvT k3 s2 p1 op1 (decoder upsample pool) -> bf16 [2l][out_ld].
hipError_t launch_adain_pool(const float* x, int64_t ld, int c, const Coef* coef, const int32_t* col_n,
                             int64_t ln, const float* pw, const float* pb, const int32_t* col_2, uint16_t* out,
                             int64_t out_ld, hipStream_t s);
// Strided f32 conv 22 -> cout (noise_convs.0: k12 s6 p3; noise_convs.1: k1) on the masked spectrum.
hipError_t launch_noise_conv(const float* spec, int64_t spec_ld, int64_t l_in, const int32_t* col_in,
                             const float* w, const float* b, int cout, int k, int stride, int pad, float* y,
                             int64_t y_ld, int64_t l_out, hipStream_t s);
// SineGen phase_pre: per item and harmonic, f64 cumulative sum of the 1/300-downsampled rad values.
hipError_t launch_phase_pre(const float* f0, const int64_t* start2, const int64_t* len2, int nb,
                            const float* rand_ini, float* pp, int64_t pp_ld, hipStream_t s);
// Harmonic source + STFT, one launch over all items: spec [F rows][spec_ld] (22 used).
struct SourceParams {
    const float* f0;          // d2 packed F0 curve
    const int64_t* start2;    // per item d2 start (= 2 a_b)
    const int64_t* len2;      // 2 N_b
    const float* pp;          // [9][pp_ld] phase_pre in d2 packing
    int64_t pp_ld;
    const uint64_t* seeds;    // per item counter seed
    const float* fixed_noise; // packed [600 ln * 9] or null
    const int32_t* noise_kind;// per item: 0 counter, 1 fixed
    const float* lw;          // [9]
    float lb;
    const int64_t* start120;  // d120 start per item (= 120 a_b)
    const int64_t* f_len;     // frames per item (120 N_b + 1)
    const int64_t* blk_item;  // work list: item of each block
    const int64_t* blk_f0;    // first frame of each block
    int64_t n_blocks;
    float* spec;
    int64_t spec_ld;
};
hipError_t launch_source_stft(const SourceParams& p, hipStream_t s);
// iSTFT frames + overlap-add, one launch over all items: audio packed at 600 a_b.
struct IstftParams {
    const float* post;        // [120 ln + 1][post_ld]
    int64_t post_ld;
    const int64_t* start120;
    const int64_t* f_len;
    const int64_t* blk_item;
    const int64_t* blk_s0;    // first output sample (item-local) of each block
    int64_t n_blocks;
    float* audio;             // packed; item b at 600 a_b
    const int64_t* audio_start;
};
hipError_t launch_istft(const IstftParams& p, hipStream_t s);
// Zero a float buffer (a kernel, so the sequence stays capturable in a graph).
hipError_t launch_zero(void* p, int64_t bytes, hipStream_t s);

constexpr int kSourceFrames = 128;  // STFT frames per source block
constexpr int kIstftSamples = 512;  // output samples per iSTFT block
hipError_t upload_stft_tables(const double* cosv, const double* sinv, const float* win);

}  // namespace kk
