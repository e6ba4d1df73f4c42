// kk_kernels.h -- launch interface of the gfx950 kernels (host side of kk_conv.hip / kk_misc.hip).
#pragma once
#include "kk_common.h"

#include <vector>

namespace kk {

// ---------------------------------------------------------------- tiles
// Convolutions and statistics run over item-aligned tiles: tile i covers GEMM columns
// [t0[i], t0[i] + n[i]) of item item[i] (n[i] <= the kernel's tile width), so no tile mixes items
// and gap columns are never computed.  Tiles of one item are consecutive; item b owns tiles
// [lo[b], hi[b]).
struct TilesDev {
    const int32_t* item;
    const int64_t* t0;
    const int32_t* n;
    const int32_t* lo;
    const int32_t* hi;
    int64_t count;
};

// Per-(partial, channel) statistics record: sums of (v - shift) and (v - shift)^2 over n columns,
// shift = the first of those columns' value (exact local centring; Chan's combination in finalize).
struct __align__(16) StatPart {
    float s1, s2, shift, n;
};

// ---------------------------------------------------------------- MFMA convolution
enum Prologue {
    PRO_BF16 = 0,         // input already bf16 [L][ld]
    PRO_F32 = 1,          // f32 input -> bf16
    PRO_LEAKY = 2,        // leaky ReLU(slope)
    PRO_ADAIN_LEAKY = 3,  // AdaIN (per item, per channel affine) + leaky ReLU(slope)
    PRO_ADAIN_SNAKE = 4,  // AdaIN + Snake x + sin^2(a x)/a
};
enum Epilogue {
    EPI_STORE = 0,          // y = conv + b
    EPI_ACCUM = 1,          // y += conv + b (y fp16, read and written, when the output is fp16)
    EPI_RESID = 2,          // y = (conv + b + y) * scale
    EPI_RESID_UP2 = 3,      // y = (conv + b + r0[t/2]) * scale
    EPI_ADD_FROM = 4,       // y = r0 + (conv + b) (r0 and y f32, or both fp16 with an fp16 output)
    EPI_CONVT = 6,          // polyphase ConvT scatter, y[o] = conv + b + r0[o]
    EPI_CONVT_REFLECT = 7,  // ConvT scatter with per-item ReflectionPad1d((1,0)), + r0
    EPI_GELU_BF16 = 8,      // y (bf16) = gelu_new(conv + b) (kernels/kokoro.cu:84-90), 2-byte output
    EPI_MEAN3_LEAKY_BF16 = 9,  // y (bf16) = leaky(((r0 + r1) + (r2 + conv + b)) / 3, slope): a
                               // generator stage's mean of its three resblocks, stored as the next
                               // layer's input operand (r0, r1, r2 the blocks' fp16 residual streams
                               // with r0_ld; 2-byte output; the slope in ConvParams.slope, which the
                               // Snake prologue does not use)
};
enum BlockShape {
    SHAPE_256x128 = 0,  // 4 waves (4 x 1), wave tile 64 x 128
    SHAPE_128x256 = 1,  // 4 waves (2 x 2)
    SHAPE_64x256 = 2,   // 2 waves (1 x 2)
    SHAPE_32x256 = 3,   // 2 waves (1 x 2), wave tile 32 x 128 (layers of at most 32 output rows)
};
constexpr int kShapeM[4] = {256, 128, 64, 32};
constexpr int kShapeN[4] = {128, 256, 256, 256};
constexpr int kShapeWN[4] = {1, 2, 2, 2};

struct ConvParams {
    const void* x;           // input [l_in][x_ld] (f32, fp16 or bf16)
    int64_t x_ld;
    int64_t l_in;
    int64_t in_max_len;      // longest item span of the input domain (rows)
    int cin, cin_pad;        // real and padded (multiple of 64) input channels
    const int64_t* in_start; // input domain item spans (rows outside an item's span read as 0)
    const int64_t* in_len;
    TilesDev tiles;          // GEMM-column tiles (output domain for convs, input domain for ConvT)
    const Coef* coef;        // [nb][cin]
    const float* alpha_rev;  // [cin] alpha / 2 pi
    const float* alpha_inv;  // [cin] 1 / alpha
    float slope;
    const uint16_t* w;       // packed bf16 [k][cin_pad/16][m_pad][16]
    const float* bias;       // [cout] (zeros for a layer without bias)
    int m, m_pad;            // GEMM rows (cout, or stride * cout for ConvT), padded to the block
    int k, dil, pad;
    float* y;                // output [rows][y_ld] (f32, or fp16 for the Snake steps' h)
    int64_t y_ld;
    int cout;
    const float* r0;         // epilogue operands
    const float* r1;
    const float* r2;
    int64_t r0_ld;
    float scale;
    int stride_t, pad_t;     // ConvT stride / padding
    const int64_t* out_start;// ConvT: output domain item spans
    const int64_t* out_len;
    StatPart* part;          // epilogue statistics [tiles * WN][cout] (null: none)
};

// in_h / out_h: fp16 input (conv2 of a Snake step) / fp16 output (conv1 of a Snake step).
// n_cu: compute units of the device (persistent grid size).  validate_only: check the parameters
// against the kernel's limits (hipErrorInvalidValue when out of range) and launch nothing.
hipError_t launch_conv(const ConvParams& p, int pro, int epi, int shape, bool stats, bool in_h, bool out_h, int n_cu,
                       hipStream_t s, bool validate_only = false);

// ---------------------------------------------------------------- bandwidth kernels (kk_misc.hip)
// Statistics partials of x [l][ld] over tiles (one partial per tile and channel).
hipError_t launch_stats_tiles(const float* x, int64_t ld, int c, TilesDev t, StatPart* part, hipStream_t s);
// Partials -> per-(item, channel) mean / rstd (chan_stats_seg semantics) -> AdaIN coefficients.
// `wn` partials per tile (records [tile * wn + w][c]); max_parts: the most partials of any item
// (tiles x wn), which sizes the reduction.
// xrow (optional): one more sample per item outside the partials, row xrow_at[b] of xrow [.][xrow_ld]
// (the reflected first row of the stage-1 ConvT output).
// outs: the 1..kFinMaxOuts AdaIN layers that normalise this tensor, each with its style offset into
// gb, norm weight / bias and coefficient array [nb][c].
constexpr int kFinMaxOuts = 3;
struct FinOut {
    int gb_off;
    const float* nw;
    const float* nb;
    Coef* coef;
};
struct FinOuts {
    FinOut o[kFinMaxOuts];
    int n;
};
// xrow (fp16 [.][xrow_ld]): one more sample per item outside the partials, row xrow_at[b].
hipError_t launch_finalize(const StatPart* part, int c, int wn, TilesDev t, int nb, int64_t max_parts,
                           const float* gb, int64_t gb_ld, const FinOuts& outs, hipStream_t s,
                           const uint16_t* xrow = nullptr, int64_t xrow_ld = 0, const int64_t* xrow_at = nullptr);
// gb[b][j] = W[j] . style[b] + bias[j] for every AdaIN layer at once.
hipError_t launch_style_fc(const float* w, const float* bias, int rows, const float* style, int nb, float* gb,
                           hipStream_t s);
// asr[t][c] = t_en[src_row[t]][c] (0 in gaps): t_en token rows [t_rows][512] -> frame rows [l][ld],
// channels [0, 512).
hipError_t launch_expand(const float* t_en, int64_t t_rows, const int32_t* src_row, int64_t l, float* asr,
                         int64_t ld, hipStream_t s);
// F0_conv / N_conv: 1 -> 1 channel, k3 s2 p1 on d2 -> dn; out at columns col_f0 / col_n of [ln][ld].
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
// Strided conv 22 -> cout on the spectrum at f32 accuracy (split-bf16 matrix-core products) --
// noise_convs.0: k12 s6 p3 over item-aligned tiles of kNoiseTile output rows; noise_convs.1: k1
// over tiles of kNoiseTile1 rows (tile_rows: the width the tiles t were built with, checked) --
// rows outside the tile's item span [in_start, in_start + in_len) read as 0 (the reference's gap
// mask), rows outside the tiles not written, with the statistics partial of each tile
// ([tile][cout], shift = bias) for the next layer's AdaIN.  wp: the weights split into bf16
// roundings and remainders, packed as A fragments ([32-row tile][K step][rounding,
// remainder][64 lanes][8] bf16; noise_convs.0: 18 K steps, k = 24 tap + channel; noise_convs.1:
// 2 K steps, k = channel; channels 22 and up zero).  y is stored as fp16
// (the noise branch's residual stream; the statistics describe the f32 values).
constexpr int kNoiseTile = 64, kNoiseTile1 = 128;
hipError_t launch_noise_conv(const float* spec, int64_t spec_ld, int64_t l_in, const int64_t* in_start,
                             const int64_t* in_len, const uint16_t* wp, const float* b, int cout, int k, int stride,
                             int pad, uint16_t* y, int64_t y_ld, TilesDev t, int tile_rows, StatPart* part,
                             hipStream_t s);
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
    float* har_tap;           // or null: the source samples at 600 a_b (a test tap)
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
// PCM_16 encoding of packed audio (src/wav.rs:63-80) over the iSTFT's work list (blocks of
// kIstftSamples samples of one item; blk_item null: one item of n samples from 0): out[i] =
// clamp(round-half-even(audio[i] * 32767)), NaN -> 0; clipped[b] += samples outside
// [-32768, 32767] after rounding (NaN and infinities included).  clipped must start at zero.
hipError_t launch_pcm16(const float* audio, const int64_t* audio_start, const int64_t* item_len,
                        const int64_t* blk_item, const int64_t* blk_s0, int64_t n_blocks, int16_t* out,
                        unsigned long long* clipped, hipStream_t s);
// Zero a buffer / fill it with a 32-bit pattern (kernels, so the sequence stays capturable in a
// graph); bytes is a multiple of 4.
hipError_t launch_zero(void* p, int64_t bytes, hipStream_t s);
hipError_t launch_fill(void* p, int64_t bytes, uint32_t value, hipStream_t s);

// ---------------------------------------------------------------- stages before the decoder (kk_upstream.hip)
// Row tables: row_item [rows] (owning item, -1 in gaps), ids [rows] (token id), start [nb] (first
// row of each item).  Gap rows are neither read nor written.
// ALBERT embeddings + LayerNorm 1e-12 -> out [rows][128].
hipError_t launch_albert_embed(const int32_t* ids, const int32_t* row_item, const int64_t* start, int64_t rows,
                               const float* word, const float* pos, const float* tok0, const float* g, const float* b,
                               float* out, hipStream_t s);
// text encoder embedding -> out [rows][512].
hipError_t launch_text_embed(const int32_t* ids, const int32_t* row_item, int64_t rows, const float* emb, float* out,
                             hipStream_t s);
// LayerNorm of channels [0, d) (d = 512 or 768) of x [rows][ld] in place: affine g, b, or
// AdaLayerNorm with gb (gamma at gb[item][gb_off + c], beta at gb[item][gb_off + d + c]) when gb is
// not null; then leaky ReLU(slope) when leaky.
hipError_t launch_layernorm(float* x, int64_t ld, int d, int64_t rows, const int32_t* row_item, const float* g,
                            const float* b, const float* gb, int64_t gb_ld, int gb_off, float eps, bool leaky,
                            float slope, hipStream_t s);
// ALBERT attention, 12 heads of 64, scale 1/8: qkv [rows][2304] -> out [rows][768]; work list of
// (item, head, first query) blocks of 64 queries.  On the f32 matrix cores, or (valu) on the VALU.
hipError_t launch_attention(const float* qkv, const int64_t* start, const int64_t* len, const int32_t* w_item,
                            const int32_t* w_head, const int32_t* w_q0, int64_t n_blocks, float* out, hipStream_t s,
                            bool valu = false);
// BiLSTM recurrence, H = 256, over the item spans [start, start + len): gx [*][gx_ld] gate
// pre-activations (W_ih x + b_ih, forward at columns [0, 1024), reverse at [1024, 2048)) at row
// gx_row[r] (or r when gx_row is null); whh_t [2][256][1024] (k-major), bhh [2][1024];
// h -> out[r][dir 256 + j].
hipError_t launch_lstm(const float* gx, int64_t gx_ld, const int32_t* gx_row, const int64_t* start, const int64_t* len,
                       int nb, const float* whh_t, const float* bhh, float* out, int64_t out_ld, hipStream_t s);
// The same recurrence with each (item, direction) split over two CUs that trade their halves of h
// every step (the whole of W_hh on chip).  xbuf: 2 nb x 512 exchange words (cleared by the launch);
// *abort is set, and every block ends, if a block waits more than wait_ticks (100 MHz clock) for
// its partner.  silent_half >= 0 (a test hook) keeps that half of every pair from publishing.
constexpr uint64_t kLstmPairWaitTicks = 200000000ull;  // 2 s
hipError_t launch_lstm_pair(const float* gx, int64_t gx_ld, const int32_t* gx_row, const int64_t* start,
                            const int64_t* len, int nb, const float* whh_t, const float* bhh, float* out, int64_t out_ld,
                            uint64_t* xbuf, int* abort, hipStream_t s, uint64_t wait_ticks = kLstmPairWaitTicks,
                            int silent_half = -1);
// Four CUs per (item, direction), each with a quarter of h and all of its W_hh rows in registers;
// the same arguments (xbuf 2 nb x 512 words), bit-identical outputs.  lstm_quads(nb) quads (one
// block per CU) run the 2 nb sequences as lists, sched = lstm_schedule(len, nb): [nq + 1] offsets,
// then the sequence ids (2 item + direction) of each quad's list.  silent_quarter >= 0 (a test
// hook) keeps that quarter of every quad from publishing.
constexpr int kLstmQuads = 64;               // 256 CUs
constexpr int64_t kLstmQuadMinSteps = 1024;  // the engine's choice: quads when a span has this many steps
inline int lstm_quads(int nb) { return 2 * nb < kLstmQuads ? 2 * nb : kLstmQuads; }
// Longest processing time first: the sequences by decreasing length (items by length, ties by
// index, both directions in turn), each to the quad with the least total length so far (ties: the
// lowest quad).
std::vector<int32_t> lstm_schedule(const int64_t* len, int nb);
hipError_t launch_lstm_quad(const float* gx, int64_t gx_ld, const int32_t* gx_row, const int64_t* start,
                            const int64_t* len, int nb, const int32_t* sched, const float* whh_t, const float* bhh,
                            float* out, int64_t out_ld, uint64_t* xbuf, int* abort, hipStream_t s,
                            uint64_t wait_ticks = kLstmPairWaitTicks, int silent_quarter = -1);
// Zeroes n 64-bit words.
hipError_t launch_clear_u64(uint64_t* x, int64_t n, hipStream_t s);
// F0_proj / N_proj: y[r] = b + w . x[r][0:c] (c = 256) on the rows with col[r] >= 0, 0 elsewhere.
hipError_t launch_proj1(const float* x, int64_t ld, int c, const float* w, const float* b, const int32_t* col,
                        int64_t rows, float* y, hipStream_t s);
// x[r][col0 .. col0 + 128) = styles[row_item[r]] for the item rows.
hipError_t launch_style_cols(float* x, int64_t ld, int col0, int64_t rows, const int32_t* row_item,
                             const float* styles, hipStream_t s);

constexpr int kSourceFrames = 128;  // STFT frames per source block
constexpr int kIstftSamples = 512;  // output samples per iSTFT block
constexpr int kStatTile = 256;      // rows per tile of the standalone statistics pass
hipError_t upload_stft_tables(const double* cosv, const double* sinv, const float* win);

}  // namespace kk
