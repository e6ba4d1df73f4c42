/*
 * kokoro_hip.h -- C ABI of the MI355X (gfx950) batched ragged Kokoro-82M decoder + iSTFTNet
 * generator path.
 *
 * This library stands in for the reference's `crate::gpu` module (src/gpu.rs + src/gpu_batch.rs)
 * on the path from the predicted durations to the audio.  Plain pointers and sizes only; every
 * entry returns KK_OK (0) or a negative KK_ERR_* status and, where a buffer is given, a message.
 * No entry aborts the process: device allocation failure is KK_ERR_OOM so a caller can split its
 * batch and retry as Engine::synth_batch does (src/engine.rs:229-234).
 *
 * Threading: a context may be created on one thread and used from another (the reference creates
 * its Gpu on a helper thread, src/engine.rs:92-96); every entry selects the context's device
 * itself.  Calls on one context must not overlap (the reference engine is not shared,
 * src/cli.rs:625-626).
 */
#ifndef KOKORO_HIP_H
#define KOKORO_HIP_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

#define KK_OK 0
#define KK_ERR_INVALID (-1) /* bad argument or shape (src/gpu_batch.rs:181-187, src/gpu.rs:494-498) */
#define KK_ERR_HIP (-2)     /* HIP runtime error */
#define KK_ERR_OOM (-3)     /* device allocation failed */
#define KK_ERR_STATE (-4)   /* model not uploaded / plan not run */

typedef struct kk_ctx kk_ctx;
typedef struct kk_plan kk_plan;

/* ------------------------------------------------------------------ context (Gpu) */

/* Gpu::new(ordinal) (src/gpu.rs:81-105): open device `ordinal`, create the stream, upload the
 * STFT twiddles and window.  Refuses devices that are not gfx950. */
int kk_open(int ordinal, kk_ctx** out, char* err, size_t errlen);
void kk_close(kk_ctx* ctx);
/* Gpu::device_name (src/gpu.rs:107-109). */
int kk_device_name(const kk_ctx* ctx, char* buf, size_t len);
/* Numerical identity of the engine, part of output provenance / resume keys
 * (KERNEL_ROUNDING src/gpu.rs:29, Engine::identity src/engine.rs:109-111). */
const char* kk_identity(void);

/* ------------------------------------------------------------------ model (GpuKokoro::with_gpu) */

/* One host tensor of the decoder + generator, by checkpoint state-dict name with weight_norm
 * already resolved (the values the reference's host structs hold, src/vocoder.rs:54-111,
 * src/nn.rs:25-166; e.g. "decoder.generator.resblocks.0.convs1.0.weight", f32, row-major). */
typedef struct {
    const char* name;
    const float* data;
    int64_t numel;
} kk_tensor;

/* GpuKokoro::with_gpu (src/gpu.rs:685-724), decoder + generator part: validates every shape,
 * packs the conv weights into the MFMA operand layout (bf16), copies everything to the device.
 * The tensors are copied; the caller keeps ownership. */
int kk_upload_model(kk_ctx* ctx, const kk_tensor* tensors, int n, char* err, size_t errlen);

/* ------------------------------------------------------------------ checkpoints and voices (host)
 * The released model file and voice packs are PyTorch zip archives (torch.save).  They are read
 * on the host, never executed: STORED zip entries, and a pickle interpreter that accepts only
 * float32 tensors in (ordered) dicts (globals collections.OrderedDict,
 * torch._utils._rebuild_tensor_v2, torch.FloatStorage); anything else is KK_ERR_INVALID. */
typedef struct kk_checkpoint kk_checkpoint;
/* load_kmodel_checkpoint (src/torchpt.rs:311-327): {submodule: state_dict} flattened to
 * "submodule.param" (a leading "module." of a parameter stripped), tensors as contiguous f32. */
int kk_checkpoint_open(const char* path, kk_checkpoint** out, char* err, size_t errlen);
int kk_checkpoint_count(const kk_checkpoint* ck);
/* Entry i (names sorted): its name, shape [ndim] and data [numel], valid until kk_checkpoint_free. */
int kk_checkpoint_entry(const kk_checkpoint* ck, int i, const char** name, const int64_t** shape, int* ndim,
                        const float** data, int64_t* numel);
void kk_checkpoint_free(kk_checkpoint* ck);
/* Weights::load_pth + GpuKokoro::with_gpu for the decoder + generator (src/weights.rs:19-26,
 * src/gpu.rs:685-724): the "decoder.*" tensors of the checkpoint, each conv weight resolved from
 * weight_g / weight_v when "X.weight" is absent (Weights::conv_weight, src/weights.rs:62-73), the
 * AdaIN InstanceNorm affine parameters defaulting to 1 / 0 when absent
 * (Weights::get_instance_norm_affine, src/weights.rs:76-84), then as kk_upload_model. */
int kk_upload_checkpoint(kk_ctx* ctx, const kk_checkpoint* ck, char* err, size_t errlen);
/* weight_norm (src/ops.rs:9-23): w = v * (g[r] / ||v_r||) per row r of `per_row` values, the norm
 * summed in f64. */
int kk_weight_norm(const float* v, const float* g, int64_t rows, int64_t per_row, float* w);
/* load_voice_pack (src/torchpt.rs:329-335) and Engine::voice (src/engine.rs:114-137): the packs at
 * paths[0..n) ([rows, 1, 256] each), element-wise mean when n > 1 (summed in order in f32), as a
 * malloc'ed [rows][256] array released by kk_voice_free. */
int kk_voice_load(const char* const* paths, int n, float** pack, int64_t* rows, char* err, size_t errlen);
void kk_voice_free(float* pack);
/* Voice::ref_s (src/engine.rs:54-59): the style of an utterance of n phoneme characters is row
 * n - 1 (256 values); n outside [1, rows] is KK_ERR_INVALID. */
int kk_voice_ref_s(const float* pack, int64_t rows, int64_t n_phoneme_chars, const float** ref_s);

/* ------------------------------------------------------------------ batch items */

#define KK_NOISE_COUNTER 0 /* ItemNoise::Counter(seed) (src/gpu_batch.rs:15) */
#define KK_NOISE_FIXED 1   /* ItemNoise::Fixed { rand_ini, sine } (src/gpu_batch.rs:16) */

/* One item at the point where forward_batch enters the decoder (src/gpu_batch.rs:244-297): its
 * predicted durations (pred_dur, src/model.rs:90-99), the text-encoder features of its tokens
 * (t_en columns, channel-major [512][n_tok]), the F0 and energy curves at 2N (the predictor's
 * F0/N outputs), its style ref_s (BatchItem::ref_s, 256 values; the decoder uses [0,128)) and its
 * noise source. */
typedef struct {
    const int64_t* dur;   /* [n_tok], each >= 1; N = sum(dur) */
    int32_t n_tok;
    const float* t_en;    /* [512][n_tok] */
    const float* f0;      /* [2N] */
    const float* energy;  /* [2N] */
    const float* ref_s;   /* [256] */
    int32_t noise_kind;   /* KK_NOISE_* */
    uint64_t seed;        /* counter seed (KK_NOISE_COUNTER) */
    const float* rand_ini;/* [9]        (KK_NOISE_FIXED) */
    const float* sine;    /* [600N * 9] (KK_NOISE_FIXED) */
    int64_t sine_len;
} kk_decoder_item;

/* Output (src/model.rs:101-104): the item's audio, 600 N samples at 24 kHz, owned by the caller
 * until released by kk_output_free.  The audio of one call lands in a block of pinned host memory
 * that the library keeps for reuse (the one-shot entries copy each group of items there as soon as
 * it is done); each item's pointer lies in that block, which is free again once kk_output_free has
 * released all of its items. */
typedef struct {
    float* audio;
    int64_t n_samples;
} kk_output;

/* The decoder + generator part of GpuKokoro::forward_batch (src/gpu_batch.rs:250-420): ragged
 * layout, duration expansion, decoder, harmonic source + STFT, generator, iSTFT, per-item audio in
 * input order.  `out` is a caller array of n entries.  The context keeps this entry's device
 * buffers between calls and reuses them for the next batch that fits (growing them when it does
 * not); every table and input of a call reaches the device in one copy.  Any failure releases the
 * kept buffers, so that a caller who splits the batch on KK_ERR_OOM (src/engine.rs:229-234) has the
 * whole device for the halves.
 * Test hooks, read from the environment at each call and plan creation:
 *   KOKORO_BATCH_NEGCTL_NOMASK (set: convolutions read neighbours and gaps as an item's own rows;
 *   the reference's negative control, src/gpu_batch.rs:62-66), KOKORO_HIP_TEST_OOM_ABOVE=k (a batch
 *   of more than k items fails with KK_ERR_OOM before allocating), KOKORO_HIP_TEST_POISON=1 (device
 *   buffers are filled with NaN bytes instead of being reused as they are).  Diagnostics, read once
 *   per process: KOKORO_HIP_TIMING=1 prints each call's host phase times to stderr (plan building,
 *   launches, the wait for the device, the output copy). */
int kk_forward_decoder_batch(kk_ctx* ctx, const kk_decoder_item* items, int n, kk_output* out, char* err,
                             size_t errlen);
void kk_output_free(kk_output* out, int n);

/* ------------------------------------------------------------------ the whole forward (ids -> audio)
 * kk_upload_model / kk_upload_checkpoint load the stages before the decoder as well when the table
 * holds them ("bert.*", "bert_encoder.*", "text_encoder.*", "predictor.*"): ALBERT, the text encoder
 * and the prosody predictor (Albert::load src/albert.rs:36-67, TextEncoder::load / Predictor::load
 * src/model.rs:29-88, Kokoro::from_weights src/model.rs:122-141). */

/* BatchItem (src/gpu_batch.rs:19-24): one utterance's input_ids (with the two boundary tokens),
 * style ref_s (256 values: [0,128) the decoder's, [128,256) the prosody predictor's), speed and
 * noise source.  A fixed noise source must hold 600 N * 9 values for the N frames the predicted
 * durations give (src/gpu_batch.rs:338); anything else is KK_ERR_INVALID. */
typedef struct {
    const int64_t* ids;   /* [n_ids], each in [0, 178) */
    int32_t n_ids;        /* 2..512 (src/gpu_batch.rs:184) */
    const float* ref_s;   /* [256] */
    float speed;          /* > 0, finite */
    int32_t noise_kind;   /* KK_NOISE_* */
    uint64_t seed;
    const float* rand_ini;/* [9]        (KK_NOISE_FIXED) */
    const float* sine;    /* [600N * 9] (KK_NOISE_FIXED) */
    int64_t sine_len;
} kk_item;

/* Output (src/model.rs:101-104): the audio (600 N samples, in the pinned output pool as kk_output)
 * and the predicted durations pred_dur [n_tok] (malloc'ed); both released by kk_result_free. */
typedef struct {
    float* audio;
    int64_t n_samples;
    int64_t* pred_dur;
    int32_t n_tok;
} kk_result;

/* GpuKokoro::forward_batch (src/gpu_batch.rs:179-420): the token phase (ALBERT, bert_encoder, the
 * duration encoder, the duration LSTM and projection; the text encoder beside them), the durations
 * from the logits on the host (durations_from_logits, src/model.rs:90-100: one copy of the logits
 * back), then the frame layout, the shared LSTM, the F0 / N stacks, the decoder, the generator and
 * the iSTFT.  Results in input order.  Kept buffers, failure release and test hooks as
 * kk_forward_decoder_batch.  Every BiLSTM recurrence runs each (item, direction) on a pair of CUs
 * that trade their halves of h each step; a block that waits more than 2 s for its partner (held
 * off its CU, e.g. by another process) ends its launch, and the call runs the forward again with
 * the one-CU kernel, which waits on no other block -- contention costs time, not an error (an
 * ids-level plan stays on the one-CU kernel for its later runs; every result path, kk_plan_sync
 * and taps included, runs that check first).  KOKORO_HIP_LSTM_SINGLE=1 (read once per process)
 * selects the one-CU kernel from the start; test hook KOKORO_HIP_TEST_LSTM_SILENT=1 (read at each
 * launch) makes every pair give up after a 10 us wait.  ALBERT's attention runs on the f32 matrix cores;
 * KOKORO_HIP_ATTENTION_VALU=1 (read once per process) selects the f32 VALU kernel instead. */
int kk_forward_batch(kk_ctx* ctx, const kk_item* items, int n, kk_result* out, char* err, size_t errlen);
void kk_result_free(kk_result* out, int n);

/* ------------------------------------------------------------------ plans (device-resident runs)
 * kk_forward_decoder_batch = kk_plan_create + kk_plan_run + kk_plan_fetch + kk_plan_free.
 * A plan builds the layout, uploads the inputs (one copy of all tables) and allocates every device
 * buffer once, and validates every launch's parameters (KK_ERR_INVALID at creation, never half-way
 * through a run); kk_plan_run only enqueues kernels (no allocation, no host synchronization), so it
 * can be timed with inputs already resident in HBM and run repeatedly.  A run that fails after
 * forking joins the side streams back into the context's stream before it returns.  It enqueues on the context's stream and on three
 * side streams of the context (the generator's independent resblock chains, the harmonic source
 * and noise branches), forked from and joined back into the context's stream within the run:
 * work enqueued on the context's stream after kk_plan_run sees all of it. */
int kk_plan_create(kk_ctx* ctx, const kk_decoder_item* items, int n, kk_plan** out, char* err, size_t errlen);
/* Generator-only plan: per item the decoder output x [512][2N] channel-major,
 * F0 [2N], ref_s [256], noise. */
typedef struct {
    const float* x;       /* [512][2N] */
    int32_t n_frames;     /* N */
    const float* f0;      /* [2N] */
    const float* ref_s;   /* [256] */
    int32_t noise_kind;
    uint64_t seed;
    const float* rand_ini;
    const float* sine;
    int64_t sine_len;
} kk_generator_item;
int kk_plan_create_generator(kk_ctx* ctx, const kk_generator_item* items, int n, kk_plan** out, char* err,
                             size_t errlen);
/* Snake-block plan: one AdaINResBlock1 (`prefix`, e.g.
 * "decoder.generator.resblocks.1") over n ragged items x_b [C][t_b], packed with `gap` zero
 * columns (snake_b, src/gpu_batch.rs:140-154). */
int kk_plan_create_snake(kk_ctx* ctx, const char* prefix, const float* const* x, const int64_t* t,
                         const float* const* ref_s, int n, int gap, kk_plan** out, char* err, size_t errlen);
/* The Snake block of kk_plan_create_snake + kk_plan_run on caller device memory, allocating nothing.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  x: device pointer,
 * time-major f32 [rows][C] (C = the block's channels), item b at rows [start[b], start[b] + len[b])
 * (spans disjoint, any rows between them), updated in place; ref_s: n host pointers to 128+ style
 * values.  Intermediates live in a fixed device scratch array of KK_NOALLOC_SCRATCH_BYTES per device
 * (held from the library's first use on that device until the process ends); calls beyond
 * KK_NOALLOC_MAX_ROWS rows or KK_NOALLOC_MAX_ITEMS items are refused with KK_ERR_INVALID.  Every
 * call on one device shares that device's array: calls that overlap on one device race.  The call
 * returns when x holds the result; a call that fails returns only after every kernel it enqueued has
 * finished, so x and the scratch are no longer written once the error is back. */
#define KK_NOALLOC_MAX_ROWS 65536
#define KK_NOALLOC_MAX_ITEMS 64
#define KK_NOALLOC_SCRATCH_BYTES (48u << 20)
int kk_snake_block_noalloc(kk_ctx* ctx, const char* prefix, float* x, int64_t rows, const int64_t* start,
                           const int64_t* len, int n, const float* const* ref_s, char* err, size_t errlen);
/* Ids-level plan (kk_forward_batch = kk_plan_create_full + run + fetch): creation runs the token
 * phase once and fixes the frame layout from its durations; kk_plan_run then runs the whole
 * forward, token phase included, on the same durations (the recomputed logits are identical). */
int kk_plan_create_full(kk_ctx* ctx, const kk_item* items, int n, kk_plan** out, char* err, size_t errlen);
/* The predicted durations of item `item` of an ids-level plan (valid while the plan lives). */
int kk_plan_durations(const kk_plan* plan, int item, const int64_t** dur, int32_t* n_tok);
/* Enqueue the plan's kernels; `until` = KK_STAGE_ALL or an earlier stage (for stage taps).
 * KK_STAGE_PROSODY (ids-level plans only): through the F0 / N curves and the text encoder. */
#define KK_STAGE_PROSODY 0
#define KK_STAGE_DECODER 1
#define KK_STAGE_SOURCE 2
#define KK_STAGE_GEN0 3
#define KK_STAGE_GEN1 4
#define KK_STAGE_POST 5
#define KK_STAGE_ALL 6
int kk_plan_run(kk_plan* plan, int until, char* err, size_t errlen);
int kk_plan_sync(kk_plan* plan, char* err, size_t errlen);
/* Copy each item's result to the host (audio for decoder/generator plans, [C][t_b] for snake
 * plans, as kk_output with n_samples = element count). */
int kk_plan_fetch(kk_plan* plan, kk_output* out, char* err, size_t errlen);
/* Copy a named device buffer of the last run to the host, per item and channel-major like the
 * reference's host tensors: "asr" [512][N], "decoder" [512][2N], "spec" [22][120N+1],
 * "gen0" [256][20N] (after a run until KK_STAGE_GEN0: generator stage 0's output as the next
 * layer's bf16 operand, leaky ReLU 0.1 applied, widened to f32), "post" [22][120N+1], "audio"
 * [600N], "har" [600N] (the harmonic source's samples, the STFT's input; only for plans created
 * with the test hook KOKORO_HIP_TEST_TAP_SOURCE=1 in the environment); of ids-level plans also "bert"
 * [768][T], "d" [640][T] (the duration encoder's output), "logits" [50][T], "t_en" [512][T],
 * "shared" [512][N], "f0" [2N], "n" [2N] (T = n_ids).  `dst` receives item `item` only; `count`
 * is its element count. */
int kk_plan_tap(kk_plan* plan, const char* name, int item, float* dst, int64_t count, char* err, size_t errlen);
typedef struct {
    int64_t n_items;
    int64_t ln;             /* frame-layout width (sum of N_b + 2) */
    int64_t frames;         /* sum of N_b */
    int64_t samples;        /* sum of 600 N_b */
    double conv_flop;       /* algorithmic conv FLOP of one run (valid columns, 2 per MAC) */
    double snake_flop;      /* of which in the Snake-block convs */
    int64_t device_bytes;   /* device memory held by the plan */
    int64_t launches;       /* kernels per run */
} kk_plan_info;
int kk_plan_get_info(const kk_plan* plan, kk_plan_info* info);
void kk_plan_free(kk_plan* plan);

/* ------------------------------------------------------------------ output formats (src/wav.rs)
 * PCM_16 encoding of the last run's audio on the device (wav::encode, src/wav.rs:63-80): per
 * sample v = round_ties_even(s * 32767) in f32; values outside [-32768, 32767] (NaN and the
 * infinities included) are clamped and counted, NaN stores 0.  dst[b] receives item b's 600 N_b
 * samples; clipped (optional) its count.  Half the bytes of kk_plan_fetch over PCIe. */
int kk_plan_fetch_pcm16(kk_plan* plan, int16_t* const* dst, int64_t* clipped, char* err, size_t errlen);
/* Asynchronous output path, so that the host writes batch n while the GPU computes batch n + 1
 * (the reference overlaps its WAV writer threads with synthesis, src/cli.rs:553-622).
 * kk_host_alloc / kk_host_free: pinned host memory (hipHostMalloc).
 * kk_plan_item_samples: item `item`'s sample offset and count in the plan's sample layout
 * (offset 600 a_b, a_b = sum_{j<b} (N_j + 2); count 600 N_b).
 * kk_plan_fetch_pcm16_async: enqueues the PCM_16 encoding of kk_plan_fetch_pcm16 and one copy of
 * the whole sample layout (600 ln int16, gap samples 0) into `dst`, and of the clip counts into
 * `clipped` (optional, n_items int64), behind the plan's work on the context's stream, and returns.
 * Both must be pinned memory from kk_host_alloc.  kk_plan_fetch_wait blocks until they have
 * landed; a later kk_plan_run of the plan is ordered after the copy (one stream), so it may be
 * enqueued before the wait.  One fetch per plan may be pending. */
int kk_host_alloc(kk_ctx* ctx, size_t bytes, void** out, char* err, size_t errlen);
void kk_host_free(void* p);
int kk_plan_item_samples(const kk_plan* plan, int item, int64_t* offset, int64_t* count);
int kk_plan_fetch_pcm16_async(kk_plan* plan, int16_t* dst, int64_t* clipped, char* err, size_t errlen);
int kk_plan_fetch_wait(kk_plan* plan, char* err, size_t errlen);
/* The same encoding of a host array (uploads, encodes on the device, downloads). */
int kk_encode_pcm16(kk_ctx* ctx, const float* audio, int64_t n, int16_t* out, int64_t* clipped, char* err,
                    size_t errlen);
/* The canonical 44-byte mono RIFF/WAVE header (wav::header, src/wav.rs:43-61): format tag 1
 * (PCM_16) or 3 (IEEE float32); data_bytes above 2^32 - 1 - 36 is refused (check_riff_size,
 * src/wav.rs:34-40), never wrapped. */
#define KK_WAV_PCM16 0
#define KK_WAV_FLOAT32 1
int kk_wav_header(int format, uint32_t sample_rate, uint64_t data_bytes, uint8_t* out, char* err, size_t errlen);

/* ------------------------------------------------------------------ measurement
 * With profiling on, kk_plan_run runs every kernel on the context's stream (no side streams, so
 * each kernel has the GPU to itself) and brackets every launch with HIP events there;
 * kk_profile_read reports, per kernel class with at least one launch since the last read, the summed
 * event time and the algorithmic FLOP and bytes of those launches (valid rows only; bytes = the
 * data the step must read and write once).  Classes: the MFMA convolutions "snake_conv",
 * "decoder_conv", "convt", "post_conv"; "stats_tiles", "finalize", "style_fc", "expand", "f0n_conv",
 * "copy_cols", "adain_pool", "noise_conv0", "noise_conv1", "phase_pre", "source_stft", "istft". */
int kk_set_profiling(kk_ctx* ctx, int on);
typedef struct {
    char name[32];
    int64_t launches;
    double ms;
    double flop;
    double bytes;
} kk_profile_entry;
int kk_profile_read(kk_ctx* ctx, kk_profile_entry* out, int max, int* n_out, char* err, size_t errlen);
/* The launches recorded since the last kk_profile_read, one record each in launch order (the first
 * `max`; *n_out = how many were recorded), without clearing them: the layer's state-dict prefix and
 * step (e.g. "resblocks.3.d1.conv1"), or the kernel class for the other kernels. */
typedef struct {
    char name[48];
    char cls[32];
    double ms;
    double flop;
    double bytes;
} kk_launch_record;
int kk_profile_launches(kk_ctx* ctx, kk_launch_record* out, int max, int* n_out, char* err, size_t errlen);

/* ------------------------------------------------------------------ host rules (bit-exact)
 * durations_from_logits (src/model.rs:90-99): d_i = max(1, round_half_even(sum_j sigmoid(l_ij) /
 * speed)) over [t][50] logits. */
int kk_durations_from_logits(const float* logits, int t, float speed, int64_t* out);
/* Frame layout (src/gpu_batch.rs:250-263): a[b] = sum_{j<b}(N_j + 2), returns ln. */
int64_t kk_layout_frames(const int64_t* nfs, int n, int64_t* a_out);
/* col_item of a domain of width l with item spans [start_b, start_b + len_b) (Dom::new,
 * src/gpu_batch.rs:42-54); KK_ERR_INVALID on overflow or overlap. */
int kk_layout_col_item(int64_t l, const int64_t* start, const int64_t* len, int n, int32_t* col_item);
/* Frame -> token-row expansion table (src/gpu_batch.rs:265-276). */
int kk_layout_src_row(const int64_t* const* dur, const int32_t* n_tok, int n, const int64_t* tstart,
                      const int64_t* a, int64_t ln, int32_t* src_row);

#ifdef __cplusplus
}
#endif
#endif
