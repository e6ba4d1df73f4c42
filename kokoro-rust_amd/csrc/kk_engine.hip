// kk_engine.hip -- host side of the gfx950 decoder + generator path: context, model hydration,
// ragged batch plans and the launch sequence, behind the C ABI of include/kokoro_hip.h.
//
// Reference structure being replaced: src/gpu.rs (Gpu, GConv/GConvT/GAdaIn/GResBlk/GSnakeBlk
// hydration) and src/gpu_batch.rs (Dom layout and forward_batch from the durations on).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "kk_ckpt.h"
#include "kk_common.h"
#include "kk_host.h"
#include "kk_kernels.h"
#include "kokoro_hip.h"

namespace kk {

struct Err {
    int code;
    std::string msg;
};

[[noreturn]] static void fail(int code, const std::string& m) { throw Err{code, m}; }
static void check(bool ok, const std::string& m) {
    if (!ok) fail(KK_ERR_INVALID, m);
}
#define KK_HIP(x)                                                                                             \
    do {                                                                                                      \
        hipError_t e_ = (x);                                                                                  \
        if (e_ != hipSuccess)                                                                                 \
            ::kk::fail(e_ == hipErrorOutOfMemory ? KK_ERR_OOM : KK_ERR_HIP,                                   \
                       std::string(#x) + ": " + hipGetErrorString(e_));                                       \
    } while (0)

// ------------------------------------------------------------------ device buffers
// A device allocation (cap > 0) or a view of part of another one (cap == 0: not freed here).
// alloc() keeps an owned allocation that is large enough (grow-only reuse: the one-shot entry's
// cached plan runs batch after batch in the same memory).
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;  // in use
    size_t cap = 0;    // owned capacity
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes), cap(o.cap) { o.p = nullptr, o.bytes = 0, o.cap = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        release();
        p = o.p, bytes = o.bytes, cap = o.cap;
        o.p = nullptr, o.bytes = 0, o.cap = 0;
        return *this;
    }
    ~DevBuf() { release(); }
    void release() {
        if (p && cap) (void)hipFree(p);
        p = nullptr, bytes = 0, cap = 0;
    }
    // Returns true when the memory is new (its contents undefined until written).
    bool alloc(size_t n) {
        if (n == 0) n = 16;
        if (p && cap >= n) {
            bytes = n;
            return false;
        }
        release();
        hipError_t e = hipMalloc(&p, n);
        if (e != hipSuccess) {
            p = nullptr;
            (void)hipGetLastError();
            fail(e == hipErrorOutOfMemory ? KK_ERR_OOM : KK_ERR_HIP,
                 "hipMalloc(" + std::to_string(n) + " bytes): " + hipGetErrorString(e));
        }
        bytes = cap = n;
        return true;
    }
    void view(void* base, size_t n) {
        release();
        p = base, bytes = n;
    }
    template <class T>
    void upload(const T* h, size_t count) {
        release();
        alloc(count * sizeof(T));
        if (count) KK_HIP(hipMemcpy(p, h, count * sizeof(T), hipMemcpyHostToDevice));
    }
    template <class T>
    void upload(const std::vector<T>& v) {
        upload(v.data(), v.size());
    }
    template <class T>
    T* as() const {
        return (T*)p;
    }
};

static uint16_t bf16_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) u |= 0x00400000u;
        return (uint16_t)(u >> 16);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static uint64_t splitmix_at(uint64_t seed, uint64_t ctr) {
    uint64_t x = seed + (ctr + 1ull) * 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// ------------------------------------------------------------------ model on the device
struct MConv {
    DevBuf w, b;
    int cin = 0, cin_pad = 0, cout = 0, m = 0, m_pad = 0, k = 0, dil = 1, pad = 0, shape = 0;
    bool bias = false;
};
struct MAdain {
    DevBuf nw, nb;
    int c = 0, gb_off = 0;
};
struct MSnake {
    std::string name;  // state-dict prefix after "decoder.generator."
    MConv c1[3], c2[3];
    MAdain a1[3], a2[3];
    DevBuf ar1[3], ai1[3], ar2[3], ai2[3];
    int c = 0;
};
struct MResblk {
    std::string name;  // state-dict prefix after "decoder."
    MConv conv1, conv2, conv1x1;
    bool has1x1 = false, up = false;
    MAdain n1, n2;
    DevBuf pool_w, pool_b;
    int din = 0, dout = 0;
};
struct MNoiseConv {
    DevBuf b, wp;  // wp: split-bf16 matrix-core packing
    int cout = 0, k = 0, stride = 1, pad = 0;
};
// A Linear [dout][din] on the MFMA conv kernel (k = 1), in pieces of at most 1024 output rows (the
// kernel stages the bias of one piece in LDS); piece i writes output columns [col0[i], ...).
struct MLinear {
    std::vector<MConv> piece;
    std::vector<int> col0;
    int din = 0, dout = 0;
};
// BiLstm (src/nn.rs:168-190) as the reference's GLstm (src/gpu.rs:600-613): W_ih of both directions
// as one linear (gx [rows][2048], forward | reverse, bias b_ih), W_hh f32 k-major [2][256][1024],
// b_hh [2][1024].
struct MLstm {
    MLinear wih;
    DevBuf whh_t, bhh;
};
// The stages before the decoder (src/albert.rs:36-67, src/model.rs:21-88, 122-141).
struct MUp {
    DevBuf word, pos, tok0, emb_g, emb_b;  // ALBERT embeddings
    MLinear map_in, qkv, dense, ffn, ffn_out, bert_enc;
    DevBuf attn_g, attn_b, full_g, full_b;
    DevBuf te_emb;  // text encoder
    MConv te_cnn[3];
    DevBuf te_g[3], te_b[3];
    MLstm te_lstm, dur_lstm[3], pred_lstm, shared;
    int dur_gb_off[3] = {0, 0, 0};  // AdaLayerNorm projections in the prosody style table
    MLinear dur_proj;
    MResblk f0[3], nn[3];
    DevBuf f0p_w, f0p_b, np_w, np_b;  // F0_proj / N_proj (256 -> 1)
    DevBuf style_wt, style_b;         // every prosody-style projection, transposed [128][rows]
    int style_rows = 0;
    bool ready = false;
};
struct Model {
    MUp up;
    MResblk encode, decode[4];
    DevBuf f0w, f0b, nw_, nb_;
    MConv asr_res;
    DevBuf lw;
    float lb = 0.f;
    MNoiseConv nc[2];
    MSnake noise_res[2];
    MConv ups[2];
    int ups_stride[2] = {10, 6}, ups_pad[2] = {5, 3}, ups_cin[2] = {512, 256}, ups_cout[2] = {256, 128};
    MSnake rb[6];
    MConv post;
    DevBuf style_wt, style_b;
    int style_rows = 0;
    bool ready = false;
};

struct ProfRec {
    int cls;
    double flop, bytes;
    hipEvent_t e0, e1;
    std::string label;  // the layer (state-dict prefix and step) or the kernel class
};
// Kernel classes of the per-launch profile: the MFMA convolutions (by role), then the bandwidth
// and glue kernels.
enum {
    PC_SNAKE = 0, PC_DECODER, PC_CONVT, PC_POST, PC_STATS, PC_FINALIZE, PC_STYLE, PC_EXPAND, PC_F0N, PC_COPY,
    PC_POOL, PC_NOISE0, PC_NOISE1, PC_PHASE, PC_SOURCE, PC_ISTFT, PC_LINEAR, PC_ATTN, PC_LSTM, PC_PCONV, PC_ROWS,
    PC_COUNT
};
static const char* kProfNames[PC_COUNT] = {"snake_conv", "decoder_conv", "convt",      "post_conv",
                                           "stats_tiles", "finalize",    "style_fc",   "expand",
                                           "f0n_conv",    "copy_cols",   "adain_pool", "noise_conv0",
                                           "noise_conv1", "phase_pre",   "source_stft", "istft",
                                           "linear",      "attention",   "lstm",       "prosody_conv",
                                           "rows"};

// Host staging of a plan's tables and inputs.  Everything a plan uploads (layout tables, tile lists,
// work lists, the items' inputs) is written into one pinned host buffer of the context and reaches
// the device in one copy into the plan's table buffer; every staged DevBuf then becomes a view of
// its range there.
struct Staging {
    char* host = nullptr;  // pinned (hipHostMalloc), grow-only; or `heap` (pageable)
    size_t cap = 0, used = 0;
    bool pageable = false;  // host heap instead of pinned memory (the no-allocation entry point)
    std::vector<char> heap;
    hipEvent_t done = nullptr;  // recorded after the last copy out of `host`
    bool pending = false;
    struct Ref {
        DevBuf* buf;
        size_t off, bytes;
    };
    std::vector<Ref> refs;
};

}  // namespace kk

struct kk_plan;
struct kk_ctx {
    int device = 0;
    int n_cu = 1;
    std::set<kk_plan*> plans;  // live plans: released (and orphaned) by kk_close
    hipStream_t stream = nullptr;
    // three more streams (default priority): the generator's independent resblock chains (0, 1) and
    // the source + noise branches (2)
    hipStream_t side[3] = {nullptr, nullptr, nullptr};
    hipEvent_t join_ev[3] = {nullptr, nullptr, nullptr};  // error path: side streams joined back
    std::string name;
    kk::Model model;
    bool profiling = false;
    std::vector<kk::ProfRec> prof;
    std::vector<hipEvent_t> event_pool;
    kk::Staging stage;
    kk::Staging stage_late;  // the one-shot decoder entry's t_en, staged while its first kernels run
    // kk_forward_decoder_batch's plan, kept between calls: its device buffers are reused whenever
    // the next batch fits (released on any failure, so that a split batch can use the memory)
    kk_plan* oneshot = nullptr;
    // device address of this device's copy of the no-allocation entry point's scratch array
    unsigned char* scratch = nullptr;
};

namespace kk {

static int round_up(int v, int m) { return (v + m - 1) / m * m; }

// Weight table lookup (names as the checkpoint's state dict).
struct Table {
    std::map<std::string, const kk_tensor*> byname;
    // Weights::get_instance_norm_affine (src/weights.rs:76-84): the AdaIN InstanceNorm affine
    // parameters are absent from the released checkpoint and take torch's initial values (weight 1,
    // bias 0); only names ending in ".norm.weight" / ".norm.bias" may default, and only when this
    // is set (checkpoint uploads).
    bool norm_defaults = false;
    mutable std::vector<std::unique_ptr<std::vector<float>>> defaults;
    const float* get(const std::string& name, int64_t numel) const {
        auto it = byname.find(name);
        if (it == byname.end() && norm_defaults) {
            auto ends = [&](const char* suf) {
                const size_t k = std::strlen(suf);
                return name.size() >= k && name.compare(name.size() - k, k, suf) == 0;
            };
            if (ends(".norm.weight") || ends(".norm.bias")) {
                defaults.push_back(std::make_unique<std::vector<float>>((size_t)numel, ends(".norm.weight") ? 1.f : 0.f));
                return defaults.back()->data();
            }
        }
        check(it != byname.end(), "missing tensor " + name);
        check(it->second->numel == numel, "tensor " + name + " has " + std::to_string(it->second->numel) +
                                              " values, expected " + std::to_string(numel));
        check(it->second->data != nullptr, "tensor " + name + " has no data");
        return it->second->data;
    }
};

// A stride-1 conv, w [cout][cin][k] -> packed [k][cin_pad/16][m_pad][16] bf16 (one MFMA A fragment,
// 32 rows x 16 channels, is a contiguous 1 KB).
static void load_conv_raw(MConv& c, const float* w, const float* bias_v, int cin, int cout, int k, int pad, int dil,
                          int shape) {
    c.cin = cin, c.cout = cout, c.k = k, c.pad = pad, c.dil = dil, c.shape = shape, c.bias = bias_v != nullptr;
    c.cin_pad = round_up(cin, 64);
    c.m = cout;
    c.m_pad = round_up(cout, kShapeM[shape]);
    const int n16 = c.cin_pad / 16;
    std::vector<uint16_t> pk((size_t)k * n16 * c.m_pad * 16, 0);
    for (int co = 0; co < cout; co++)
        for (int ci = 0; ci < cin; ci++)
            for (int kk = 0; kk < k; kk++)
                pk[(((size_t)kk * n16 + ci / 16) * c.m_pad + co) * 16 + (ci & 15)] =
                    bf16_bits(w[((size_t)co * cin + ci) * k + kk]);
    c.w.upload(pk);
    // a layer without a bias gets a zero vector: the conv epilogue always reads one
    std::vector<float> b(round_up(cout, 4), 0.f);
    if (bias_v) std::memcpy(b.data(), bias_v, sizeof(float) * cout);
    c.b.upload(b);
}
static void load_conv(MConv& c, const Table& t, const std::string& p, int cin, int cout, int k, int pad, int dil,
                      bool bias, int shape) {
    load_conv_raw(c, t.get(p + ".weight", (int64_t)cout * cin * k), bias ? t.get(p + ".bias", cout) : nullptr, cin,
                  cout, k, pad, dil, shape);
}

// ConvTranspose1d with K = 2 * stride as a 2-tap conv over input rows (i - 1, i) whose GEMM row
// m = phase * cout + co produces output column stride * i + phase - pad (see kk_conv.hip).
static void load_convt(MConv& c, const Table& t, const std::string& p, int cin, int cout, int kw, int stride) {
    check(kw == 2 * stride, p + ": polyphase ConvT needs K = 2 * stride");
    c.cin = cin, c.cout = cout, c.k = 2, c.pad = 1, c.dil = 1, c.shape = SHAPE_256x128, c.bias = true;
    c.cin_pad = round_up(cin, 64);
    c.m = stride * cout;
    c.m_pad = round_up(c.m, kShapeM[c.shape]);
    const float* w = t.get(p + ".weight", (int64_t)cin * cout * kw);
    const int n16 = c.cin_pad / 16;
    std::vector<uint16_t> pk((size_t)2 * n16 * c.m_pad * 16, 0);
    for (int tap = 0; tap < 2; tap++)
        for (int r = 0; r < stride; r++)
            for (int co = 0; co < cout; co++) {
                const int m = r * cout + co, kk = tap == 0 ? r + stride : r;
                for (int ci = 0; ci < cin; ci++)
                    pk[(((size_t)tap * n16 + ci / 16) * c.m_pad + m) * 16 + (ci & 15)] =
                        bf16_bits(w[((size_t)ci * cout + co) * kw + kk]);
            }
    c.w.upload(pk);
    std::vector<float> b(round_up(cout, 4), 0.f);
    std::memcpy(b.data(), t.get(p + ".bias", cout), sizeof(float) * cout);
    c.b.upload(b);
}

struct StyleRows {
    std::vector<float> wt_rows;  // [rows][128] (transposed at upload)
    std::vector<float> bias;
    int rows = 0;
};

static void load_adain(MAdain& a, const Table& t, const std::string& p, int c, StyleRows& sr) {
    a.c = c;
    a.nw.upload(t.get(p + ".norm.weight", c), c);
    a.nb.upload(t.get(p + ".norm.bias", c), c);
    const float* fw = t.get(p + ".fc.weight", (int64_t)2 * c * kStyleDim);
    const float* fb = t.get(p + ".fc.bias", 2 * c);
    a.gb_off = sr.rows;
    sr.wt_rows.insert(sr.wt_rows.end(), fw, fw + (size_t)2 * c * kStyleDim);
    sr.bias.insert(sr.bias.end(), fb, fb + 2 * c);
    sr.rows += 2 * c;
}

// AdaInResBlock1::load (src/nn.rs:154-165): convs1 pad (k d - d) / 2 dil d; convs2 pad (k - 1) / 2.
static void load_snake(MSnake& s, const Table& t, const std::string& p, int c, int k, StyleRows& sr) {
    static const int dil[3] = {1, 3, 5};
    s.c = c;
    s.name = p.substr(p.find("generator.") == std::string::npos ? 0 : p.find("generator.") + 10);
    const int shape = c >= 256 ? SHAPE_256x128 : SHAPE_128x256;
    for (int i = 0; i < 3; i++) {
        const std::string si = std::to_string(i);
        load_conv(s.c1[i], t, p + ".convs1." + si, c, c, k, (k * dil[i] - dil[i]) / 2, dil[i], true, shape);
        load_conv(s.c2[i], t, p + ".convs2." + si, c, c, k, (k - 1) / 2, 1, true, shape);
        load_adain(s.a1[i], t, p + ".adain1." + si, c, sr);
        load_adain(s.a2[i], t, p + ".adain2." + si, c, sr);
        for (int j = 0; j < 2; j++) {
            const float* al = t.get(p + (j ? ".alpha2." : ".alpha1.") + si, c);
            std::vector<float> rev(c), inv(c);
            for (int ch = 0; ch < c; ch++) {
                check(al[ch] != 0.f && std::isfinite(al[ch]), p + ": Snake alpha must be finite and nonzero");
                rev[ch] = (float)((double)al[ch] / (2.0 * M_PI));
                inv[ch] = 1.0f / al[ch];
            }
            (j ? s.ar2[i] : s.ar1[i]).upload(rev);
            (j ? s.ai2[i] : s.ai1[i]).upload(inv);
        }
    }
}

// AdainResBlk1d::load (src/nn.rs:119-140).
static void load_resblk(MResblk& r, const Table& t, const std::string& p, int din, int dout, bool up,
                        StyleRows& sr) {
    r.din = din, r.dout = dout, r.up = up;
    r.name = p.substr(p.find("decoder.") == std::string::npos ? 0 : 8);
    load_conv(r.conv1, t, p + ".conv1", din, dout, 3, 1, 1, true, SHAPE_256x128);
    load_conv(r.conv2, t, p + ".conv2", dout, dout, 3, 1, 1, true, SHAPE_256x128);
    load_adain(r.n1, t, p + ".norm1", din, sr);
    load_adain(r.n2, t, p + ".norm2", dout, sr);
    r.has1x1 = din != dout;
    if (r.has1x1) load_conv(r.conv1x1, t, p + ".conv1x1", din, dout, 1, 0, 1, false, SHAPE_256x128);
    if (up) {
        r.pool_w.upload(t.get(p + ".pool.weight", (int64_t)din * 3), (size_t)din * 3);
        r.pool_b.upload(t.get(p + ".pool.bias", din), din);
    }
}

// ------------------------------------------------------------------ the stages before the decoder
// One piece of a linear: rows [r0, r0 + rows) of w [.][din] (and of its bias) -> output columns
// col0 + [0, rows).
static void add_piece(MLinear& L, const float* w, const float* b, int din, int r0, int rows, int col0, int shape) {
    L.piece.emplace_back();
    load_conv_raw(L.piece.back(), w + (size_t)r0 * din, b ? b + r0 : nullptr, din, rows, 1, 0, 1, shape);
    L.col0.push_back(col0);
    L.din = din;
    L.dout = std::max(L.dout, col0 + rows);
}
// Linear::load (src/nn.rs:14-22) of `prefix`, in pieces of at most 1024 rows.
static void load_linear(MLinear& L, const Table& t, const std::string& prefix, int din, int dout, int col0 = 0,
                        int shape = SHAPE_256x128) {
    const float* w = t.get(prefix + ".weight", (int64_t)dout * din);
    const float* b = t.get(prefix + ".bias", dout);
    for (int r0 = 0; r0 < dout; r0 += 1024) add_piece(L, w, b, din, r0, std::min(1024, dout - r0), col0 + r0, shape);
}
// BiLstm::load (src/nn.rs:178-189): torch.nn.LSTM names, H = 256.
static void load_lstm(MLstm& l, const Table& t, const std::string& p, int din) {
    constexpr int H = 256;
    std::vector<float> whh_t((size_t)2 * H * 4 * H), bhh((size_t)2 * 4 * H);
    for (int d = 0; d < 2; d++) {
        const std::string sfx = d ? "_reverse" : "";
        const float* wih = t.get(p + ".weight_ih_l0" + sfx, (int64_t)4 * H * din);
        const float* bih = t.get(p + ".bias_ih_l0" + sfx, 4 * H);
        add_piece(l.wih, wih, bih, din, 0, 4 * H, d * 4 * H, SHAPE_256x128);
        const float* whh = t.get(p + ".weight_hh_l0" + sfx, (int64_t)4 * H * H);
        for (int r = 0; r < 4 * H; r++)
            for (int k = 0; k < H; k++) whh_t[((size_t)d * H + k) * 4 * H + r] = whh[(size_t)r * H + k];
        std::memcpy(&bhh[(size_t)d * 4 * H], t.get(p + ".bias_hh_l0" + sfx, 4 * H), sizeof(float) * 4 * H);
    }
    l.whh_t.upload(whh_t);
    l.bhh.upload(bhh);
}
static void upload_style_table(DevBuf& wt_d, DevBuf& b_d, int& rows, const StyleRows& sr) {
    std::vector<float> wt((size_t)kStyleDim * sr.rows);
    for (int r = 0; r < sr.rows; r++)
        for (int k = 0; k < kStyleDim; k++) wt[(size_t)k * sr.rows + r] = sr.wt_rows[(size_t)r * kStyleDim + k];
    wt_d.upload(wt);
    b_d.upload(sr.bias);
    rows = sr.rows;
}

// ALBERT, bert_encoder, the text encoder and the prosody predictor (Albert::load src/albert.rs:36-67,
// TextEncoder::load / Predictor::load src/model.rs:29-88, Kokoro::from_weights src/model.rs:122-141).
static void load_upstream(MUp& u, const Table& t) {
    constexpr int NT = 178, EMB = 128, HID = 768, FFN = 2048, POS = 512, HIDDEN = 512;
    u.ready = false;
    u.word.upload(t.get("bert.embeddings.word_embeddings.weight", NT * EMB), (size_t)NT * EMB);
    u.pos.upload(t.get("bert.embeddings.position_embeddings.weight", POS * EMB), (size_t)POS * EMB);
    u.tok0.upload(t.get("bert.embeddings.token_type_embeddings.weight", 2 * EMB), EMB);  // token type 0
    u.emb_g.upload(t.get("bert.embeddings.LayerNorm.weight", EMB), EMB);
    u.emb_b.upload(t.get("bert.embeddings.LayerNorm.bias", EMB), EMB);
    const std::string L = "bert.encoder.albert_layer_groups.0.albert_layers.0";
    u.map_in = MLinear{}, u.qkv = MLinear{}, u.dense = MLinear{}, u.ffn = MLinear{}, u.ffn_out = MLinear{};
    u.bert_enc = MLinear{}, u.dur_proj = MLinear{};
    load_linear(u.map_in, t, "bert.encoder.embedding_hidden_mapping_in", EMB, HID);
    load_linear(u.qkv, t, L + ".attention.query", HID, HID, 0);
    load_linear(u.qkv, t, L + ".attention.key", HID, HID, HID);
    load_linear(u.qkv, t, L + ".attention.value", HID, HID, 2 * HID);
    load_linear(u.dense, t, L + ".attention.dense", HID, HID);
    u.attn_g.upload(t.get(L + ".attention.LayerNorm.weight", HID), HID);
    u.attn_b.upload(t.get(L + ".attention.LayerNorm.bias", HID), HID);
    load_linear(u.ffn, t, L + ".ffn", HID, FFN);
    load_linear(u.ffn_out, t, L + ".ffn_output", FFN, HID);
    u.full_g.upload(t.get(L + ".full_layer_layer_norm.weight", HID), HID);
    u.full_b.upload(t.get(L + ".full_layer_layer_norm.bias", HID), HID);
    load_linear(u.bert_enc, t, "bert_encoder", HID, HIDDEN);
    // text encoder: Conv1d 512 -> 512 k5 p2, LayerNorm(gamma, beta), BiLSTM
    u.te_emb.upload(t.get("text_encoder.embedding.weight", NT * HIDDEN), (size_t)NT * HIDDEN);
    for (int i = 0; i < 3; i++) {
        const std::string c = "text_encoder.cnn." + std::to_string(i);
        load_conv(u.te_cnn[i], t, c + ".0", HIDDEN, HIDDEN, 5, 2, 1, true, SHAPE_256x128);
        u.te_g[i].upload(t.get(c + ".1.gamma", HIDDEN), HIDDEN);
        u.te_b[i].upload(t.get(c + ".1.beta", HIDDEN), HIDDEN);
    }
    u.te_lstm = MLstm{}, u.pred_lstm = MLstm{}, u.shared = MLstm{};
    load_lstm(u.te_lstm, t, "text_encoder.lstm", HIDDEN);
    // prosody predictor: its style is ref_s[128:256] (src/gpu_batch.rs:206-210)
    StyleRows sr;
    const int cin = HIDDEN + kStyleDim;
    for (int i = 0; i < 3; i++) {
        u.dur_lstm[i] = MLstm{};
        load_lstm(u.dur_lstm[i], t, "predictor.text_encoder.lstms." + std::to_string(2 * i), cin);
        const std::string fc = "predictor.text_encoder.lstms." + std::to_string(2 * i + 1) + ".fc";
        const float* fw = t.get(fc + ".weight", (int64_t)2 * HIDDEN * kStyleDim);
        const float* fb = t.get(fc + ".bias", 2 * HIDDEN);
        u.dur_gb_off[i] = sr.rows;
        sr.wt_rows.insert(sr.wt_rows.end(), fw, fw + (size_t)2 * HIDDEN * kStyleDim);
        sr.bias.insert(sr.bias.end(), fb, fb + 2 * HIDDEN);
        sr.rows += 2 * HIDDEN;
    }
    load_lstm(u.pred_lstm, t, "predictor.lstm", cin);
    load_linear(u.dur_proj, t, "predictor.duration_proj.linear_layer", HIDDEN, 50, 0, SHAPE_64x256);
    load_lstm(u.shared, t, "predictor.shared", cin);
    for (int s = 0; s < 2; s++) {
        MResblk* blk = s == 0 ? u.f0 : u.nn;
        const std::string nm = std::string("predictor.") + (s == 0 ? "F0" : "N");
        load_resblk(blk[0], t, nm + ".0", HIDDEN, HIDDEN, false, sr);
        load_resblk(blk[1], t, nm + ".1", HIDDEN, HIDDEN / 2, true, sr);
        load_resblk(blk[2], t, nm + ".2", HIDDEN / 2, HIDDEN / 2, false, sr);
    }
    u.f0p_w.upload(t.get("predictor.F0_proj.weight", HIDDEN / 2), HIDDEN / 2);
    u.f0p_b.upload(t.get("predictor.F0_proj.bias", 1), 1);
    u.np_w.upload(t.get("predictor.N_proj.weight", HIDDEN / 2), HIDDEN / 2);
    u.np_b.upload(t.get("predictor.N_proj.bias", 1), 1);
    upload_style_table(u.style_wt, u.style_b, u.style_rows, sr);
    u.ready = true;
}

static void load_model(kk_ctx* ctx, const kk_tensor* tensors, int n, bool norm_defaults = false) {
    Table t;
    t.norm_defaults = norm_defaults;
    for (int i = 0; i < n; i++) {
        check(tensors[i].name != nullptr, "tensor without a name");
        t.byname[tensors[i].name] = &tensors[i];
    }
    Model& m = ctx->model;
    m.ready = false;
    StyleRows sr;
    // Shapes: Decoder::load / Generator::load (src/vocoder.rs:54-111).
    load_resblk(m.encode, t, "decoder.encode", 514, 1024, false, sr);
    for (int i = 0; i < 4; i++)
        load_resblk(m.decode[i], t, "decoder.decode." + std::to_string(i), 1090, i == 3 ? 512 : 1024, i == 3, sr);
    m.f0w.upload(t.get("decoder.F0_conv.weight", 3), 3);
    m.f0b.upload(t.get("decoder.F0_conv.bias", 1), 1);
    m.nw_.upload(t.get("decoder.N_conv.weight", 3), 3);
    m.nb_.upload(t.get("decoder.N_conv.bias", 1), 1);
    load_conv(m.asr_res, t, "decoder.asr_res.0", 512, 64, 1, 0, 1, true, SHAPE_64x256);
    const std::string g = "decoder.generator";
    m.lw.upload(t.get(g + ".m_source.l_linear.weight", kHarmonics), kHarmonics);
    m.lb = t.get(g + ".m_source.l_linear.bias", 1)[0];
    const int nc_cout[2] = {256, 128}, nc_k[2] = {12, 1}, nc_s[2] = {6, 1}, nc_p[2] = {3, 0};
    for (int i = 0; i < 2; i++) {
        const std::string p = g + ".noise_convs." + std::to_string(i);
        MNoiseConv& c = m.nc[i];
        c.cout = nc_cout[i], c.k = nc_k[i], c.stride = nc_s[i], c.pad = nc_p[i];
        const float* w = t.get(p + ".weight", (int64_t)c.cout * 22 * c.k);
        c.b.upload(t.get(p + ".bias", c.cout), c.cout);
        {
            // A fragments of the split-precision kernels: [32-row tile mt][K step st][part][lane][e]
            // = the bf16 rounding (part 0) or the bf16 rounding of the remainder (part 1) of
            // W[32 mt + lane % 32][ci][tap], k = 16 st + 8 (lane / 32) + e = 24 tap + ci (ci >= 22: 0;
            // noise_convs.1: k = ci, two steps)
            const int kSteps = c.k == 12 ? 18 : 2;
            std::vector<uint16_t> wp((size_t)(c.cout / 32) * kSteps * 2 * 64 * 8, 0);
            for (int mt = 0; mt < c.cout / 32; mt++)
                for (int st = 0; st < kSteps; st++)
                    for (int lane = 0; lane < 64; lane++)
                        for (int e = 0; e < 8; e++) {
                            const int k = 16 * st + 8 * (lane / 32) + e;
                            const int tap = c.k == 12 ? k / 24 : 0, ci = c.k == 12 ? k % 24 : k;
                            const float v = ci < 22 ? w[((size_t)(32 * mt + lane % 32) * 22 + ci) * c.k + tap] : 0.f;
                            const uint16_t hi = bf16_bits(v);
                            uint32_t hb = (uint32_t)hi << 16;
                            float hf;
                            std::memcpy(&hf, &hb, 4);
                            const size_t o = ((((size_t)mt * kSteps + st) * 2) * 64 + lane) * 8 + e;
                            wp[o] = hi;
                            wp[o + 64 * 8] = bf16_bits(v - hf);
                        }
            c.wp.upload(wp);
        }
    }
    load_snake(m.noise_res[0], t, g + ".noise_res.0", 256, 7, sr);
    load_snake(m.noise_res[1], t, g + ".noise_res.1", 128, 11, sr);
    load_convt(m.ups[0], t, g + ".ups.0", 512, 256, 20, 10);
    load_convt(m.ups[1], t, g + ".ups.1", 256, 128, 12, 6);
    static const int ks[3] = {3, 7, 11};
    for (int i = 0; i < 6; i++)
        load_snake(m.rb[i], t, g + ".resblocks." + std::to_string(i), i < 3 ? 256 : 128, ks[i % 3], sr);
    load_conv(m.post, t, g + ".conv_post", 128, 22, 7, 3, 1, true, SHAPE_32x256);
    // style projections of every AdaIN, transposed [128][rows]
    upload_style_table(m.style_wt, m.style_b, m.style_rows, sr);
    // the stages before the decoder, when the table holds them (kk_forward_batch needs them)
    m.up.ready = false;
    if (t.byname.count("bert.embeddings.word_embeddings.weight")) load_upstream(m.up, t);
    KK_HIP(hipDeviceSynchronize());
    m.ready = true;
}

// ------------------------------------------------------------------ plans
static void stage_begin(kk_ctx* ctx) {
    Staging& s = ctx->stage;
    if (s.pending) {
        KK_HIP(hipEventSynchronize(s.done));  // the previous plan's copy has left the buffer
        s.pending = false;
    }
    s.used = 0;
    s.refs.clear();
}

// Reserves `count` elements for `b` in the staging buffer and returns where to write them (valid
// until the next stage call, which may move the buffer).
template <class T>
static T* stage(kk_ctx* ctx, DevBuf& b, size_t count) {
    Staging& s = ctx->stage;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 16);
    const size_t off = (s.used + 255) / 256 * 256;
    if (off + bytes > s.cap) {
        const size_t ncap = std::max<size_t>(off + bytes + (off + bytes) / 2, (size_t)4 << 20);
        if (s.pageable) {
            s.heap.resize(ncap);
            s.host = s.heap.data();
        } else {
            void* nh = nullptr;
            KK_HIP(hipHostMalloc(&nh, ncap, hipHostMallocDefault));
            if (s.used) std::memcpy(nh, s.host, s.used);
            if (s.host) (void)hipHostFree(s.host);
            s.host = (char*)nh;
        }
        s.cap = ncap;
    }
    s.used = off + bytes;
    s.refs.push_back(Staging::Ref{&b, off, bytes});
    return (T*)(s.host + off);
}
template <class T>
static void stage_copy(kk_ctx* ctx, DevBuf& b, const T* h, size_t count) {
    T* d = stage<T>(ctx, b, count);
    if (count) std::memcpy(d, h, count * sizeof(T));
}
template <class T>
static void stage_vec(kk_ctx* ctx, DevBuf& b, const std::vector<T>& v) {
    stage_copy(ctx, b, v.data(), v.size());
}
// Everything staged since stage_begin goes to the device in one copy into `table` (grow-only), on
// stream st; the staged buffers become views of it.
static void stage_flush(kk_ctx* ctx, DevBuf& table, hipStream_t st) {
    Staging& s = ctx->stage;
    table.alloc(s.used);
    if (s.used) KK_HIP(hipMemcpyAsync(table.p, s.host, s.used, hipMemcpyHostToDevice, st));
    KK_HIP(hipEventRecord(s.done, st));
    s.pending = true;
    for (const auto& r : s.refs) r.buf->view((char*)table.p + r.off, r.bytes);
    s.refs.clear();
}

struct Dom {
    int64_t l = 0;
    std::vector<int64_t> start, len;
    DevBuf col_d, start_d, len_d;
    // every item's span widened to the whole domain: what the convolutions read as an item's rows
    // when gap masking is switched off (the negative-control hook)
    DevBuf wstart_d, wlen_d;
    int64_t valid() const {
        int64_t s = 0;
        for (auto v : len) s += v;
        return s;
    }
    // Dom::new (src/gpu_batch.rs:42-54), through kk_layout_col_item: col_item per column (-1 in
    // gaps, built only for the domains a kernel masks with it), overflow and overlap are errors.
    void build(kk_ctx* ctx, int64_t l_, std::vector<int64_t> st, std::vector<int64_t> ln, bool with_col, bool whole) {
        l = l_, start = std::move(st), len = std::move(ln);
        const int n = (int)start.size();
        for (int b = 0; b < n; b++) check(start[b] >= 0 && len[b] >= 0 && start[b] + len[b] <= l, "layout overflow");
        stage_vec(ctx, start_d, start);
        stage_vec(ctx, len_d, len);
        if (with_col) {
            int32_t* col = stage<int32_t>(ctx, col_d, (size_t)l);
            check(kk_layout_col_item(l, start.data(), len.data(), n, col) == KK_OK, "overlapping item spans");
        } else {
            col_d.release();
        }
        if (whole) {
            int64_t* ws = stage<int64_t>(ctx, wstart_d, n);
            for (int b = 0; b < n; b++) ws[b] = 0;
            int64_t* wl = stage<int64_t>(ctx, wlen_d, n);
            for (int b = 0; b < n; b++) wl[b] = l;
        } else {
            wstart_d.release(), wlen_d.release();
        }
    }
    void release() {
        for (DevBuf* b : {&col_d, &start_d, &len_d, &wstart_d, &wlen_d}) b->release();
    }
};

// Item-aligned GEMM-column tiles of a domain (see TilesDev in kk_kernels.h).
struct Tiles {
    DevBuf item, t0, n, lo, hi;
    std::vector<int32_t> lo_h, hi_h;  // per item: its tiles are [lo_h, hi_h)
    int64_t count = 0;
    int64_t max_tiles = 0;  // the most tiles of any item
    int width = 0;
    TilesDev dev() const {
        return TilesDev{item.as<int32_t>(), t0.as<int64_t>(), n.as<int32_t>(), lo.as<int32_t>(), hi.as<int32_t>(),
                        count};
    }
    // tiles of width `w` over [start_b, start_b + len_b + extra) for every item (extra = 1: the
    // ConvT GEMM column one past the item's last input)
    void build(kk_ctx* ctx, const Dom& d, int w, int extra) {
        const int nb = (int)d.start.size();
        std::vector<int32_t> it, nn, lo_(nb), hi_(nb);
        std::vector<int64_t> t;
        max_tiles = 0;
        for (int b = 0; b < nb; b++) {
            lo_[b] = (int32_t)it.size();
            const int64_t len = d.len[b] + extra;
            for (int64_t j = 0; j < len; j += w) {
                it.push_back((int32_t)b);
                t.push_back(d.start[b] + j);
                nn.push_back((int32_t)std::min<int64_t>(w, len - j));
            }
            hi_[b] = (int32_t)it.size();
            max_tiles = std::max<int64_t>(max_tiles, hi_[b] - lo_[b]);
        }
        count = (int64_t)it.size(), width = w;
        stage_vec(ctx, item, it), stage_vec(ctx, t0, t), stage_vec(ctx, n, nn);
        stage_vec(ctx, lo, lo_), stage_vec(ctx, hi, hi_);
        lo_h = std::move(lo_), hi_h = std::move(hi_);
    }
};

enum PlanKind { PLAN_DECODER = 0, PLAN_GENERATOR = 1, PLAN_SNAKE = 2, PLAN_FULL = 3 };

}  // namespace kk

struct kk_plan {
    kk_ctx* ctx = nullptr;
    int kind = 0;
    int nb = 0;
    std::vector<int64_t> nfr;  // N_b
    std::vector<int64_t> a;    // frame layout starts
    int64_t ln = 0;
    kk::Dom dn, d2, d20, d120, ds;
    // test hooks read at plan creation (see apply_test_hooks)
    bool nomask = false, poison = false, tap_source = false;
    // the recurrences on the one-CU kernel: set once a two-CU pair of this plan gave up (the plan's
    // later runs stay there), reset for each new batch
    bool lstm_single = false;
    // snake plans
    const kk::MSnake* sblk = nullptr;
    int sc = 0;
    // every staged table and input of the plan, one device buffer (see Staging)
    kk::DevBuf tables;
    // inputs
    kk::DevBuf t_en, src_row, f0, en, style, seeds, kinds, rand_ini, fixed_noise;
    int64_t t_rows = 0;
    // intermediates
    kk::DevBuf gb, xcat, xin_a, xin_b, hdec, pool, sc_half, dec_out, pp, spec, B[6], post, audio, audio_start;
    kk::DevBuf har;  // the harmonic source's samples [600 ln] (only with KOKORO_HIP_TEST_TAP_SOURCE)
    kk::DevBuf xs[2], hn;  // the noise branches' fp16 streams (d20 x 256, d120 x 128) and their fp16 h
    // coef[0..1]: the Snake steps' AdaIN pair; [2..4]: the resblocks' first AdaIN; [5..8]: the pair
    // of resblock chains 0 and 1 (run on the context's side streams); [9..10]: the noise branches'
    kk::DevBuf part, coef[11];
    int64_t part_bytes = 0;
    std::map<std::tuple<const kk::Dom*, int, int>, std::unique_ptr<kk::Tiles>> tiles;
    // item-aligned tiles of domain d, width w (built on first use: by the dry run at plan creation)
    const kk::Tiles& tl(const kk::Dom& d, int w, int extra = 0) {
        auto key = std::make_tuple(&d, w, extra);
        auto it = tiles.find(key);
        if (it == tiles.end()) {
            kk::check(!frozen, "internal: tile list requested after plan creation");
            auto t = std::make_unique<kk::Tiles>();
            t->build(ctx, d, w, extra);
            it = tiles.emplace(key, std::move(t)).first;
        }
        return *it->second;
    }
    // the quad recurrences' schedule over the items of domain d (built on first use, like the tiles)
    std::map<const kk::Dom*, kk::DevBuf> lstm_sched;
    const int32_t* lstm_sched_of(const kk::Dom& d) {
        auto it = lstm_sched.find(&d);
        if (it == lstm_sched.end()) {
            kk::check(!frozen, "internal: recurrence schedule requested after plan creation");
            kk::stage_vec(ctx, lstm_sched[&d], kk::lstm_schedule(d.len.data(), (int)d.len.size()));
            it = lstm_sched.find(&d);
        }
        return it->second.as<int32_t>();
    }
    bool frozen = false;  // tables uploaded: no more staging
    kk::DevBuf src_item, src_f0, ist_item, ist_s0;
    // ids-level plans (PLAN_FULL): the stages before the decoder.  dt: the token rows by item (the
    // text encoder's convolutions, the attention, the recurrences); dtf: every token row as one span
    // (the linear layers: a row's output depends on that row only, so gap rows may be computed and
    // are never read)
    kk::Dom dt, dtf;
    std::vector<int64_t> tstart, ntok;          // token layout
    std::vector<std::vector<int64_t>> pred;     // predicted durations per item
    kk::DevBuf tables_tok;                      // the token phase's staged tables
    kk::DevBuf ids, row_item, att_item, att_head, att_q0, style_pro, gbp;
    kk::DevBuf u_emb, u_h, u_qkv, u_ctx, u_ffn, u_x, u_gx, u_xl, u_logits, u_te, u_te2, u_gxt, u_gxs, u_sh;
    kk::DevBuf u_fx[2], u_fpool[2], u_fh[2], u_fsc[2], u_fy[2];  // the F0 and N stacks
    // the two-CU recurrences' exchange words: word 0 the run's abort flag, then one region per
    // stream that runs recurrences (the main stream, and side stream 0 for the text encoder)
    kk::DevBuf u_lstmx;
    static constexpr int64_t kLstmXHead = 64;
    int64_t n_att = 0;
    float* logits_host = nullptr;  // pinned, grow-only (the duration logits come back through it)
    size_t logits_cap = 0;
    uint64_t* abort_host = nullptr;  // pinned: the recurrences' abort flag comes back through it
    hipEvent_t te_ev[2] = {nullptr, nullptr};  // fork / join of the text encoder and of the N stack
    kk::DevBuf pcm, pcm_len, pcm_clip;  // PCM_16 output: samples [600 ln], samples per item, clip counts
    int64_t n_src = 0, n_ist = 0;
    int64_t dev_bytes = 0;
    double conv_flop = 0, snake_flop = 0;
    int64_t launches = 0;
    int last_until = -1;  // the last run's stage (-1: none)
    // kk_plan_fetch_pcm16_async: recorded after its copies; pending until kk_plan_fetch_wait
    hipEvent_t fetch_ev = nullptr;
    bool fetch_pending = false;
    int16_t* fetch_dst = nullptr;  // the pending fetch's destinations (a fallback run fetches again)
    int64_t* fetch_clipped = nullptr;
    void drop_events() {
        if (fetch_ev) (void)hipEventDestroy(fetch_ev);
        fetch_ev = nullptr, fetch_pending = false;
        for (auto& e : chain_ev)
            if (e) (void)hipEventDestroy(e), e = nullptr;
        for (auto& e : noise_ev)
            if (e) (void)hipEventDestroy(e), e = nullptr;
        for (auto& e : out_ev)
            if (e) (void)hipEventDestroy(e), e = nullptr;
        for (auto& e : te_ev)
            if (e) (void)hipEventDestroy(e), e = nullptr;
        if (logits_host) (void)hipHostFree(logits_host);
        logits_host = nullptr, logits_cap = 0;
        if (abort_host) (void)hipHostFree(abort_host);
        abort_host = nullptr;
    }
    // fork / join of the resblock chains, and of the noise branches (created with the plan)
    hipEvent_t chain_ev[3] = {nullptr, nullptr, nullptr};
    hipEvent_t noise_ev[3] = {nullptr, nullptr, nullptr};
    // the one-shot entries' audio: the run copies each item group's samples into early_out (a
    // pinned block) on side stream 0 as soon as the group's iSTFT is done; out_ev[g] after the
    // group's iSTFT, out_ev[kOutGroups] after the last copy
    static constexpr int kOutGroups = 4;
    hipEvent_t out_ev[kOutGroups + 1] = {nullptr, nullptr, nullptr, nullptr, nullptr};
    float* early_out = nullptr;
    bool early_issued = false;
    // the one-shot decoder entry stages t_en during its run, after the harmonic source and the noise
    // branch are launched (late_items: the call's items until then; tables_late: its upload)
    const kk_decoder_item* late_items = nullptr;
    std::vector<int64_t> late_tstart;
    kk::DevBuf tables_late;
    std::vector<int64_t> ist_first;  // per item: its first iSTFT block (and the total at nb)
    std::vector<kk::DevBuf*> owned() {
        return {&tables, &t_en, &src_row, &f0, &en, &style, &seeds, &kinds, &rand_ini, &fixed_noise, &gb, &xcat,
                &xin_a, &xin_b, &hdec, &pool, &sc_half, &dec_out, &pp, &spec, &B[0], &B[1], &B[2], &B[3], &B[4], &B[5],
                &post, &audio, &audio_start, &part, &coef[0], &coef[1], &coef[2], &coef[3], &coef[4], &coef[5],
                &coef[6], &coef[7], &coef[8], &coef[9], &coef[10], &xs[0], &xs[1], &hn, &src_item, &src_f0,
                &ist_item, &ist_s0, &pcm, &pcm_len, &pcm_clip, &tables_tok, &ids, &row_item, &att_item,
                &att_head, &att_q0, &style_pro, &gbp, &u_emb, &u_h, &u_qkv, &u_ctx, &u_ffn, &u_x, &u_gx, &u_xl,
                &u_logits, &u_te, &u_te2, &u_gxt, &u_gxs, &u_sh, &u_fx[0], &u_fx[1], &u_fpool[0], &u_fpool[1],
                &u_fh[0], &u_fh[1], &u_fsc[0], &u_fsc[1], &u_fy[0], &u_fy[1], &u_lstmx, &tables_late};
    }
};

namespace kk {

constexpr int64_t kXcatLd = 576, kXinLd = 1152, kSpecLd = 32, kPostLd = 32;

// A plan buffer.  Every element a run reads was written earlier in the same run (convolutions and
// statistics read only the rows of their tiles' items, the masks of the reference are row-range
// tests), so reused memory is not cleared; new memory is zeroed once.  With the poison hook every
// buffer is filled with 0xff bytes (NaN in f32, fp16 and bf16) at every plan creation instead.
static void alloc_buf(kk_plan* p, DevBuf& b, size_t bytes) {
    const bool fresh = b.alloc((bytes + 255) / 256 * 256);
    if (p->poison)
        KK_HIP(launch_fill(b.p, (int64_t)b.bytes, 0xffffffffu, p->ctx->stream));
    else if (fresh)
        KK_HIP(launch_zero(b.p, (int64_t)b.bytes, p->ctx->stream));
}

static int64_t env_i64(const char* name, int64_t dflt) {
    const char* v = std::getenv(name);
    return v && *v ? std::strtoll(v, nullptr, 10) : dflt;
}

// Test hooks, read from the environment at plan creation:
// - KOKORO_BATCH_NEGCTL_NOMASK (any value): the convolutions read every item's neighbours and gaps
//   as if they were the item's own rows -- the reference's negative-control hook that turns gap
//   masking off (src/gpu_batch.rs:62-66), so that tests can show they detect leakage;
// - KOKORO_HIP_TEST_OOM_ABOVE=k: a batch of more than k items fails with KK_ERR_OOM before any
//   allocation, as a device allocation failure would (the Err that Engine::synth_batch splits on,
//   src/engine.rs:229-234);
// - KOKORO_HIP_TEST_POISON=1: plan buffers are filled with NaN bytes instead of reused or zeroed;
// - KOKORO_HIP_TEST_TAP_SOURCE=1: the harmonic source kernel also stores the samples it transforms
//   (tap "har"), so that a test can run a CPU STFT and generator on exactly the device's source.
static void apply_test_hooks(kk_plan* p, int n) {
    const int64_t lim = env_i64("KOKORO_HIP_TEST_OOM_ABOVE", -1);
    if (lim >= 0 && n > lim)
        fail(KK_ERR_OOM, "batch of " + std::to_string(n) + " items refused by KOKORO_HIP_TEST_OOM_ABOVE=" +
                             std::to_string(lim) + " (simulated device allocation failure)");
    p->nomask = std::getenv("KOKORO_BATCH_NEGCTL_NOMASK") != nullptr;
    p->poison = env_i64("KOKORO_HIP_TEST_POISON", 0) != 0;
    p->tap_source = env_i64("KOKORO_HIP_TEST_TAP_SOURCE", 0) != 0;
}

// Resets a plan's host state for a new batch (a fresh plan, or the one-shot plan being reused).
static void reset_plan(kk_plan* p, int kind, int n) {
    p->kind = kind, p->nb = n;
    p->nfr.clear(), p->a.clear();
    p->tstart.clear(), p->ntok.clear(), p->pred.clear(), p->n_att = 0;
    p->tiles.clear(), p->lstm_sched.clear();  // views of the previous batch's staged tables
    p->frozen = false;
    p->sblk = nullptr, p->sc = 0;
    p->ln = 0, p->t_rows = 0, p->n_src = p->n_ist = 0;
    p->conv_flop = p->snake_flop = 0, p->launches = 0, p->last_until = -1;
    p->fetch_pending = false;
    p->lstm_single = false;
    apply_test_hooks(p, n);
}

// Layout shared by decoder and generator plans (src/gpu_batch.rs:250-263), through kk_layout_frames.
static void build_frame_layout(kk_plan* p) {
    kk_ctx* ctx = p->ctx;
    p->a.resize(p->nb);
    p->ln = kk_layout_frames(p->nfr.data(), p->nb, p->a.data());
    check(p->ln >= 0, "frame layout: negative frame count");
    auto scale = [&](int64_t f) {
        std::vector<int64_t> v(p->nb);
        for (int b = 0; b < p->nb; b++) v[b] = p->a[b] * f;
        return v;
    };
    auto lens = [&](int64_t f, int64_t add) {
        std::vector<int64_t> v(p->nb);
        for (int b = 0; b < p->nb; b++) v[b] = p->nfr[b] * f + add;
        return v;
    };
    const int64_t ln = p->ln;
    const bool w = p->nomask;
    p->dn.build(ctx, ln, scale(1), lens(1, 0), true, w);
    p->d2.build(ctx, 2 * ln, scale(2), lens(2, 0), true, w);
    p->d20.build(ctx, 20 * ln, scale(20), lens(20, 0), false, w);
    p->d120.build(ctx, 120 * ln + 1, scale(120), lens(120, 1), false, w);
}

struct NoiseIn {
    int32_t kind;
    uint64_t seed;
    const float* rand_ini;
    const float* sine;
    int64_t sine_len;
};

// Generator inputs: F0 at d2, styles, noise (src/gpu_batch.rs:319-341) and all generator buffers.
static void setup_generator(kk_plan* p, const std::vector<const float*>& f0s, const std::vector<const float*>& ref_s,
                            const std::vector<NoiseIn>& noise) {
    kk_ctx* ctx = p->ctx;
    const int nb = p->nb;
    const int64_t ln = p->ln, l2 = 2 * ln, l20 = 20 * ln, l120 = 120 * ln + 1;
    if (f0s.empty()) {
        // ids-level plans compute F0 on the device (F0_proj writes every row, 0 in the gaps)
        alloc_buf(p, p->f0, (size_t)l2 * sizeof(float));
    } else {
        // F0 in the d2 layout, 0 in the gaps (F0_conv reads one gap sample at each item edge)
        float* f0h = stage<float>(ctx, p->f0, (size_t)l2);
        std::memset(f0h, 0, sizeof(float) * l2);
        for (int b = 0; b < nb; b++) std::memcpy(&f0h[2 * p->a[b]], f0s[b], sizeof(float) * 2 * p->nfr[b]);
    }
    {
        float* st = stage<float>(ctx, p->style, (size_t)nb * kStyleDim);
        for (int b = 0; b < nb; b++) std::memcpy(&st[(size_t)b * kStyleDim], ref_s[b], sizeof(float) * kStyleDim);
    }
    std::vector<uint64_t> seeds(nb);
    std::vector<int32_t> kinds(nb);
    std::vector<float> ri((size_t)nb * kHarmonics);
    bool any_fixed = false;
    for (int b = 0; b < nb; b++) {
        seeds[b] = noise[b].seed;
        kinds[b] = noise[b].kind;
        if (noise[b].kind == KK_NOISE_COUNTER) {
            // RngNoise::rand_ini (src/vocoder.rs:34-40)
            for (int h = 0; h < kHarmonics; h++)
                ri[(size_t)b * kHarmonics + h] =
                    (float)(splitmix_at(noise[b].seed, (uint64_t)h) >> 40) * (1.0f / 16777216.0f);
        } else {
            any_fixed = true;
            std::memcpy(&ri[(size_t)b * kHarmonics], noise[b].rand_ini, sizeof(float) * kHarmonics);
        }
    }
    stage_vec(ctx, p->seeds, seeds);
    stage_vec(ctx, p->kinds, kinds);
    stage_vec(ctx, p->rand_ini, ri);
    if (any_fixed) {
        // caller-provided noise (rare, and 216 B per sample): its own buffer and copy
        std::vector<float> fx((size_t)600 * ln * kHarmonics, 0.f);
        for (int b = 0; b < nb; b++)
            if (noise[b].kind == KK_NOISE_FIXED)
                std::memcpy(&fx[(size_t)600 * p->a[b] * kHarmonics], noise[b].sine,
                            sizeof(float) * 600 * p->nfr[b] * kHarmonics);
        p->fixed_noise.upload(fx);
    } else {
        p->fixed_noise.release();
    }
    // work lists of the one-launch source+STFT and iSTFT kernels
    std::vector<int64_t> si, sf, ii, is;
    p->ist_first.assign(nb + 1, 0);
    for (int b = 0; b < nb; b++) {
        const int64_t frames = 120 * p->nfr[b] + 1, samples = 600 * p->nfr[b];
        for (int64_t f = 0; f < frames; f += kSourceFrames) si.push_back(b), sf.push_back(f);
        p->ist_first[b] = (int64_t)ii.size();
        for (int64_t q = 0; q < samples; q += kIstftSamples) ii.push_back(b), is.push_back(q);
    }
    p->ist_first[nb] = (int64_t)ii.size();
    p->n_src = (int64_t)si.size(), p->n_ist = (int64_t)ii.size();
    stage_vec(ctx, p->src_item, si), stage_vec(ctx, p->src_f0, sf);
    stage_vec(ctx, p->ist_item, ii), stage_vec(ctx, p->ist_s0, is);
    std::vector<int64_t> as(nb), ns(nb);
    for (int b = 0; b < nb; b++) as[b] = 600 * p->a[b], ns[b] = 600 * p->nfr[b];
    stage_vec(ctx, p->audio_start, as);
    stage_vec(ctx, p->pcm_len, ns);
    // the PCM_16 layout's gap samples are 0 (kk_plan_fetch_pcm16_async copies the whole layout)
    p->pcm.alloc((size_t)600 * ln * sizeof(int16_t));
    KK_HIP(launch_zero(p->pcm.p, (int64_t)p->pcm.bytes, ctx->stream));
    alloc_buf(p, p->pcm_clip, (size_t)nb * sizeof(unsigned long long));

    alloc_buf(p, p->gb, (size_t)nb * ctx->model.style_rows * sizeof(float));
    alloc_buf(p, p->pp, (size_t)kHarmonics * l2 * sizeof(float));
    alloc_buf(p, p->spec, (size_t)l120 * kSpecLd * sizeof(float));
    const size_t big = (size_t)std::max(l20 * 256, l120 * 128) * sizeof(float);
    for (int i = 0; i < 6; i++) alloc_buf(p, p->B[i], big);
    alloc_buf(p, p->post, (size_t)l120 * kPostLd * sizeof(float));
    alloc_buf(p, p->audio, (size_t)600 * ln * sizeof(float));
    if (p->tap_source) alloc_buf(p, p->har, (size_t)600 * ln * sizeof(float));
    for (int i = 0; i < 11; i++) alloc_buf(p, p->coef[i], (size_t)nb * kXinLd * sizeof(Coef));
    alloc_buf(p, p->xs[0], (size_t)l20 * 256 * sizeof(uint16_t));
    alloc_buf(p, p->xs[1], (size_t)l120 * 128 * sizeof(uint16_t));
    alloc_buf(p, p->hn, (size_t)std::max(l20 * 256, l120 * 128) * sizeof(uint16_t));
    // statistics partials: every partial but the last two of each item covers at least 64 columns
    // of one item (the noise convs' 64-column tiles; the convs' 128-column wave spans)
    auto bound = [&](int64_t l, int64_t c) { return (l / 64 + 2 * (int64_t)nb + 2) * c; };
    // the ConvTs' partials: per 128-column input tile, phase and output channel
    auto bound_t = [&](int64_t l_in, int64_t stride, int64_t c) { return (l_in / 128 + 2 * (int64_t)nb + 1) * stride * c; };
    const int64_t np = std::max({bound(ln, 1152), bound(2 * ln, 512), bound(l20, 256), bound(l120, 128),
                                 bound_t(l2, 10, 256), bound_t(l20, 6, 128)});
    // four regions: one per concurrent resblock chain and one for the noise branches; part_bytes
    // is one region
    alloc_buf(p, p->part, (size_t)4 * np * sizeof(StatPart));
    p->part_bytes = (int64_t)np * (int64_t)sizeof(StatPart);
}

struct Runner;
static void prebuild_tiles(kk_plan* p);

// Completes a plan: the dry run builds every tile list and validates every launch, the staged
// tables go to the device in one copy, the fork / join events are made.  The copy is ordered before
// any run on the context's stream; kk_plan_create waits for it besides.
static void finish_plan(kk_plan* p) {
    prebuild_tiles(p);
    stage_flush(p->ctx, p->tables, p->ctx->stream);
    p->frozen = true;
    for (auto& e : p->chain_ev)
        if (!e) KK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    for (auto& e : p->noise_ev)
        if (!e) KK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    for (auto& e : p->out_ev)
        if (!e) KK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    p->dev_bytes = 0;
    for (DevBuf* b : p->owned()) p->dev_bytes += (int64_t)b->cap;
}

static void check_noise(const NoiseIn& nz, int64_t n_frames, int b) {
    const std::string sb = std::to_string(b);
    check(nz.kind == KK_NOISE_COUNTER || nz.kind == KK_NOISE_FIXED, "item " + sb + ": unknown noise kind");
    if (nz.kind == KK_NOISE_FIXED) {
        check(nz.rand_ini && nz.sine, "item " + sb + ": fixed noise needs rand_ini and sine");
        // src/gpu_batch.rs:338: fixed noise size mismatch is an error
        check(nz.sine_len == 600 * n_frames * kHarmonics, "fixed noise size mismatch for item " + sb);
    }
}

// KOKORO_HIP_TIMING=1: host-side times between the marks of one call on stderr (diagnostics).
struct PhaseMarks {
    bool on = env_i64("KOKORO_HIP_TIMING", 0) != 0;
    std::chrono::steady_clock::time_point t = std::chrono::steady_clock::now();
    std::string line;
    void mark(const char* what) {
        if (!on) return;
        const auto now = std::chrono::steady_clock::now();
        char buf[96];
        std::snprintf(buf, sizeof buf, " %s %.3f ms,", what, std::chrono::duration<double, std::milli>(now - t).count());
        line += buf;
        t = now;
    }
    void print(const char* who) {
        if (on) std::fprintf(stderr, "%s:%s\n", who, line.c_str());
    }
};

// Fills plan p (new, or the one-shot plan whose device buffers are reused) for a decoder batch.
// t_en in the token layout, time-major [rows][512] (the items hand it over channel-major).
static void stage_t_en(kk_ctx* ctx, kk_plan* p, const kk_decoder_item* items, const std::vector<int64_t>& tstart) {
    float* te = stage<float>(ctx, p->t_en, (size_t)512 * p->t_rows);
    for (int b = 0; b < p->nb; b++) {
        const int nt = items[b].n_tok;
        float* dst = te + (size_t)tstart[b] * 512;
        for (int i = 0; i < nt; i++)
            for (int c = 0; c < 512; c++) dst[(size_t)i * 512 + c] = items[b].t_en[(size_t)c * nt + i];
        std::memset(dst + (size_t)nt * 512, 0, sizeof(float) * 512 * kGapT);
    }
}

// late_ten: t_en is staged by the run itself (stage_late_ten), after its first launches.
static void init_decoder_plan(kk_plan* p, const kk_decoder_item* items, int n, bool late_ten = false) {
    kk_ctx* ctx = p->ctx;
    check(ctx->model.ready, "no model uploaded");
    check(items != nullptr && n > 0, "empty batch");
    PhaseMarks pm;
    reset_plan(p, PLAN_DECODER, n);
    std::vector<int64_t> tstart(n);
    std::vector<const int64_t*> durs(n);
    std::vector<int32_t> ntok(n);
    int64_t rows = 0;
    for (int b = 0; b < n; b++) {
        const kk_decoder_item& it = items[b];
        const std::string sb = std::to_string(b);
        check(it.dur && it.t_en && it.f0 && it.energy && it.ref_s, "item " + sb + ": null input");
        check(it.n_tok >= 1, "item " + sb + ": no tokens");
        int64_t nf = 0;
        for (int i = 0; i < it.n_tok; i++) {  // the message is built only for a failing duration
            if (it.dur[i] < 1) check(false, "item " + sb + ": durations must be >= 1");
            nf += it.dur[i];
        }
        check(nf <= (int64_t)1 << 22, "item " + sb + ": too many frames");
        check_noise(NoiseIn{it.noise_kind, it.seed, it.rand_ini, it.sine, it.sine_len}, nf, b);
        p->nfr.push_back(nf);
        tstart[b] = rows;  // token layout (src/gpu_batch.rs:188-197)
        rows += it.n_tok + kGapT;
        durs[b] = it.dur, ntok[b] = it.n_tok;
    }
    pm.mark("checks");
    stage_begin(ctx);
    build_frame_layout(p);
    const int64_t ln = p->ln;
    pm.mark("layout");
    // t_en in the token layout, time-major [rows][512] (the items hand it over channel-major)
    p->t_rows = rows;
    p->late_items = nullptr;
    if (late_ten) {
        p->late_items = items, p->late_tstart = tstart;
    } else {
        stage_t_en(ctx, p, items, tstart);
    }
    pm.mark("t_en");
    // frame -> token row table (src/gpu_batch.rs:265-276), through kk_layout_src_row
    {
        int32_t* sr = stage<int32_t>(ctx, p->src_row, (size_t)ln);
        check(kk_layout_src_row(durs.data(), ntok.data(), n, tstart.data(), p->a.data(), ln, sr) == KK_OK,
              "duration expansion overflows the frame layout");
    }
    {
        float* eh = stage<float>(ctx, p->en, (size_t)2 * ln);
        std::memset(eh, 0, sizeof(float) * 2 * ln);
        for (int b = 0; b < n; b++) std::memcpy(&eh[2 * p->a[b]], items[b].energy, sizeof(float) * 2 * p->nfr[b]);
    }
    std::vector<const float*> f0s(n), refs(n);
    std::vector<NoiseIn> nz(n);
    for (int b = 0; b < n; b++) {
        f0s[b] = items[b].f0, refs[b] = items[b].ref_s;
        nz[b] = NoiseIn{items[b].noise_kind, items[b].seed, items[b].rand_ini, items[b].sine, items[b].sine_len};
    }
    pm.mark("src_row, energy");
    setup_generator(p, f0s, refs, nz);
    pm.mark("generator setup");
    alloc_buf(p, p->xcat, (size_t)ln * kXcatLd * sizeof(float));
    alloc_buf(p, p->xin_a, (size_t)ln * kXinLd * sizeof(float));
    alloc_buf(p, p->xin_b, (size_t)ln * kXinLd * sizeof(float));
    alloc_buf(p, p->hdec, (size_t)ln * 1024 * sizeof(float));
    alloc_buf(p, p->pool, (size_t)2 * ln * kXinLd * sizeof(uint16_t));
    alloc_buf(p, p->sc_half, (size_t)ln * 512 * sizeof(float));
    alloc_buf(p, p->dec_out, (size_t)2 * ln * 512 * sizeof(float));
    pm.mark("buffers");
    finish_plan(p);
    pm.mark("tiles, dry run, upload");
    pm.print("init_decoder_plan");
}

// A user plan is complete (its inputs on the device) when kk_plan_create returns.
static kk_plan* register_plan(kk_ctx* ctx, std::unique_ptr<kk_plan> p) {
    KK_HIP(hipStreamSynchronize(ctx->stream));
    ctx->plans.insert(p.get());
    return p.release();
}

static kk_plan* create_decoder_plan(kk_ctx* ctx, const kk_decoder_item* items, int n) {
    auto p = std::make_unique<kk_plan>();
    p->ctx = ctx;
    init_decoder_plan(p.get(), items, n);
    return register_plan(ctx, std::move(p));
}

static kk_plan* create_generator_plan(kk_ctx* ctx, const kk_generator_item* items, int n) {
    check(ctx->model.ready, "no model uploaded");
    check(items != nullptr && n > 0, "empty batch");
    auto p = std::make_unique<kk_plan>();
    p->ctx = ctx;
    reset_plan(p.get(), PLAN_GENERATOR, n);
    for (int b = 0; b < n; b++) {
        const std::string sb = std::to_string(b);
        check(items[b].x && items[b].f0 && items[b].ref_s, "item " + sb + ": null input");
        check(items[b].n_frames >= 1 && items[b].n_frames <= (1 << 22), "item " + sb + ": frames out of range");
        check_noise(NoiseIn{items[b].noise_kind, items[b].seed, items[b].rand_ini, items[b].sine, items[b].sine_len},
                    items[b].n_frames, b);
        p->nfr.push_back(items[b].n_frames);
    }
    stage_begin(ctx);
    build_frame_layout(p.get());
    std::vector<const float*> f0s(n), refs(n);
    std::vector<NoiseIn> nz(n);
    for (int b = 0; b < n; b++) {
        f0s[b] = items[b].f0, refs[b] = items[b].ref_s;
        nz[b] = NoiseIn{items[b].noise_kind, items[b].seed, items[b].rand_ini, items[b].sine, items[b].sine_len};
    }
    setup_generator(p.get(), f0s, refs, nz);
    // decoder output x [512][2N] per item -> time-major d2 rows, 0 in the gaps
    const int64_t l2 = 2 * p->ln;
    float* xh = stage<float>(ctx, p->dec_out, (size_t)l2 * 512);
    std::memset(xh, 0, sizeof(float) * l2 * 512);
    for (int b = 0; b < n; b++) {
        const int64_t t2 = 2 * p->nfr[b];
        for (int c = 0; c < 512; c++)
            for (int64_t t = 0; t < t2; t++) xh[(size_t)(2 * p->a[b] + t) * 512 + c] = items[b].x[(size_t)c * t2 + t];
    }
    finish_plan(p.get());
    return register_plan(ctx, std::move(p));
}

static const MSnake* find_snake(const Model& m, const std::string& prefix) {
    for (int i = 0; i < 2; i++)
        if (prefix == "decoder.generator.noise_res." + std::to_string(i)) return &m.noise_res[i];
    for (int i = 0; i < 6; i++)
        if (prefix == "decoder.generator.resblocks." + std::to_string(i)) return &m.rb[i];
    return nullptr;
}

static kk_plan* create_snake_plan(kk_ctx* ctx, const char* prefix, const float* const* x, const int64_t* t,
                                  const float* const* ref_s, int n, int gap) {
    check(ctx->model.ready, "no model uploaded");
    check(prefix && x && t && ref_s && n > 0 && gap >= 0, "bad arguments");
    const MSnake* blk = find_snake(ctx->model, prefix);
    check(blk != nullptr, std::string("no Snake block named ") + prefix);
    auto p = std::make_unique<kk_plan>();
    p->ctx = ctx;
    reset_plan(p.get(), PLAN_SNAKE, n);
    p->sblk = blk, p->sc = blk->c;
    // receptive field of one dilation step: (k - 1) * 5 / 2 + (k - 1) / 2 columns
    const int k = blk->c1[0].k;
    check(gap >= (k - 1) * 5 / 2, "gap narrower than the block's conv reach");
    std::vector<int64_t> st(n), ln(n);
    int64_t l = 0;
    for (int b = 0; b < n; b++) {
        check(x[b] && ref_s[b] && t[b] >= 1, "item " + std::to_string(b) + ": bad input");
        st[b] = l, ln[b] = t[b];
        p->nfr.push_back(t[b]);
        l += t[b] + gap;
    }
    stage_begin(ctx);
    p->ds.build(ctx, l, st, ln, false, p->nomask);
    const int c = blk->c;
    {
        float* xh = stage<float>(ctx, p->B[0], (size_t)l * c);
        std::memset(xh, 0, sizeof(float) * l * c);
        for (int b = 0; b < n; b++)
            for (int ch = 0; ch < c; ch++)
                for (int64_t i = 0; i < t[b]; i++) xh[(size_t)(st[b] + i) * c + ch] = x[b][(size_t)ch * t[b] + i];
    }
    {
        float* sth = stage<float>(ctx, p->style, (size_t)n * kStyleDim);
        for (int b = 0; b < n; b++) std::memcpy(&sth[(size_t)b * kStyleDim], ref_s[b], sizeof(float) * kStyleDim);
    }
    alloc_buf(p.get(), p->gb, (size_t)n * ctx->model.style_rows * sizeof(float));
    alloc_buf(p.get(), p->B[1], (size_t)l * c * sizeof(float));
    for (int i = 0; i < 2; i++) alloc_buf(p.get(), p->coef[i], (size_t)n * c * sizeof(Coef));
    alloc_buf(p.get(), p->part, (size_t)(l / 128 + 2 * (int64_t)n + 2) * c * sizeof(StatPart));
    p->part_bytes = (int64_t)p->part.bytes;
    finish_plan(p.get());
    return register_plan(ctx, std::move(p));
}

// ------------------------------------------------------------------ the launch sequence

struct Runner {
    kk_plan* p;
    kk_ctx* ctx;
    const Model& m;
    hipStream_t s;
    bool dry = false;  // build the plan's tile lists only, launch nothing
    double flop = 0, snake_flop = 0;
    int64_t launches = 0;
    // AdaIN projections: the decoder + generator table (ref_s[0:128]) or, while pro_style is set,
    // the prosody predictor's (ref_s[128:256])
    bool pro_style = false;
    const float* gbuf() const { return pro_style ? p->gbp.as<float>() : p->gb.as<float>(); }
    int64_t gb_ld() const { return pro_style ? m.up.style_rows : m.style_rows; }
    bool skip_tokens = false;  // the token phase ran at plan creation (kk_forward_batch)
    Coef* cf(int i) const { return p->coef[i].as<Coef>(); }
    int region = 0;  // statistics partials region of the current chain
    StatPart* part() const { return p->part.as<StatPart>() + (size_t)region * (size_t)(p->part_bytes / sizeof(StatPart)); }

    hipEvent_t ev() {
        if (!ctx->event_pool.empty()) {
            hipEvent_t e = ctx->event_pool.back();
            ctx->event_pool.pop_back();
            return e;
        }
        hipEvent_t e;
        KK_HIP(hipEventCreate(&e));
        return e;
    }

    // One kernel launch (nothing in the dry run): counted and, with profiling on, bracketed by an
    // event pair on the launch stream and recorded under class `cls` with its algorithmic FLOP and
    // bytes (valid rows only: the data the step must read and write once).
    std::string label;  // the next launch's profile label (default: its class)
    template <class F>
    void launch(int cls, double f, double bytes, F&& fn) {
        launches++;
        std::string lb = label.empty() ? std::string(kProfNames[cls]) : label;
        label.clear();
        if (dry) return;
        hipEvent_t e0 = nullptr, e1 = nullptr;
        if (ctx->profiling) {
            e0 = ev(), e1 = ev();
            KK_HIP(hipEventRecord(e0, s));
        }
        KK_HIP(fn());
        if (ctx->profiling) {
            KK_HIP(hipEventRecord(e1, s));
            ctx->prof.push_back(ProfRec{cls, f, bytes, e0, e1, std::move(lb)});
        }
    }
    int64_t frames() const { return p->dn.valid(); }

    void need_part(int64_t n) {
        check(n * (int64_t)sizeof(StatPart) <= p->part_bytes, "statistics partials buffer too small");
    }

    // Standalone statistics partials of x over domain d (tiles of kStatTile rows).
    const Tiles& stats(const float* x, int64_t ld, int c, const Dom& d) {
        const Tiles& t = p->tl(d, kStatTile);
        need_part(t.count * c);
        const double bytes = (double)d.valid() * c * 4 + (double)t.count * c * sizeof(StatPart);
        launch(PC_STATS, 0, bytes, [&] { return launch_stats_tiles(x, ld, c, t.dev(), part(), s); });
        return t;
    }
    // Partials -> coefficients of AdaIN layer a (`wn` partials per tile; xrow: one more sample per
    // item, row xrow_at[b] of xrow [.][c] fp16).
    void fin(const Tiles& t, int wn, int c, const MAdain& a, Coef* coef, const uint16_t* xrow = nullptr,
             const int64_t* xrow_at = nullptr) {
        const MAdain* as[1] = {&a};
        Coef* const cs[1] = {coef};
        fin_n(t, wn, c, 1, as, cs, xrow, xrow_at);
    }
    // One finalize for the n (<= kFinMaxOuts) AdaIN layers as[k] of one tensor: its statistics once,
    // each layer's coefficients into cs[k].
    void fin_n(const Tiles& t, int wn, int c, int n, const MAdain* const* as, Coef* const* cs,
               const uint16_t* xrow = nullptr, const int64_t* xrow_at = nullptr) {
        check(n >= 1 && n <= kFinMaxOuts, "finalize outputs");
        FinOuts fo{};
        fo.n = n;
        for (int k = 0; k < n; k++) fo.o[k] = FinOut{as[k]->gb_off, as[k]->nw.as<float>(), as[k]->nb.as<float>(), cs[k]};
        const double bytes =
            (double)t.count * wn * c * sizeof(StatPart) + (double)n * p->nb * c * (sizeof(Coef) + 8);
        launch(PC_FINALIZE, 0, bytes, [&] {
            return launch_finalize(part(), c, wn, t.dev(), p->nb, t.max_tiles * wn, gbuf(), gb_ld(), fo, s, xrow, c,
                                   xrow_at);
        });
    }
    void stats_fin(const float* x, int64_t ld, int c, const Dom& d, const MAdain& a, Coef* coef) {
        fin(stats(x, ld, c, d), 1, c, a, coef);
    }

    // One MFMA conv launch.
    struct Op {
        int64_t t_lo = 0, t_hi = -1;  // a range of the output domain's tiles (t_hi < 0: all)
        int pro = PRO_F32, epi = EPI_STORE;
        const void* x = nullptr;
        int64_t x_ld = 0;
        const Dom* din = nullptr;   // input domain: rows outside the tile's item read as 0
        float* y = nullptr;
        int64_t y_ld = 0;
        const Dom* dout = nullptr;  // output domain (tiles of stride-1 convs)
        const Coef* coef = nullptr;
        const DevBuf* ar = nullptr;
        const DevBuf* ai = nullptr;
        float slope = 0.f;
        const float *r0 = nullptr, *r1 = nullptr, *r2 = nullptr;
        int64_t r0_ld = 0;
        float scale = 1.f;
        bool stats = false;
        int cls = PC_DECODER;
        std::string label;  // profile label
        bool convt = false;
        int stride = 1, pad_t = 0;
        bool in_h = false, out_h = false;  // fp16 input / output (the Snake steps' h)
    };
    const Tiles& conv(const MConv& c, const Op& o) {
        const int wn = kShapeWN[c.shape], bn = kShapeN[c.shape];
        const Tiles& t = o.convt ? p->tl(*o.din, bn, 1) : p->tl(*o.dout, bn);
        ConvParams q{};
        q.x = o.x, q.x_ld = o.x_ld, q.l_in = o.din->l, q.cin = c.cin, q.cin_pad = c.cin_pad;
        q.in_max_len = o.din->len.empty() ? 0 : *std::max_element(o.din->len.begin(), o.din->len.end());
        q.in_start = o.din->start_d.as<int64_t>(), q.in_len = o.din->len_d.as<int64_t>();
        if (p->nomask) {  // negative-control hook: every item reads the whole domain as its rows
            q.in_max_len = o.din->l;
            q.in_start = o.din->wstart_d.as<int64_t>(), q.in_len = o.din->wlen_d.as<int64_t>();
        }
        q.tiles = t.dev();
        if (o.t_hi >= 0) {  // a range of the tiles (they are in item order): a group of items
            q.tiles.item += o.t_lo, q.tiles.t0 += o.t_lo, q.tiles.n += o.t_lo;
            q.tiles.count = o.t_hi - o.t_lo;
        }
        q.coef = o.coef, q.alpha_rev = o.ar ? o.ar->as<float>() : nullptr;
        q.alpha_inv = o.ai ? o.ai->as<float>() : nullptr, q.slope = o.slope;
        q.w = c.w.as<uint16_t>(), q.bias = c.b.as<float>();
        q.m = c.m, q.m_pad = c.m_pad, q.k = c.k, q.dil = c.dil, q.pad = c.pad;
        q.y = o.y, q.y_ld = o.y_ld, q.cout = c.cout;
        q.r0 = o.r0, q.r1 = o.r1, q.r2 = o.r2, q.r0_ld = o.r0_ld, q.scale = o.scale;
        q.stride_t = o.stride, q.pad_t = o.pad_t;
        q.out_start = o.dout->start_d.as<int64_t>(), q.out_len = o.dout->len_d.as<int64_t>();
        if (o.stats) {
            need_part(t.count * wn * (o.convt ? o.stride : 1) * c.cout);  // ConvT: per phase too
            q.part = part();
        }
        // algorithmic FLOP over valid columns; ConvT (K = 2 stride): each input column feeds
        // K x cout outputs = 2 m MACs per input channel
        // (a tile range counts its share of the domain)
        const double share = o.t_hi >= 0 && t.count > 0 ? (double)(o.t_hi - o.t_lo) / (double)t.count : 1.0;
        const double valid = share * (double)(o.convt ? o.din->valid() : o.dout->valid());
        const double f = 2.0 * (double)c.cin * valid * (o.convt ? 2.0 * c.m : (double)c.cout * c.k);
        flop += f;
        if (o.cls == PC_SNAKE) snake_flop += f;
        // algorithmic bytes: the input read once, the output written once, residual operands read
        const double v_in = share * (double)o.din->valid(), v_out = share * (double)o.dout->valid();
        const double es_in = (o.in_h || o.pro == PRO_BF16) ? 2 : 4, es_out = o.out_h ? 2 : 4;
        const int nres = o.convt ? 1
                         : o.epi == EPI_MEAN3_LEAKY_BF16 ? 3
                         : (o.epi == EPI_ACCUM || o.epi == EPI_RESID || o.epi == EPI_ADD_FROM) ? 1
                                                                                                 : 0;
        // residual operands: fp16 streams for the means and wherever the output is an fp16 stream
        const double es_res =
            o.epi == EPI_MEAN3_LEAKY_BF16 || (o.out_h && (o.convt || o.epi == EPI_ACCUM || o.epi == EPI_ADD_FROM)) ? 2 : 4;
        double bytes = v_in * c.cin * es_in + v_out * c.cout * (es_out + es_res * nres);
        if (o.epi == EPI_RESID_UP2) bytes += v_out / 2 * c.cout * 4;
        // the dry run (plan creation) validates the launch parameters without launching
        if (dry) {
            if (launch_conv(q, o.pro, o.epi, c.shape, o.stats, o.in_h, o.out_h, ctx->n_cu, s, true) != hipSuccess)
                fail(KK_ERR_INVALID, "convolution parameters out of the kernel's range (batch too large?)");
        }
        label = o.label;
        launch(o.cls, f, bytes,
               [&] { return launch_conv(q, o.pro, o.epi, c.shape, o.stats, o.in_h, o.out_h, ctx->n_cu, s); });
        return t;
    }

    Op snake_op(const MSnake& blk, const Dom& d, const void* x, float* y, int epi, const Coef* coef, int i,
                bool second, bool stats) {
        Op o;
        o.pro = PRO_ADAIN_SNAKE, o.epi = epi, o.x = x, o.x_ld = blk.c, o.din = o.dout = &d, o.y = y;
        o.y_ld = blk.c, o.coef = coef, o.stats = stats, o.cls = PC_SNAKE;
        o.label = blk.name + ".d" + std::to_string(2 * i + 1) + (second ? ".conv2" : ".conv1");
        o.ar = second ? &blk.ar2[i] : &blk.ar1[i];
        o.ai = second ? &blk.ai2[i] : &blk.ai1[i];
        // conv1 writes h in fp16, conv2 reads it
        o.out_h = !second, o.in_h = second;
        return o;
    }

    // snake_b (src/gpu_batch.rs:140-154) in place on X: an f32 stream, or an fp16 one (x16: the
    // noise branches', which start from the noise conv's fp16 output).  The statistics of each
    // conv's output are reduced in its epilogue; the block input's come from the kernel that
    // produced X (`xin`: its tiles, one partial per tile and channel) or, when null, from a
    // statistics pass here (f32 streams only).
    // ca / cb: the coefficient pair of the block's two AdaIN per step (default cf(0), cf(1)).
    void snake_block(const MSnake& blk, void* X, float* h, const Dom& d, const Tiles* xin = nullptr,
                     Coef* ca = nullptr, Coef* cb = nullptr, bool x16 = false) {
        const int c = blk.c, wn = kShapeWN[blk.c1[0].shape];
        if (!ca) ca = cf(0), cb = cf(1);
        if (xin) {
            fin(*xin, 1, c, blk.a1[0], ca);
        } else {
            check(!x16, "an fp16 Snake stream needs its producer's statistics");
            stats_fin((const float*)X, c, c, d, blk.a1[0], ca);
        }
        for (int i = 0; i < 3; i++) {
            Op o1 = snake_op(blk, d, X, h, EPI_STORE, ca, i, false, true);
            o1.in_h = x16;
            const Tiles& t = conv(blk.c1[i], o1);
            fin(t, wn, c, blk.a2[i], cb);
            Op o2 = snake_op(blk, d, h, (float*)X, EPI_ACCUM, cb, i, true, i < 2);
            o2.out_h = x16;
            conv(blk.c2[i], o2);
            if (i < 2) fin(t, wn, c, blk.a1[i + 1], ca);
        }
    }

    // x = (rb0(y) + rb1(y) + rb2(y)) / 3 (src/gpu_batch.rs:395-401), stored in post_out as the next
    // layer's bf16 operand (leaky ReLU with post_slope applied; nothing else reads a stage's output);
    // post_out must not be a buffer the mean reads (X, block 2's h).
    // The stage input y and each block's running sum X[j] are fp16 streams (half the traffic of the
    // f32 streams the reference keeps; 2^-11 relative rounding per step against the 2^-8 of the
    // bf16 operands that every conv reads): conv2 of step 0 adds y into X[j], the later steps add
    // in place, conv1 reads y at step 0 and X[j] after, and the mean reads the three X.
    // yt: the tiles whose partials of y its producer (the ConvT) wrote, `yparts` per tile, with the
    // reflected first row of each item (xrow_at) outside them when y_refl.
    // hs: the fp16 h buffer of each block (distinct when the blocks run concurrently).
    void resblock_mean(const MSnake* rbs, const uint16_t* y, float* X[3], float* const hs[3], const Dom& d,
                       const Tiles& yt, int yparts, bool y_refl, void* post_out, float post_slope) {
        const int c = rbs[0].c, wn = kShapeWN[rbs[0].c1[0].shape];
        // the three blocks' first AdaIN share one set of statistics of y: one finalize for all three
        const MAdain* a1s[3] = {&rbs[0].a1[0], &rbs[1].a1[0], &rbs[2].a1[0]};
        Coef* const c1s[3] = {cf(2), cf(3), cf(4)};
        fin_n(yt, yparts, c, 3, a1s, c1s, y_refl ? y : nullptr, y_refl ? d.start_d.as<int64_t>() : nullptr);
        // The three blocks are independent until the mean: blocks 0 and 1 run on the context's
        // side streams and block 2 on the main stream, each with its own h, statistics region and
        // AdaIN coefficients, and the mean (block 2's last conv) waits for the other two.  One
        // chain's kernels fill the CUs that another's tail leaves idle.  The kernels and their
        // arithmetic are those of the serial order (kept for per-launch profiling).
        const bool conc = !ctx->profiling && !dry;
        hipStream_t main_s = s;
        if (conc) {
            KK_HIP(hipEventRecord(p->chain_ev[2], main_s));
            for (int q = 0; q < 2; q++) KK_HIP(hipStreamWaitEvent(ctx->side[q], p->chain_ev[2], 0));
        }
        // Concurrent: the longest chain (block 2, k = 11) is enqueued first and its last conv (the
        // mean) after the other two chains and the join.
        Op mean_op;
        bool mean_pending = false;
        for (int jj = 0; jj < 3; jj++) {
            const int j = conc ? 2 - jj : jj;
            const MSnake& blk = rbs[j];
            const bool side = conc && j < 2;
            s = side ? ctx->side[j] : main_s;
            region = conc ? j : 0;
            Coef* ca = side ? cf(5 + 2 * j) : cf(0);  // the steps' AdaIN pair
            Coef* cb = side ? cf(6 + 2 * j) : cf(1);
            float* h = hs[j];  // each block its own h in both orders (the mean's output may use hs[0..1])
            for (int i = 0; i < 3; i++) {
                Op o1 = snake_op(blk, d, i == 0 ? (const void*)y : X[j], h, EPI_STORE, i == 0 ? cf(2 + j) : ca, i,
                                 false, true);
                o1.in_h = true;  // y, then X[j]
                const Tiles& t = conv(blk.c1[i], o1);
                fin(t, wn, c, blk.a2[i], cb);
                Op o2 = snake_op(blk, d, h, X[j], EPI_ACCUM, cb, i, true, i < 2);
                o2.out_h = true;  // X[j] in fp16
                if (i == 0) o2.epi = EPI_ADD_FROM, o2.r0 = (const float*)y, o2.r0_ld = c;
                if (j == 2 && i == 2) {
                    o2.epi = EPI_MEAN3_LEAKY_BF16, o2.r0 = X[0], o2.r1 = X[1], o2.r2 = X[2], o2.r0_ld = c;
                    o2.slope = post_slope, o2.y = (float*)post_out;
                    if (conc) {
                        mean_op = o2, mean_pending = true;
                        continue;
                    }
                }
                conv(blk.c2[i], o2);
                if (i < 2) fin(t, wn, c, blk.a1[i + 1], ca);
            }
        }
        if (mean_pending) {
            s = main_s;
            for (int q = 0; q < 2; q++) {
                KK_HIP(hipEventRecord(p->chain_ev[q], ctx->side[q]));
                KK_HIP(hipStreamWaitEvent(main_s, p->chain_ev[q], 0));
            }
            conv(rbs[2].c2[2], mean_op);
        }
        s = main_s, region = 0;
    }

    // AdainResBlk1d (src/gpu_batch.rs:104-135) without upsampling: in [ln][in_ld] -> out[:, 0:dout].
    void resblk(const MResblk& r, const float* in, int64_t in_ld, float* out, int64_t out_ld) {
        const Dom& d = p->dn;
        float* h = p->hdec.as<float>();
        stats_fin(in, in_ld, r.din, d, r.n1, cf(0));
        Op o1;
        o1.pro = PRO_ADAIN_LEAKY, o1.x = in, o1.x_ld = in_ld, o1.din = o1.dout = &d, o1.y = h, o1.y_ld = r.dout;
        o1.coef = cf(0), o1.slope = 0.2f, o1.stats = true;
        o1.label = r.name + ".conv1";
        const Tiles& t = conv(r.conv1, o1);
        fin(t, kShapeWN[r.conv1.shape], r.dout, r.n2, cf(1));
        Op os;
        os.x = in, os.x_ld = in_ld, os.din = os.dout = &d, os.y = out, os.y_ld = out_ld;
        os.label = r.name + ".conv1x1";
        conv(r.conv1x1, os);
        Op o2;
        o2.pro = PRO_ADAIN_LEAKY, o2.epi = EPI_RESID, o2.x = h, o2.x_ld = r.dout, o2.din = o2.dout = &d;
        o2.y = out, o2.y_ld = out_ld, o2.coef = cf(1), o2.slope = 0.2f, o2.scale = 1.0f / sqrtf(2.0f);
        o2.label = r.name + ".conv2";
        conv(r.conv2, o2);
    }

    // The one-shot decoder entry's t_en: staged in the context's second staging buffer and uploaded
    // on the run's stream now, while the harmonic source and the noise branch (launched before,
    // on a side stream) already run; the decoder's launches follow it on the same stream.
    void stage_late_ten() {
        std::swap(ctx->stage, ctx->stage_late);
        struct Restore {
            kk_ctx* ctx;
            ~Restore() { std::swap(ctx->stage, ctx->stage_late); }
        } restore{ctx};
        stage_begin(ctx);
        stage_t_en(ctx, p, p->late_items, p->late_tstart);
        stage_flush(ctx, p->tables_late, s);
        p->late_items = nullptr;
    }

    void decoder() {
        const Dom& dn = p->dn;
        const Dom& d2 = p->d2;
        const int64_t ln = p->ln;
        const int32_t* col = dn.col_d.as<int32_t>();
        float* xcat = p->xcat.as<float>();
        float* xa = p->xin_a.as<float>();
        float* xb = p->xin_b.as<float>();
        // asr = t_en expanded by the durations; F0 / N convs (src/gpu_batch.rs:295-302)
        const double nf = (double)frames();
        launch(PC_EXPAND, 0, nf * 512 * 8, [&] {
            return launch_expand(p->t_en.as<float>(), p->t_rows, p->src_row.as<int32_t>(), ln, xcat, kXcatLd, s);
        });
        launch(PC_F0N, 0, nf * 24, [&] {
            return launch_f0n_conv(p->f0.as<float>(), p->en.as<float>(), 2 * ln, m.f0w.as<float>(), m.f0b.as<float>(),
                                   m.nw_.as<float>(), m.nb_.as<float>(), xcat, kXcatLd, 512, 513, col, ln, s);
        });
        resblk(m.encode, xcat, kXcatLd, xa, kXinLd);
        // asr_res (512 -> 64, k1) into channels [1024, 1088); F0n, Nn into 1088, 1089
        Op oa;
        oa.x = xcat, oa.x_ld = kXcatLd, oa.din = oa.dout = &dn, oa.y = xa + 1024, oa.y_ld = kXinLd;
        oa.label = "asr_res";
        conv(m.asr_res, oa);
        launch(PC_COPY, 0, nf * 2 * 8, [&] { return launch_copy_cols(xcat + 512, kXcatLd, 2, xa, kXinLd, 1088, col, ln, s); });
        launch(PC_COPY, 0, nf * 66 * 8, [&] { return launch_copy_cols(xa + 1024, kXinLd, 66, xb, kXinLd, 1024, col, ln, s); });
        resblk(m.decode[0], xa, kXinLd, xb, kXinLd);
        resblk(m.decode[1], xb, kXinLd, xa, kXinLd);
        resblk(m.decode[2], xa, kXinLd, xb, kXinLd);
        // decode.3: upsample block to 2N (src/gpu_batch.rs:106-133)
        const MResblk& r = m.decode[3];
        stats_fin(xb, kXinLd, r.din, dn, r.n1, cf(0));
        launch(PC_POOL, 0, nf * r.din * 4 + 2 * nf * kXinLd * 2, [&] {
            return launch_adain_pool(xb, kXinLd, r.din, cf(0), col, ln, r.pool_w.as<float>(), r.pool_b.as<float>(),
                                     d2.col_d.as<int32_t>(), p->pool.as<uint16_t>(), kXinLd, s);
        });
        float* h = p->hdec.as<float>();
        Op o1;
        o1.pro = PRO_BF16, o1.x = p->pool.p, o1.x_ld = kXinLd, o1.din = o1.dout = &d2, o1.y = h, o1.y_ld = 512;
        o1.stats = true;
        o1.label = r.name + ".conv1";
        const Tiles& t = conv(r.conv1, o1);
        fin(t, kShapeWN[r.conv1.shape], 512, r.n2, cf(1));
        // shortcut conv1x1(nearest x2 (x)) = nearest x2 (conv1x1(x)) for a 1x1 conv: computed at N
        Op os;
        os.x = xb, os.x_ld = kXinLd, os.din = os.dout = &dn, os.y = p->sc_half.as<float>(), os.y_ld = 512;
        os.label = r.name + ".conv1x1";
        conv(r.conv1x1, os);
        Op o2;
        o2.pro = PRO_ADAIN_LEAKY, o2.epi = EPI_RESID_UP2, o2.x = h, o2.x_ld = 512, o2.din = o2.dout = &d2;
        o2.y = p->dec_out.as<float>(), o2.y_ld = 512, o2.coef = cf(1), o2.slope = 0.2f;
        o2.r0 = p->sc_half.as<float>(), o2.r0_ld = 512, o2.scale = 1.0f / sqrtf(2.0f);
        o2.label = r.name + ".conv2";
        conv(r.conv2, o2);
    }

    void source() {
        const double n2 = (double)p->d2.valid(), nfr120 = (double)p->d120.valid();
        launch(PC_PHASE, 0, n2 * 4 * (1 + kHarmonics), [&] {
            return launch_phase_pre(p->f0.as<float>(), p->d2.start_d.as<int64_t>(), p->d2.len_d.as<int64_t>(), p->nb,
                                    p->rand_ini.as<float>(), p->pp.as<float>(), 2 * p->ln, s);
        });
        SourceParams q{};
        q.f0 = p->f0.as<float>(), q.start2 = p->d2.start_d.as<int64_t>(), q.len2 = p->d2.len_d.as<int64_t>();
        q.pp = p->pp.as<float>(), q.pp_ld = 2 * p->ln, q.seeds = p->seeds.as<uint64_t>();
        q.fixed_noise = p->fixed_noise.as<float>(), q.noise_kind = p->kinds.as<int32_t>();
        q.lw = m.lw.as<float>(), q.lb = m.lb;
        q.start120 = p->d120.start_d.as<int64_t>(), q.f_len = p->d120.len_d.as<int64_t>();
        q.blk_item = p->src_item.as<int64_t>(), q.blk_f0 = p->src_f0.as<int64_t>(), q.n_blocks = p->n_src;
        q.spec = p->spec.as<float>(), q.spec_ld = kSpecLd;
        q.har_tap = p->tap_source ? p->har.as<float>() : nullptr;
        // reads F0 and the phases (d2), writes 22 f32 per STFT frame
        launch(PC_SOURCE, 0, n2 * 4 * (1 + kHarmonics) + nfr120 * 88, [&] { return launch_source_stft(q, s); });
    }

    // xs_i = noise_res[i](noise_convs[i](masked spec)) (src/gpu_batch.rs:362-375) into p->xs[i],
    // with its own h, statistics region (3) and coefficient pair, so that it can run beside the
    // decoder and the previous stage.
    void noise_branch(int i) {
        const Dom& dout = i == 0 ? p->d20 : p->d120;
        const int c = m.ups[i].cout;
        uint16_t* xs = p->xs[i].as<uint16_t>();  // an fp16 stream from the noise conv on
        const int reg = region;
        region = 3;
        const MNoiseConv& nc = m.nc[i];
        const int tile_rows = i == 0 ? kNoiseTile : kNoiseTile1;
        const Tiles& tn = p->tl(dout, tile_rows);
        need_part(tn.count * c);
        // reads the spectrum's valid rows once (22 f32), writes cout fp16 per output row
        const double bytes = (double)p->d120.valid() * 88 + (double)dout.valid() * c * 2;
        launch(i == 0 ? PC_NOISE0 : PC_NOISE1, 2.0 * 22 * nc.k * c * (double)dout.valid(), bytes, [&] {
            return launch_noise_conv(p->spec.as<float>(), kSpecLd, p->d120.l, p->d120.start_d.as<int64_t>(),
                                     p->d120.len_d.as<int64_t>(), nc.wp.as<uint16_t>(), nc.b.as<float>(), nc.cout,
                                     nc.k, nc.stride, nc.pad, xs, c, tn.dev(), tile_rows, part(), s);
        });
        snake_block(m.noise_res[i], xs, p->hn.as<float>(), dout, &tn, cf(9), cf(10), true);
        region = reg;
    }

    void gen_stage(int i) {
        const Dom& din = i == 0 ? p->d2 : p->d20;
        const Dom& dout = i == 0 ? p->d20 : p->d120;
        const int c = m.ups[i].cout;
        float* B[6];
        for (int j = 0; j < 6; j++) B[j] = p->B[j].as<float>();
        // y = ups[i](leaky_0.1(x) masked) (+ per-item reflect pad on stage 1) + xs (noise branch i),
        // both fp16 streams
        Op ou;
        // ups.1 reads stage 0's output as the bf16 operand stage 0's mean stored (leaky 0.1 applied)
        ou.pro = i == 0 ? PRO_LEAKY : PRO_BF16, ou.epi = i == 0 ? EPI_CONVT : EPI_CONVT_REFLECT, ou.slope = 0.1f;
        ou.x = i == 0 ? (const void*)p->dec_out.p : (const void*)B[2], ou.x_ld = i == 0 ? 512 : 256;
        ou.din = &din, ou.dout = &dout, ou.y = B[3], ou.y_ld = c, ou.r0 = p->xs[i].as<float>(), ou.r0_ld = c;
        ou.convt = true, ou.stride = m.ups_stride[i], ou.pad_t = m.ups_pad[i], ou.cls = PC_CONVT;
        ou.out_h = true;
        ou.stats = true;  // partials of y per (tile, phase, wave column) for the resblocks' first AdaIN
        ou.label = "ups." + std::to_string(i);
        const Tiles& tu = conv(m.ups[i], ou);
        float* X[3] = {B[4], B[5], B[0]};
        // h of the three blocks: the two halves of B[2] (an fp16 [rows][c] fits in half of a buffer
        // sized for f32 [rows][128] at d120 and [rows][256] at d20) and B[1]
        float* const hs[3] = {B[2], B[2] + p->B[2].bytes / 2 / sizeof(float), B[1]};
        // the stage's mean as the next layer's bf16 operand: stage 0's (ups.1: leaky 0.1) in B[2],
        // blocks 0 and 1's h, free after the join (not B[3]: ups.1 writes there); stage 1's
        // (conv_post: leaky 0.01) in B[3], the stage's input, free once every block's first step ran
        resblock_mean(&m.rb[3 * i], (const uint16_t*)B[3], X, hs, dout, tu, kShapeWN[m.ups[i].shape] * ou.stride,
                      i == 1, i == 0 ? (void*)B[2] : (void*)B[3], i == 0 ? 0.1f : 0.01f);
    }

    // conv_post over the items [b0, b1) (all: b1 < 0)
    void post_istft(int b0 = 0, int b1 = -1) {
        const Dom& d = p->d120;
        Op o;
        // the input: stage 1's output as the bf16 operand its last conv stored (leaky ReLU 0.01 applied)
        o.pro = PRO_BF16, o.x = p->B[3].p, o.x_ld = 128, o.din = o.dout = &d;
        o.y = p->post.as<float>(), o.y_ld = kPostLd, o.cls = PC_POST;
        o.label = "conv_post";
        if (b1 >= 0) {
            const Tiles& t = p->tl(d, kShapeN[m.post.shape]);
            o.t_lo = t.lo_h[b0], o.t_hi = t.hi_h[b1 - 1];
        }
        conv(m.post, o);
    }

    // the iSTFT of the items [b0, b1) (all: b1 < 0)
    void istft(int b0 = 0, int b1 = -1) {
        IstftParams q{};
        q.post = p->post.as<float>(), q.post_ld = kPostLd;
        q.start120 = p->d120.start_d.as<int64_t>(), q.f_len = p->d120.len_d.as<int64_t>();
        q.blk_item = p->ist_item.as<int64_t>(), q.blk_s0 = p->ist_s0.as<int64_t>(), q.n_blocks = p->n_ist;
        q.audio = p->audio.as<float>(), q.audio_start = p->audio_start.as<int64_t>();
        double share = 1.0;
        if (b1 >= 0) {
            const int64_t k0 = p->ist_first[b0], k1 = p->ist_first[b1];
            q.blk_item += k0, q.blk_s0 += k0, q.n_blocks = k1 - k0;
            share = p->n_ist > 0 ? (double)(k1 - k0) / (double)p->n_ist : 0.0;
        }
        // 22 f32 read per frame, one f32 written per sample (21.6 B per sample)
        launch(PC_ISTFT, 0, share * ((double)p->d120.valid() * 88 + (double)frames() * 600 * 4),
               [&] { return launch_istft(q, s); });
    }

    // conv_post and the iSTFT in up to kOutGroups groups of items (about equal frames each); after
    // each group's iSTFT its samples go to p->early_out on side stream 0, while the next groups
    // compute.  out_ev[kOutGroups] is recorded after the last copy.
    void post_istft_copy() {
        const int nb = p->nb, ng = std::min(nb, (int)kk_plan::kOutGroups);
        int64_t total = 0;
        for (int b = 0; b < nb; b++) total += p->nfr[b];
        int b0 = 0;
        int64_t acc = 0;
        for (int g = 0; g < ng; g++) {
            // the group ends where the running frame count passes (g + 1) / ng of the total,
            // leaving at least one item to each later group
            int b1 = b0 + 1;
            acc += p->nfr[b0];
            while (b1 < nb - (ng - 1 - g) && acc + p->nfr[b1] <= total * (g + 1) / ng) acc += p->nfr[b1++];
            if (g == ng - 1) {
                while (b1 < nb) acc += p->nfr[b1++];
            }
            post_istft(b0, b1);
            istft(b0, b1);
            KK_HIP(hipEventRecord(p->out_ev[g], s));
            KK_HIP(hipStreamWaitEvent(ctx->side[0], p->out_ev[g], 0));
            const int64_t a0 = 600 * p->a[b0], a1 = 600 * (p->a[b1 - 1] + p->nfr[b1 - 1]);
            KK_HIP(hipMemcpyAsync(p->early_out + a0, p->audio.as<float>() + a0, sizeof(float) * (a1 - a0),
                                  hipMemcpyDeviceToHost, ctx->side[0]));
            b0 = b1;
        }
        KK_HIP(hipEventRecord(p->out_ev[kk_plan::kOutGroups], ctx->side[0]));
        p->early_issued = true;
    }

    // ------------------------------------------------------------ the stages before the decoder
    // Linear L over the rows of domain d: x [rows][x_ld] -> y [rows][y_ld] (piece i at its columns;
    // y_ld and the columns in elements of y: f32, or bf16 for EPI_GELU_BF16).
    void linear(const MLinear& L, const void* x, int64_t x_ld, const Dom& d, void* y, int64_t y_ld,
                const std::string& name, int pro = PRO_F32, int epi = EPI_STORE) {
        const bool out_h = epi == EPI_GELU_BF16;
        for (size_t i = 0; i < L.piece.size(); i++) {
            Op o;
            o.pro = pro, o.epi = epi, o.x = x, o.x_ld = x_ld, o.din = o.dout = &d, o.out_h = out_h;
            o.y = (float*)((char*)y + L.col0[i] * (out_h ? 2 : 4));
            o.y_ld = y_ld, o.cls = PC_LINEAR, o.label = name;
            conv(L.piece[i], o);
        }
    }
    // BiLSTM recurrence over the item spans of d (gx rows through gx_row, or the spans' own rows);
    // h into out[row][0:512].  Algorithmic traffic: gx read and h written once per row, W_hh once.
    // Each sequence runs on four CUs (launch_lstm_quad, at most 64 quads running scheduled lists)
    // when the longest span has at least kLstmQuadMinSteps steps (below, the quads' per-step gain
    // does not pay for their lists), else on two (launch_lstm_pair; bit-identical), with its
    // exchange words in `region` (one per stream that runs recurrences at the same time);
    // KOKORO_HIP_LSTM_SINGLE=1 selects the one-CU kernel (W_hh partly streamed from L2 each step),
    // as does a plan whose pairs or quads gave up before (lstm_single).  Test hook, read at each
    // launch: KOKORO_HIP_TEST_LSTM_SILENT=1 keeps the second half of every pair (the second quarter
    // of every quad) from publishing and cuts the wait to 10 us, so that they give up.
    void recur(const MLstm& l, const float* gx, const int32_t* gx_row, const Dom& d, float* out, int64_t out_ld,
               const std::string& name, int region = 0) {
        static const bool single = env_i64("KOKORO_HIP_LSTM_SINGLE", 0) != 0;
        // KOKORO_HIP_LSTM_QUAD, read at each launch: 1 quads, 0 pairs for every span
        check((int)d.len.size() == p->nb, "internal: recurrence domain");
        const int32_t* sched = p->lstm_sched_of(d);
        int64_t longest = 0;
        for (int64_t v : d.len) longest = std::max(longest, v);
        const int64_t qsel = env_i64("KOKORO_HIP_LSTM_QUAD", -1);
        const bool quad = qsel < 0 ? longest >= kLstmQuadMinSteps : qsel != 0;
        const bool silent = env_i64("KOKORO_HIP_TEST_LSTM_SILENT", 0) != 0;
        const double v = (double)d.valid();
        label = name;
        launch(PC_LSTM, v * 2 * 1024 * 256 * 2, v * (2048 + 512) * 4 + 2.0 * 1024 * 257 * 4, [&] {
            if (single || p->lstm_single)
                return launch_lstm(gx, 2048, gx_row, d.start_d.as<int64_t>(), d.len_d.as<int64_t>(), p->nb,
                                   l.whh_t.as<float>(), l.bhh.as<float>(), out, out_ld, s);
            uint64_t* x = p->u_lstmx.as<uint64_t>();
            if (quad)
                return launch_lstm_quad(gx, 2048, gx_row, d.start_d.as<int64_t>(), d.len_d.as<int64_t>(), p->nb,
                                        sched, l.whh_t.as<float>(), l.bhh.as<float>(), out, out_ld,
                                        x + kk_plan::kLstmXHead + (int64_t)region * 2 * p->nb * 512, (int*)x, s,
                                        silent ? 1000 : kLstmPairWaitTicks, silent ? 1 : -1);
            return launch_lstm_pair(gx, 2048, gx_row, d.start_d.as<int64_t>(), d.len_d.as<int64_t>(), p->nb,
                                    l.whh_t.as<float>(), l.bhh.as<float>(), out, out_ld,
                                    x + kk_plan::kLstmXHead + (int64_t)region * 2 * p->nb * 512, (int*)x, s,
                                    silent ? 1000 : kLstmPairWaitTicks, silent ? 1 : -1);
        });
    }
    void layernorm(float* x, int64_t ld, int d, const float* g, const float* b, int gb_off, float eps, bool leaky,
                   const std::string& name) {
        const double v = (double)p->dt.valid();
        label = name;
        launch(PC_ROWS, 0, v * d * 8, [&] {
            return launch_layernorm(x, ld, d, p->dtf.l, p->row_item.as<int32_t>(), g, b,
                                    g ? nullptr : p->gbp.as<float>(), m.up.style_rows, gb_off, eps, leaky, 0.2f, s);
        });
    }
    // text_encoder_b (src/gpu_batch.rs:457-481): embedding, 3 x (conv k5, LayerNorm, leaky 0.2),
    // BiLSTM into t_en [rows][512].
    void text_encoder() {
        const MUp& u = m.up;
        const Dom& dt = p->dt;
        const int64_t R = p->dtf.l;
        float* in = p->u_te.as<float>();
        float* out = p->u_te2.as<float>();
        label = "text_encoder.embedding";
        launch(PC_ROWS, 0, (double)dt.valid() * 512 * 8, [&] {
            return launch_text_embed(p->ids.as<int32_t>(), p->row_item.as<int32_t>(), R, u.te_emb.as<float>(), in, s);
        });
        for (int i = 0; i < 3; i++) {
            const std::string nm = "text_encoder.cnn." + std::to_string(i);
            Op o;
            o.x = in, o.x_ld = 512, o.din = o.dout = &dt, o.y = out, o.y_ld = 512, o.cls = PC_PCONV, o.label = nm + ".0";
            conv(u.te_cnn[i], o);
            layernorm(out, 512, 512, u.te_g[i].as<float>(), u.te_b[i].as<float>(), 0, 1e-5f, true, nm + ".1");
            std::swap(in, out);
        }
        linear(u.te_lstm.wih, in, 512, p->dtf, p->u_gxt.as<float>(), 2048, "text_encoder.lstm.ih");
        recur(u.te_lstm, p->u_gxt.as<float>(), nullptr, dt, p->t_en.as<float>(), 512, "text_encoder.lstm", 1);
    }
    // The token phase (src/gpu_batch.rs:198-248): ALBERT, bert_encoder, the duration encoder, the
    // duration LSTM and projection (logits [rows][kLogitsLd]), the shared LSTM's gate
    // pre-activations on the token rows; the text encoder beside them on side stream 0.
    static constexpr int64_t kLogitsLd = 52;  // 50 logits, the row padded to the epilogue's 4 channels
    void tokens() {
        const MUp& u = m.up;
        const Dom& dt = p->dt;
        const Dom& dtf = p->dtf;
        const int64_t R = dtf.l;
        const double v = (double)dt.valid();
        const bool conc = !ctx->profiling && !dry;
        hipStream_t main_s = s;
        if (!dry) KK_HIP(launch_clear_u64(p->u_lstmx.as<uint64_t>(), 1, s));  // the run's abort flag
        if (conc) {
            KK_HIP(hipEventRecord(p->te_ev[0], main_s));
            KK_HIP(hipStreamWaitEvent(ctx->side[0], p->te_ev[0], 0));
            s = ctx->side[0];
        }
        text_encoder();
        if (conc) {
            KK_HIP(hipEventRecord(p->te_ev[1], s));
            s = main_s;
        }
        // prosody styles: every AdaLayerNorm / AdaIN projection of the predictor
        label = "predictor.style_fc";
        launch(PC_STYLE, 0, (double)u.style_rows * (kStyleDim + 1 + p->nb) * 4, [&] {
            return launch_style_fc(u.style_wt.as<float>(), u.style_b.as<float>(), u.style_rows,
                                   p->style_pro.as<float>(), p->nb, p->gbp.as<float>(), s);
        });
        // ALBERT (albert_b, src/gpu_batch.rs:423-455)
        float* H = p->u_h.as<float>();
        float* QKV = p->u_qkv.as<float>();
        float* CTX = p->u_ctx.as<float>();
        uint16_t* FF = p->u_ffn.as<uint16_t>();
        label = "bert.embeddings";
        launch(PC_ROWS, 0, v * 128 * 12, [&] {
            return launch_albert_embed(p->ids.as<int32_t>(), p->row_item.as<int32_t>(), dt.start_d.as<int64_t>(), R,
                                       u.word.as<float>(), u.pos.as<float>(), u.tok0.as<float>(), u.emb_g.as<float>(),
                                       u.emb_b.as<float>(), p->u_emb.as<float>(), s);
        });
        linear(u.map_in, p->u_emb.p, 128, dtf, H, 768, "bert.embedding_hidden_mapping_in");
        double att_flop = 0;
        for (int64_t t : dt.len) att_flop += 12.0 * 4 * 64 * (double)t * (double)t;
        for (int l = 0; l < 12; l++) {
            const std::string nm = "bert.layer" + std::to_string(l);
            linear(u.qkv, H, 768, dtf, QKV, 2304, nm + ".qkv");
            label = nm + ".attention";
            launch(PC_ATTN, att_flop, v * (2304 + 768) * 4, [&] {
                // KOKORO_HIP_ATTENTION_VALU=1: the f32 VALU kernel instead of the f32 matrix cores
                static const bool valu = env_i64("KOKORO_HIP_ATTENTION_VALU", 0) != 0;
                return launch_attention(QKV, dt.start_d.as<int64_t>(), dt.len_d.as<int64_t>(),
                                        p->att_item.as<int32_t>(), p->att_head.as<int32_t>(), p->att_q0.as<int32_t>(),
                                        p->n_att, CTX, s, valu);
            });
            linear(u.dense, CTX, 768, dtf, H, 768, nm + ".dense", PRO_F32, EPI_RESID);
            layernorm(H, 768, 768, u.attn_g.as<float>(), u.attn_b.as<float>(), 0, 1e-12f, false, nm + ".attention_ln");
            linear(u.ffn, H, 768, dtf, FF, 2048, nm + ".ffn", PRO_F32, EPI_GELU_BF16);  // bf16 gelu_new(ffn)
            linear(u.ffn_out, FF, 2048, dtf, H, 768, nm + ".ffn_output", PRO_BF16, EPI_RESID);
            layernorm(H, 768, 768, u.full_g.as<float>(), u.full_b.as<float>(), 0, 1e-12f, false, nm + ".full_ln");
        }
        // duration encoder on x = [h | s] (640 wide): bert_encoder and each LSTM write h in place,
        // the style half is written once (src/gpu_batch.rs:212-233)
        float* X = p->u_x.as<float>();
        float* GX = p->u_gx.as<float>();
        linear(u.bert_enc, H, 768, dtf, X, 640, "bert_encoder");
        label = "predictor.cat_style";
        launch(PC_ROWS, 0, v * 128 * 4, [&] {
            return launch_style_cols(X, 640, 512, R, p->row_item.as<int32_t>(), p->style_pro.as<float>(), s);
        });
        for (int i = 0; i < 3; i++) {
            const std::string nm = "predictor.text_encoder.lstms." + std::to_string(2 * i);
            linear(u.dur_lstm[i].wih, X, 640, dtf, GX, 2048, nm + ".ih");
            recur(u.dur_lstm[i], GX, nullptr, dt, X, 640, nm);
            layernorm(X, 640, 512, nullptr, nullptr, u.dur_gb_off[i], 1e-5f, false,
                      "predictor.text_encoder.lstms." + std::to_string(2 * i + 1));
        }
        linear(u.pred_lstm.wih, X, 640, dtf, GX, 2048, "predictor.lstm.ih");
        recur(u.pred_lstm, GX, nullptr, dt, p->u_xl.as<float>(), 512, "predictor.lstm");
        linear(u.dur_proj, p->u_xl.p, 512, dtf, p->u_logits.as<float>(), kLogitsLd, "predictor.duration_proj");
        // the shared LSTM's gate pre-activations on the token rows: a frame's are its token's
        linear(u.shared.wih, X, 640, dtf, p->u_gxs.as<float>(), 2048, "predictor.shared.ih");
        if (conc) KK_HIP(hipStreamWaitEvent(main_s, p->te_ev[1], 0));
    }
    // AdainResBlk1d with an identity shortcut (din = dout), in place on X [rows][ld] of domain d.
    void resblk_same(const MResblk& r, float* X, int64_t ld, const Dom& d, float* h, Coef* ca, Coef* cb) {
        stats_fin(X, ld, r.din, d, r.n1, ca);
        Op o1;
        o1.pro = PRO_ADAIN_LEAKY, o1.x = X, o1.x_ld = ld, o1.din = o1.dout = &d, o1.y = h, o1.y_ld = r.dout;
        o1.coef = ca, o1.slope = 0.2f, o1.stats = true, o1.cls = PC_PCONV, o1.label = r.name + ".conv1";
        const Tiles& t = conv(r.conv1, o1);
        fin(t, kShapeWN[r.conv1.shape], r.dout, r.n2, cb);
        Op o2;
        o2.pro = PRO_ADAIN_LEAKY, o2.epi = EPI_RESID, o2.x = h, o2.x_ld = r.dout, o2.din = o2.dout = &d, o2.y = X;
        o2.y_ld = ld, o2.coef = cb, o2.slope = 0.2f, o2.scale = 1.0f / sqrtf(2.0f), o2.cls = PC_PCONV;
        o2.label = r.name + ".conv2";
        conv(r.conv2, o2);
    }
    // The upsampling AdainResBlk1d (src/gpu_batch.rs:104-135): X [ln][xld] at dn -> Y [2 ln][yld] at d2.
    void resblk_up(const MResblk& r, const float* X, int64_t xld, float* Y, int64_t yld, uint16_t* pool, float* h,
                   float* sc, Coef* ca, Coef* cb) {
        const Dom& dn = p->dn;
        const Dom& d2 = p->d2;
        const double nf = (double)frames();
        stats_fin(X, xld, r.din, dn, r.n1, ca);
        label = r.name + ".pool";
        launch(PC_POOL, 0, nf * r.din * 4 + 2 * nf * r.din * 2, [&] {
            return launch_adain_pool(X, xld, r.din, ca, dn.col_d.as<int32_t>(), p->ln, r.pool_w.as<float>(),
                                     r.pool_b.as<float>(), d2.col_d.as<int32_t>(), pool, r.din, s);
        });
        Op o1;
        o1.pro = PRO_BF16, o1.x = pool, o1.x_ld = r.din, o1.din = o1.dout = &d2, o1.y = h, o1.y_ld = r.dout;
        o1.stats = true, o1.cls = PC_PCONV, o1.label = r.name + ".conv1";
        const Tiles& t = conv(r.conv1, o1);
        fin(t, kShapeWN[r.conv1.shape], r.dout, r.n2, cb);
        // shortcut conv1x1(nearest x2 (x)) = nearest x2 (conv1x1(x)) for a 1x1 conv: computed at N
        Op os;
        os.x = X, os.x_ld = xld, os.din = os.dout = &dn, os.y = sc, os.y_ld = r.dout, os.cls = PC_PCONV;
        os.label = r.name + ".conv1x1";
        conv(r.conv1x1, os);
        Op o2;
        o2.pro = PRO_ADAIN_LEAKY, o2.epi = EPI_RESID_UP2, o2.x = h, o2.x_ld = r.dout, o2.din = o2.dout = &d2;
        o2.y = Y, o2.y_ld = yld, o2.coef = cb, o2.slope = 0.2f, o2.r0 = sc, o2.r0_ld = r.dout;
        o2.scale = 1.0f / sqrtf(2.0f), o2.cls = PC_PCONV, o2.label = r.name + ".conv2";
        conv(r.conv2, o2);
    }
    // F0 (k = 0) or N (k = 1) from the shared LSTM's output (src/gpu_batch.rs:282-292) into p->f0 /
    // p->en at d2, 0 in the gaps.
    void f0n_stack(int k, Coef* ca, Coef* cb) {
        const MUp& u = m.up;
        const MResblk* blk = k == 0 ? u.f0 : u.nn;
        float* fx = p->u_fx[k].as<float>();
        float* fh = p->u_fh[k].as<float>();
        float* fy = p->u_fy[k].as<float>();
        const double nf = (double)frames();
        launch(PC_COPY, 0, nf * 512 * 8, [&] {
            return launch_copy_cols(p->u_sh.as<float>(), 512, 512, fx, 512, 0, p->dn.col_d.as<int32_t>(), p->ln, s);
        });
        resblk_same(blk[0], fx, 512, p->dn, fh, ca, cb);
        resblk_up(blk[1], fx, 512, fy, 256, p->u_fpool[k].as<uint16_t>(), fh, p->u_fsc[k].as<float>(), ca, cb);
        resblk_same(blk[2], fy, 256, p->d2, fh, ca, cb);
        label = k == 0 ? "predictor.F0_proj" : "predictor.N_proj";
        launch(PC_ROWS, 2.0 * 2 * nf * 256, 2 * nf * 256 * 4 + 2 * (double)p->ln * 4, [&] {
            return launch_proj1(fy, 256, 256, (k == 0 ? u.f0p_w : u.np_w).as<float>(),
                                (k == 0 ? u.f0p_b : u.np_b).as<float>(), p->d2.col_d.as<int32_t>(), 2 * p->ln,
                                (k == 0 ? p->f0 : p->en).as<float>(), s);
        });
    }
    // The frame phase before the decoder: the shared BiLSTM over the frames (a frame's gate
    // pre-activations are its token row's, through src_row), then the F0 and N stacks, N on side
    // stream 0 beside F0 (each with its own statistics region and AdaIN coefficients).
    void prosody() {
        recur(m.up.shared, p->u_gxs.as<float>(), p->src_row.as<int32_t>(), p->dn, p->u_sh.as<float>(), 512,
              "predictor.shared");
        pro_style = true;
        const bool conc = !ctx->profiling && !dry;
        hipStream_t main_s = s;
        if (conc) {
            KK_HIP(hipEventRecord(p->te_ev[0], main_s));
            KK_HIP(hipStreamWaitEvent(ctx->side[0], p->te_ev[0], 0));
            s = ctx->side[0], region = 1;
            f0n_stack(1, cf(5), cf(6));
            KK_HIP(hipEventRecord(p->te_ev[1], s));
            s = main_s, region = 0;
            f0n_stack(0, cf(0), cf(1));
            KK_HIP(hipStreamWaitEvent(main_s, p->te_ev[1], 0));
        } else {
            f0n_stack(0, cf(0), cf(1));
            f0n_stack(1, cf(0), cf(1));
        }
        pro_style = false;
    }

    void run(int until) {
        if (p->kind == PLAN_FULL) {
            if (!skip_tokens) tokens();
            prosody();
            if (until <= KK_STAGE_PROSODY) return;
        }
        launch(PC_STYLE, 0, (double)m.style_rows * (kStyleDim + 1 + p->nb) * 4, [&] {
            return launch_style_fc(m.style_wt.as<float>(), m.style_b.as<float>(), m.style_rows, p->style.as<float>(),
                                   p->nb, p->gb.as<float>(), s);
        });
        if (p->kind == PLAN_SNAKE) {
            snake_block(*p->sblk, p->B[0].as<float>(), p->B[1].as<float>(), p->ds);
            return;
        }
        // The harmonic source and both stages' noise branches depend only on the inputs and the style:
        // they run on a third side stream beside the decoder and stage 0 (per-launch profiling and
        // runs that stop at the source keep them in order on the main stream).
        const bool conc = !ctx->profiling && !dry && until > KK_STAGE_SOURCE;
        hipStream_t main_s = s;
        if (conc) {
            KK_HIP(hipEventRecord(p->noise_ev[0], main_s));  // after style_fc
            KK_HIP(hipStreamWaitEvent(ctx->side[2], p->noise_ev[0], 0));
            s = ctx->side[2];
            source();
            noise_branch(0);
            KK_HIP(hipEventRecord(p->noise_ev[1], s));
            if (until > KK_STAGE_GEN0) {
                noise_branch(1);
                KK_HIP(hipEventRecord(p->noise_ev[2], s));
            }
            s = main_s;
        }
        if (p->late_items && !dry) stage_late_ten();
        if (p->kind == PLAN_DECODER || p->kind == PLAN_FULL) decoder();
        if (until <= KK_STAGE_DECODER) return;
        if (!conc) source();
        if (until <= KK_STAGE_SOURCE) return;
        if (conc)
            KK_HIP(hipStreamWaitEvent(main_s, p->noise_ev[1], 0));
        else
            noise_branch(0);
        gen_stage(0);
        if (until <= KK_STAGE_GEN0) return;
        if (conc)
            KK_HIP(hipStreamWaitEvent(main_s, p->noise_ev[2], 0));
        else
            noise_branch(1);
        gen_stage(1);
        if (until <= KK_STAGE_GEN1) return;
        if (p->early_out && until >= KK_STAGE_ALL && !dry && !ctx->profiling && p->nb > 1) {
            post_istft_copy();
            return;
        }
        post_istft();
        if (until <= KK_STAGE_POST) return;
        istft();
    }
};

// Every tile list a run needs is built (and uploaded) here, so kk_plan_run allocates nothing.
static void prebuild_tiles(kk_plan* p) {
    Runner r{p, p->ctx, p->ctx->model, p->ctx->stream};
    r.dry = true;
    r.run(KK_STAGE_ALL);
}

// Fills plan p (new, or the one-shot plan whose device buffers are reused) for an ids-level batch
// (GpuKokoro::forward_batch, src/gpu_batch.rs:179-297).  Phase A, at once: the token layout
// (src/gpu_batch.rs:188-197), the token phase on the device, its logits back to the host and the
// durations (src/gpu_batch.rs:234-248).  Phase B: the frame layout and everything after, as a
// decoder plan whose t_en, F0 and N the plan computes itself.
// A two-CU recurrence whose block waited more than 2 s for its partner ends every block of its
// launch and leaves the run's abort flag set (read back into abort_host with the run's last copy).
static void check_lstm_abort(kk_plan* p) {
    if (p->abort_host && *p->abort_host != 0)
        fail(KK_ERR_HIP, "BiLSTM recurrence: a block of a two-CU pair waited more than 2 s for its partner "
                          "(set KOKORO_HIP_LSTM_SINGLE=1 for the one-CU kernel)");
}

static void run_plan(kk_plan* plan, int until, bool skip_tokens = false);

// Drains the stream and reads back the run's abort flag (ids-level plans).
static bool drain_aborted(kk_plan* p) {
    hipStream_t s = p->ctx->stream;
    const bool full = p->kind == PLAN_FULL && p->abort_host;
    if (full) KK_HIP(hipMemcpyAsync(p->abort_host, p->u_lstmx.p, sizeof(uint64_t), hipMemcpyDeviceToHost, s));
    KK_HIP(hipStreamSynchronize(s));
    return full && *p->abort_host != 0;
}

// Every path that hands an ids-level plan's results to the caller (audio, PCM, taps, sync) drains the
// stream and checks that no recurrence of the last run gave up (its h rows would hold an earlier
// run's values).  If one did -- a two-CU pair whose partner was held off its CU past the 2 s bound,
// e.g. by another process -- the plan switches to the one-CU kernel, which waits on no other block,
// and runs again: contention costs time, not an error.  Plans of the other kinds run no recurrence.
static void drain_and_check_abort(kk_plan* p) {
    if (drain_aborted(p) && !p->lstm_single) {
        p->lstm_single = true;
        run_plan(p, p->last_until);
        drain_aborted(p);
    }
    if (p->kind == PLAN_FULL) check_lstm_abort(p);
}


static void init_full_plan(kk_plan* p, const kk_item* items, int n) {
    kk_ctx* ctx = p->ctx;
    const Model& m = ctx->model;
    check(m.ready && m.up.ready, "no model with the stages before the decoder uploaded");
    check(items != nullptr && n > 0, "empty batch");
    PhaseMarks pm;
    reset_plan(p, PLAN_FULL, n);
    int64_t rows = 0;
    p->tstart.assign(n, 0), p->ntok.assign(n, 0);
    for (int b = 0; b < n; b++) {
        const kk_item& it = items[b];
        // src/gpu_batch.rs:182-187
        const std::string e = ids_item_error(it, b);
        check(e.empty(), e);
        p->tstart[b] = rows, p->ntok[b] = it.n_ids;
        rows += it.n_ids + kGapT;
    }
    // ---- phase A: the token phase
    stage_begin(ctx);
    p->dt.build(ctx, rows, p->tstart, p->ntok, false, p->nomask);
    p->dtf.build(ctx, rows, {0}, {rows}, false, p->nomask);
    {
        int32_t* idh = stage<int32_t>(ctx, p->ids, (size_t)rows);
        for (int64_t r = 0; r < rows; r++) idh[r] = 0;
        for (int b = 0; b < n; b++)
            for (int i = 0; i < items[b].n_ids; i++) idh[p->tstart[b] + i] = (int32_t)items[b].ids[i];
    }
    {
        int32_t* ri = stage<int32_t>(ctx, p->row_item, (size_t)rows);
        for (int64_t r = 0; r < rows; r++) ri[r] = -1;
        for (int b = 0; b < n; b++)
            for (int i = 0; i < items[b].n_ids; i++) ri[p->tstart[b] + i] = b;
    }
    {
        float* sp = stage<float>(ctx, p->style_pro, (size_t)n * kStyleDim);
        for (int b = 0; b < n; b++) std::memcpy(&sp[(size_t)b * kStyleDim], items[b].ref_s + kStyleDim, sizeof(float) * kStyleDim);
    }
    {
        // attention work list: (item, head, first query) per 64 queries
        std::vector<int32_t> wi, wh, wq;
        for (int b = 0; b < n; b++)
            for (int h = 0; h < 12; h++)
                for (int q = 0; q < items[b].n_ids; q += 64) wi.push_back(b), wh.push_back(h), wq.push_back(q);
        p->n_att = (int64_t)wi.size();
        stage_vec(ctx, p->att_item, wi), stage_vec(ctx, p->att_head, wh), stage_vec(ctx, p->att_q0, wq);
    }
    const size_t R = (size_t)rows;
    alloc_buf(p, p->gbp, (size_t)n * m.up.style_rows * sizeof(float));
    alloc_buf(p, p->u_emb, R * 128 * sizeof(float));
    alloc_buf(p, p->u_h, R * 768 * sizeof(float));
    alloc_buf(p, p->u_qkv, R * 2304 * sizeof(float));
    alloc_buf(p, p->u_ctx, R * 768 * sizeof(float));
    alloc_buf(p, p->u_ffn, R * 2048 * sizeof(uint16_t));
    alloc_buf(p, p->u_x, R * 640 * sizeof(float));
    alloc_buf(p, p->u_gx, R * 2048 * sizeof(float));
    alloc_buf(p, p->u_xl, R * 512 * sizeof(float));
    alloc_buf(p, p->u_logits, R * Runner::kLogitsLd * sizeof(float));
    alloc_buf(p, p->u_te, R * 512 * sizeof(float));
    alloc_buf(p, p->u_te2, R * 512 * sizeof(float));
    alloc_buf(p, p->u_gxt, R * 2048 * sizeof(float));
    alloc_buf(p, p->u_gxs, R * 2048 * sizeof(float));
    alloc_buf(p, p->t_en, R * 512 * sizeof(float));
    alloc_buf(p, p->u_lstmx, (size_t)(kk_plan::kLstmXHead + 2 * 2 * (int64_t)n * 512) * sizeof(uint64_t));
    if (!p->abort_host) KK_HIP(hipHostMalloc((void**)&p->abort_host, sizeof(uint64_t), hipHostMallocDefault));
    p->t_rows = rows;
    for (auto& e : p->te_ev)
        if (!e) KK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    {
        Runner r{p, ctx, m, ctx->stream};
        r.dry = true;  // builds (stages) the token phase's tile lists and validates its launches
        r.tokens();
    }
    stage_flush(ctx, p->tables_tok, ctx->stream);
    pm.mark("token plan");
    {
        Runner r{p, ctx, m, ctx->stream};
        r.tokens();
    }
    pm.mark("token enqueue");
    const size_t lg_bytes = R * Runner::kLogitsLd * sizeof(float);
    if (p->logits_cap < lg_bytes) {
        if (p->logits_host) (void)hipHostFree(p->logits_host);
        p->logits_host = nullptr, p->logits_cap = 0;
        KK_HIP(hipHostMalloc((void**)&p->logits_host, lg_bytes, hipHostMallocDefault));
        p->logits_cap = lg_bytes;
    }
    for (int attempt = 0;; attempt++) {
        KK_HIP(hipMemcpyAsync(p->logits_host, p->u_logits.p, lg_bytes, hipMemcpyDeviceToHost, ctx->stream));
        KK_HIP(hipMemcpyAsync(p->abort_host, p->u_lstmx.p, sizeof(uint64_t), hipMemcpyDeviceToHost, ctx->stream));
        KK_HIP(hipStreamSynchronize(ctx->stream));
        if (*p->abort_host == 0 || attempt > 0 || p->lstm_single) break;
        // a two-CU pair gave up: the token phase again with the one-CU recurrences (see
        // drain_and_check_abort)
        p->lstm_single = true;
        Runner r{p, ctx, m, ctx->stream};
        r.tokens();
    }
    check_lstm_abort(p);
    pm.mark("token device");
    // durations_from_logits (src/model.rs:90-100) per item, the items spread over a few host
    // threads (each item's arithmetic is the rule's own, in its own order)
    p->pred.assign(n, {});
    for (int b = 0; b < n; b++) p->pred[b].assign(items[b].n_ids, 0);
    std::vector<int> drc(n, KK_OK);
    auto durations_of = [&](int b0, int stride) {
        std::vector<float> lg;
        for (int b = b0; b < n; b += stride) {
            const int t = items[b].n_ids;
            lg.resize((size_t)t * 50);
            for (int i = 0; i < t; i++)
                std::memcpy(&lg[(size_t)i * 50], p->logits_host + (size_t)(p->tstart[b] + i) * Runner::kLogitsLd,
                            sizeof(float) * 50);
            drc[b] = kk_durations_from_logits(lg.data(), t, items[b].speed, p->pred[b].data());
        }
    };
    {
        const int nt = std::max(1, std::min({n, 8, (int)std::thread::hardware_concurrency()}));
        std::vector<std::thread> th;
        for (int k = 1; k < nt; k++) th.emplace_back(durations_of, k, nt);
        durations_of(0, nt);
        for (auto& x : th) x.join();
    }
    for (int b = 0; b < n; b++) {
        check(drc[b] == KK_OK, "durations");
        int64_t nf = 0;
        for (int64_t d : p->pred[b]) nf += d;
        check(nf <= (int64_t)1 << 22, "item " + std::to_string(b) + ": too many frames");
        check_noise(NoiseIn{items[b].noise_kind, items[b].seed, items[b].rand_ini, items[b].sine, items[b].sine_len},
                    nf, b);
        p->nfr.push_back(nf);
    }
    pm.mark("durations");
    // ---- phase B: the frame layout and the decoder + generator inputs
    stage_begin(ctx);
    build_frame_layout(p);
    const int64_t ln = p->ln;
    {
        std::vector<const int64_t*> durs(n);
        std::vector<int32_t> nt(n);
        for (int b = 0; b < n; b++) durs[b] = p->pred[b].data(), nt[b] = (int32_t)p->ntok[b];
        int32_t* sr = stage<int32_t>(ctx, p->src_row, (size_t)ln);
        check(kk_layout_src_row(durs.data(), nt.data(), n, p->tstart.data(), p->a.data(), ln, sr) == KK_OK,
              "duration expansion overflows the frame layout");
    }
    std::vector<const float*> refs(n);
    std::vector<NoiseIn> nz(n);
    for (int b = 0; b < n; b++) {
        refs[b] = items[b].ref_s;
        nz[b] = NoiseIn{items[b].noise_kind, items[b].seed, items[b].rand_ini, items[b].sine, items[b].sine_len};
    }
    pm.mark("frame layout");
    setup_generator(p, {}, refs, nz);
    pm.mark("generator setup");
    alloc_buf(p, p->en, (size_t)2 * ln * sizeof(float));
    alloc_buf(p, p->u_sh, (size_t)ln * 512 * sizeof(float));
    for (int k = 0; k < 2; k++) {
        alloc_buf(p, p->u_fx[k], (size_t)ln * 512 * sizeof(float));
        alloc_buf(p, p->u_fpool[k], (size_t)2 * ln * 512 * sizeof(uint16_t));
        alloc_buf(p, p->u_fh[k], (size_t)2 * ln * 256 * sizeof(float));
        alloc_buf(p, p->u_fsc[k], (size_t)ln * 256 * sizeof(float));
        alloc_buf(p, p->u_fy[k], (size_t)2 * ln * 256 * sizeof(float));
    }
    alloc_buf(p, p->xcat, (size_t)ln * kXcatLd * sizeof(float));
    alloc_buf(p, p->xin_a, (size_t)ln * kXinLd * sizeof(float));
    alloc_buf(p, p->xin_b, (size_t)ln * kXinLd * sizeof(float));
    alloc_buf(p, p->hdec, (size_t)ln * 1024 * sizeof(float));
    alloc_buf(p, p->pool, (size_t)2 * ln * kXinLd * sizeof(uint16_t));
    alloc_buf(p, p->sc_half, (size_t)ln * 512 * sizeof(float));
    alloc_buf(p, p->dec_out, (size_t)2 * ln * 512 * sizeof(float));
    pm.mark("frame buffers");
    finish_plan(p);
    pm.mark("frame plan");
    pm.print("init_full_plan");
}

static void release_plan_device(kk_plan* p) {
    p->drop_events();
    p->tiles.clear(), p->lstm_sched.clear();
    for (kk::Dom* d : {&p->dn, &p->d2, &p->d20, &p->d120, &p->ds, &p->dt, &p->dtf}) d->release();
    for (DevBuf* b : p->owned()) b->release();
    p->ctx = nullptr;
}

// After a failed run: work the run left on the side streams (between a fork and its join) is
// joined back into the context's stream, so that later work there -- a retried run, a fetch, a
// free -- is ordered after it.
static void join_side_streams(kk_ctx* ctx) {
    for (int q = 0; q < 3; q++) {
        if (!ctx->side[q] || !ctx->join_ev[q]) continue;
        if (hipEventRecord(ctx->join_ev[q], ctx->side[q]) == hipSuccess)
            (void)hipStreamWaitEvent(ctx->stream, ctx->join_ev[q], 0);
    }
}

// Drops the one-shot plan and its device memory (after a failure, or at kk_close).
static void drop_oneshot(kk_ctx* ctx) {
    if (!ctx->oneshot) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (auto ss : ctx->side)
        if (ss) (void)hipStreamSynchronize(ss);
    release_plan_device(ctx->oneshot);
    delete ctx->oneshot;
    ctx->oneshot = nullptr;
}

// ------------------------------------------------------------------ host output memory
// The audio of kk_plan_fetch / kk_forward_decoder_batch lands in pinned host blocks that the
// library keeps for reuse: one block per fetch holds the whole packed sample layout (one DMA copy,
// no host-side copy), and each item's kk_output points into it.  kk_output_free returns the
// item's reference; the block is free again when all its items are.  Blocks are process-wide (an
// output may outlive its context) and never shrink below the largest batch fetched.
struct OutBlock {
    char* base;
    size_t bytes;
    int refs;  // live items pointing into the block
};
static std::mutex g_out_mu;
static std::vector<OutBlock> g_out;

static char* out_block_take(size_t bytes, int refs) {
    std::lock_guard<std::mutex> lock(g_out_mu);
    int best = -1;
    for (int i = 0; i < (int)g_out.size(); i++)
        if (g_out[i].refs == 0 && g_out[i].bytes >= bytes && (best < 0 || g_out[i].bytes < g_out[best].bytes)) best = i;
    if (best < 0) {
        // free blocks too small for this size would only grow the pool: release them
        for (int i = (int)g_out.size() - 1; i >= 0; i--)
            if (g_out[i].refs == 0) {
                (void)hipHostFree(g_out[i].base);
                g_out.erase(g_out.begin() + i);
            }
        void* p = nullptr;
        KK_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
        g_out.push_back(OutBlock{(char*)p, bytes, 0});
        best = (int)g_out.size() - 1;
    }
    g_out[best].refs = refs;
    return g_out[best].base;
}

// Releases one item reference; false when `p` is not inside a block of the pool.
static bool out_block_release(const void* p) {
    std::lock_guard<std::mutex> lock(g_out_mu);
    for (auto& b : g_out)
        if ((const char*)p >= b.base && (const char*)p < b.base + b.bytes && b.refs > 0) {
            b.refs--;
            return true;
        }
    return false;
}

static void set_err(char* err, size_t errlen, const std::string& m) {
    if (err && errlen) {
        std::snprintf(err, errlen, "%s", m.c_str());
    }
}

template <class F>
static int guard(char* err, size_t errlen, F&& f) {
    try {
        f();
        return KK_OK;
    } catch (const Err& e) {
        set_err(err, errlen, e.msg);
        return e.code;
    } catch (const std::bad_alloc&) {
        set_err(err, errlen, "host allocation failed");
        return KK_ERR_OOM;
    } catch (const std::exception& e) {
        set_err(err, errlen, e.what());
        return KK_ERR_INVALID;
    }
}

static void use_device(const kk_ctx* ctx) { KK_HIP(hipSetDevice(ctx->device)); }

// Copy rows [r0, r0 + rows) x channels [0, c) of a time-major buffer and transpose to [c][rows].
static void tap_rows(const void* dev, int64_t ld, int64_t r0, int64_t rows, int c, float* dst) {
    std::vector<float> h((size_t)rows * ld);
    KK_HIP(hipMemcpy(h.data(), (const float*)dev + r0 * ld, sizeof(float) * rows * ld, hipMemcpyDeviceToHost));
    for (int ch = 0; ch < c; ch++)
        for (int64_t t = 0; t < rows; t++) dst[(size_t)ch * rows + t] = h[(size_t)t * ld + ch];
}
// The same for a bf16 [rows][ld] tensor (each value widened exactly).
static void tap_rows_bf16(const void* dev, int64_t ld, int64_t r0, int64_t rows, int c, float* dst) {
    std::vector<uint16_t> h((size_t)rows * ld);
    KK_HIP(hipMemcpy(h.data(), (const uint16_t*)dev + r0 * ld, sizeof(uint16_t) * rows * ld,
                     hipMemcpyDeviceToHost));
    for (int ch = 0; ch < c; ch++)
        for (int64_t t = 0; t < rows; t++) {
            const uint32_t bits = (uint32_t)h[(size_t)t * ld + ch] << 16;
            float v;
            std::memcpy(&v, &bits, sizeof v);
            dst[(size_t)ch * rows + t] = v;
        }
}

}  // namespace kk

using namespace kk;

// A model checkpoint read on the host: flattened "submodule.param" names (sorted) to tensors.
struct kk_checkpoint {
    std::map<std::string, kk::HostTensor> t;
    std::vector<const std::string*> names;  // index -> name
};

namespace kk {
// The model's tensors of a checkpoint as the weight table kk_upload_model takes, with weight_norm
// resolved: a conv whose "X.weight" is absent is built from "X.weight_g" / "X.weight_v"
// (Weights::conv_weight, src/weights.rs:62-73).
static void upload_checkpoint(kk_ctx* ctx, const kk_checkpoint* ck) {
    std::vector<kk_tensor> tab;
    std::vector<std::unique_ptr<std::vector<float>>> resolved;
    std::vector<std::unique_ptr<std::string>> names;
    for (const auto& kv : ck->t) {
        const std::string& nm = kv.first;
        static const char* const kPrefixes[] = {"decoder.", "bert.", "bert_encoder.", "predictor.", "text_encoder."};
        bool keep = false;
        for (const char* pre : kPrefixes) keep = keep || nm.compare(0, std::strlen(pre), pre) == 0;
        if (!keep) continue;
        tab.push_back(kk_tensor{nm.c_str(), kv.second.data.data(), (int64_t)kv.second.data.size()});
        const std::string suf = ".weight_v";
        if (nm.size() > suf.size() && nm.compare(nm.size() - suf.size(), suf.size(), suf) == 0) {
            const std::string base = nm.substr(0, nm.size() - suf.size());
            if (ck->t.count(base + ".weight")) continue;
            auto g = ck->t.find(base + ".weight_g");
            check(g != ck->t.end(), "checkpoint: " + nm + " without " + base + ".weight_g");
            const HostTensor& v = kv.second;
            check(!v.shape.empty() && v.shape[0] > 0, "checkpoint: " + nm + " has no rows");
            const int64_t rows = v.shape[0], per = (int64_t)v.data.size() / rows;
            check(g->second.data.size() == (size_t)rows, "checkpoint: " + base + ".weight_g holds " +
                                                             std::to_string(g->second.data.size()) + " values for " +
                                                             std::to_string(rows) + " rows");
            resolved.push_back(std::make_unique<std::vector<float>>(v.data.size()));
            weight_norm(v.data.data(), g->second.data.data(), rows, per, resolved.back()->data());
            names.push_back(std::make_unique<std::string>(base + ".weight"));
            tab.push_back(kk_tensor{names.back()->c_str(), resolved.back()->data(), (int64_t)v.data.size()});
        }
    }
    load_model(ctx, tab.data(), (int)tab.size(), true);
}
}  // namespace kk

// ------------------------------------------------------------------ no-allocation entry point
// kk_snake_block_noalloc's device scratch: one array per device, held from the first use of the
// library on that device until the process ends.  Regions (bytes, 256-aligned):
//   h        fp16 [rows][C]                          (the Snake steps' conv1 output)
//   part     statistics partials                     (rows / 128 + 2 items + 2) x C records
//   coef     two AdaIN coefficient sets              [items][C] each
//   gb       style projections of every AdaIN        [items][style rows]
//   tables   the call's layout, tile lists, styles   (one copy from the host)
// Nothing in it must start at zero: every region is written by the call before it is read.
namespace {
constexpr size_t kNaRows = KK_NOALLOC_MAX_ROWS, kNaItems = KK_NOALLOC_MAX_ITEMS, kNaMaxC = 256;
constexpr size_t na_align(size_t v) { return (v + 255) / 256 * 256; }
constexpr size_t kNaH = 0;
constexpr size_t kNaPart = kNaH + na_align(kNaRows * kNaMaxC * 2);
constexpr size_t kNaPartBytes = na_align((kNaRows / 128 + 2 * kNaItems + 2) * kNaMaxC * sizeof(StatPart));
constexpr size_t kNaCoef = kNaPart + kNaPartBytes;
constexpr size_t kNaCoefBytes = na_align(kNaItems * kNaMaxC * sizeof(Coef));
constexpr size_t kNaGb = kNaCoef + 2 * kNaCoefBytes;
constexpr size_t kNaGbBytes = (size_t)12 << 20;  // items x style rows x 4 (37,396 rows for Kokoro-82M)
constexpr size_t kNaTables = kNaGb + kNaGbBytes;
constexpr size_t kNaTablesBytes = (size_t)1 << 20;
constexpr size_t kNaTotal = kNaTables + kNaTablesBytes;
static_assert(kNaTotal <= KK_NOALLOC_SCRATCH_BYTES, "scratch regions exceed the array");
}  // namespace
static __device__ __align__(256) unsigned char scratch[KK_NOALLOC_SCRATCH_BYTES];

namespace kk {
static void run_plan(kk_plan* plan, int until, bool skip_tokens) {
    use_device(plan->ctx);
    check(plan->ctx->model.ready, "no model uploaded");
    check(plan->kind != PLAN_FULL || plan->ctx->model.up.ready, "no model with the stages before the decoder uploaded");
    check(until >= (plan->kind == PLAN_FULL ? KK_STAGE_PROSODY : KK_STAGE_DECODER) && until <= KK_STAGE_ALL,
          "unknown stage");
    hipStream_t s = plan->ctx->stream;
    Runner r{plan, plan->ctx, plan->ctx->model, s};
    r.skip_tokens = skip_tokens;
    plan->last_until = -1;
    try {
        // Eager launches: the generator's three resblock chains run on three streams at once, which
        // a captured HIP graph executes one node at a time on this runtime (measured: the graph
        // replay of the same sequence is 1.7% slower per step).
        r.run(until);
    } catch (...) {
        join_side_streams(plan->ctx);
        throw;
    }
    plan->conv_flop = r.flop, plan->snake_flop = r.snake_flop, plan->launches = r.launches;
    plan->last_until = until;
}


// The Snake block on caller memory: a plan whose buffers are views of x and of the scratch regions;
// its tables are staged in host heap memory and copied into the tables region (a pageable copy:
// no pinned allocation).
static void snake_block_noalloc(kk_ctx* ctx, const char* prefix, float* x, int64_t rows, const int64_t* start,
                                const int64_t* len, int n, const float* const* ref_s) {
    use_device(ctx);
    check(ctx->model.ready, "no model uploaded");
    check(ctx->scratch != nullptr, "context without scratch");
    check(prefix && x && start && len && ref_s, "null argument");
    const MSnake* blk = find_snake(ctx->model, prefix);
    check(blk != nullptr, std::string("no Snake block named ") + prefix);
    check(n >= 1 && n <= (int)kNaItems, "kk_snake_block_noalloc takes 1 to " + std::to_string(kNaItems) +
                                            " items (" + std::to_string(n) + " given)");
    check(rows >= 1 && rows <= (int64_t)kNaRows, "kk_snake_block_noalloc takes at most " +
                                                     std::to_string(kNaRows) + " rows (" + std::to_string(rows) +
                                                     " given)");
    const int c = blk->c;
    check((size_t)c <= kNaMaxC, "block wider than the scratch");
    check((size_t)n * ctx->model.style_rows * sizeof(float) <= kNaGbBytes, "too many items for the style scratch");
    // item spans: inside [0, rows), pairwise disjoint
    std::vector<std::pair<int64_t, int64_t>> sp(n);
    for (int b = 0; b < n; b++) {
        check(ref_s[b] != nullptr, "item " + std::to_string(b) + ": null style");
        check(start[b] >= 0 && len[b] >= 1 && start[b] + len[b] <= rows,
              "item " + std::to_string(b) + ": span outside [0, rows)");
        sp[b] = {start[b], len[b]};
    }
    std::sort(sp.begin(), sp.end());
    for (int b = 1; b < n; b++) check(sp[b - 1].first + sp[b - 1].second <= sp[b].first, "overlapping item spans");

    kk_plan p;
    p.ctx = ctx;
    reset_plan(&p, PLAN_SNAKE, n);
    p.sblk = blk, p.sc = c;
    for (int b = 0; b < n; b++) p.nfr.push_back(len[b]);
    // host staging of the tables in heap memory, in place of the context's pinned buffer
    Staging local;
    local.pageable = true;
    std::swap(local, ctx->stage);
    struct Restore {
        kk_ctx* ctx;
        Staging* saved;
        ~Restore() { std::swap(*saved, ctx->stage); }
    } restore{ctx, &local};
    stage_begin(ctx);
    p.ds.build(ctx, rows, std::vector<int64_t>(start, start + n), std::vector<int64_t>(len, len + n), false,
               p.nomask);
    {
        float* sth = stage<float>(ctx, p.style, (size_t)n * kStyleDim);
        for (int b = 0; b < n; b++) std::memcpy(&sth[(size_t)b * kStyleDim], ref_s[b], sizeof(float) * kStyleDim);
    }
    unsigned char* base = ctx->scratch;
    p.B[0].view(x, (size_t)rows * c * sizeof(float));
    p.B[1].view(base + kNaH, (size_t)rows * c * 2);
    p.part.view(base + kNaPart, kNaPartBytes);
    p.part_bytes = (int64_t)kNaPartBytes;
    for (int i = 0; i < 2; i++) p.coef[i].view(base + kNaCoef + i * kNaCoefBytes, (size_t)n * c * sizeof(Coef));
    p.gb.view(base + kNaGb, (size_t)n * ctx->model.style_rows * sizeof(float));
    prebuild_tiles(&p);  // tile lists staged, launches validated (partials bound included)
    Staging& st = ctx->stage;
    check(st.used <= kNaTablesBytes, "layout tables exceed the scratch");
    hipStream_t s = ctx->stream;
    try {
        KK_HIP(hipMemcpyAsync(base + kNaTables, st.host, st.used, hipMemcpyHostToDevice, s));
        for (const auto& r : st.refs) r.buf->view(base + kNaTables + r.off, r.bytes);
        st.refs.clear();
        p.frozen = true;
        run_plan(&p, KK_STAGE_ALL);
    } catch (...) {
        // a failure after the first enqueue: run_plan has joined its side streams into s, so draining
        // s leaves no kernel of this call writing x or the scratch once the error is returned
        (void)hipStreamSynchronize(s);
        throw;
    }
    // x holds the result when the call returns (and the host tables outlive their copy)
    KK_HIP(hipStreamSynchronize(s));
}
}  // namespace kk

extern "C" {

const char* kk_identity(void) { return "hip-gfx950 bf16-mfma f32-acc"; }

int kk_open(int ordinal, kk_ctx** out, char* err, size_t errlen) {
    if (!out) return KK_ERR_INVALID;
    *out = nullptr;
    return guard(err, errlen, [&] {
        int n = 0;
        KK_HIP(hipGetDeviceCount(&n));
        check(ordinal >= 0 && ordinal < n, "device ordinal " + std::to_string(ordinal) + " out of range (" +
                                               std::to_string(n) + " devices visible)");
        hipDeviceProp_t prop;
        KK_HIP(hipGetDeviceProperties(&prop, ordinal));
        check(std::strncmp(prop.gcnArchName, "gfx950", 6) == 0,
              std::string("device ") + std::to_string(ordinal) + " is " + prop.gcnArchName +
                  "; this build carries gfx950 code only");
        auto ctx = std::make_unique<kk_ctx>();
        ctx->device = ordinal;
        ctx->name = prop.name[0] ? prop.name : prop.gcnArchName;
        ctx->n_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;
        KK_HIP(hipSetDevice(ordinal));
        KK_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
        for (auto& ss : ctx->side) KK_HIP(hipStreamCreateWithFlags(&ss, hipStreamNonBlocking));
        for (auto& e : ctx->join_ev) KK_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        KK_HIP(hipEventCreateWithFlags(&ctx->stage.done, hipEventDisableTiming));
        KK_HIP(hipEventCreateWithFlags(&ctx->stage_late.done, hipEventDisableTiming));
        // twiddles and periodic Hann window in f64 (src/gpu.rs:93-101)
        double cs[220], sn[220];
        float win[20];
        for (int k = 0; k < 11; k++)
            for (int j = 0; j < 20; j++) {
                const double a = 2.0 * M_PI * (double)((k * j) % 20) / 20.0;
                cs[k * 20 + j] = std::cos(a);
                sn[k * 20 + j] = std::sin(a);
            }
        for (int j = 0; j < 20; j++) win[j] = (float)(0.5 - 0.5 * std::cos(2.0 * M_PI * (double)j / 20.0));
        KK_HIP(upload_stft_tables(cs, sn, win));
        // this device's copy of kk_snake_block_noalloc's scratch array: its device address, taken
        // once per context with the device current (in host code the array's name is only a
        // stand-in, not a device address)
        void* sp = nullptr;
        KK_HIP(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
        check(sp != nullptr, "no device address for the scratch array");
        ctx->scratch = (unsigned char*)sp;
        *out = ctx.release();
    });
}

void kk_close(kk_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto ss : ctx->side)
        if (ss) (void)hipStreamSynchronize(ss);
    // plans still alive lose their device memory now and become orphans: kk_plan_free later only
    // releases the host object, and every other entry on them reports KK_ERR_STATE
    for (kk_plan* p : ctx->plans) release_plan_device(p);
    ctx->plans.clear();
    drop_oneshot(ctx);
    if (ctx->stage.host) (void)hipHostFree(ctx->stage.host);
    if (ctx->stage.done) (void)hipEventDestroy(ctx->stage.done);
    if (ctx->stage_late.host) (void)hipHostFree(ctx->stage_late.host);
    if (ctx->stage_late.done) (void)hipEventDestroy(ctx->stage_late.done);
    for (auto e : ctx->join_ev)
        if (e) (void)hipEventDestroy(e);
    for (auto& r : ctx->prof) {
        (void)hipEventDestroy(r.e0);
        (void)hipEventDestroy(r.e1);
    }
    for (auto e : ctx->event_pool) (void)hipEventDestroy(e);
    ctx->model = Model();
    for (auto ss : ctx->side)
        if (ss) (void)hipStreamSynchronize(ss), (void)hipStreamDestroy(ss);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int kk_device_name(const kk_ctx* ctx, char* buf, size_t len) {
    if (!ctx || !buf || !len) return KK_ERR_INVALID;
    std::snprintf(buf, len, "%s", ctx->name.c_str());
    return KK_OK;
}

int kk_checkpoint_open(const char* path, kk_checkpoint** out, char* err, size_t errlen) {
    if (!path || !out) return KK_ERR_INVALID;
    *out = nullptr;
    return guard(err, errlen, [&] {
        auto ck = std::make_unique<kk_checkpoint>();
        try {
            ck->t = read_model_checkpoint(path);
        } catch (const std::runtime_error& e) {
            fail(KK_ERR_INVALID, e.what());
        }
        for (const auto& kv : ck->t) ck->names.push_back(&kv.first);
        *out = ck.release();
    });
}

int kk_checkpoint_count(const kk_checkpoint* ck) { return ck ? (int)ck->names.size() : KK_ERR_INVALID; }

int kk_checkpoint_entry(const kk_checkpoint* ck, int i, const char** name, const int64_t** shape, int* ndim,
                        const float** data, int64_t* numel) {
    if (!ck || i < 0 || i >= (int)ck->names.size()) return KK_ERR_INVALID;
    const std::string& nm = *ck->names[i];
    const HostTensor& t = ck->t.at(nm);
    if (name) *name = nm.c_str();
    if (shape) *shape = t.shape.data();
    if (ndim) *ndim = (int)t.shape.size();
    if (data) *data = t.data.data();
    if (numel) *numel = (int64_t)t.data.size();
    return KK_OK;
}

void kk_checkpoint_free(kk_checkpoint* ck) { delete ck; }

int kk_upload_checkpoint(kk_ctx* ctx, const kk_checkpoint* ck, char* err, size_t errlen) {
    if (!ctx || !ck) return KK_ERR_INVALID;
    return guard(err, errlen, [&] {
        use_device(ctx);
        upload_checkpoint(ctx, ck);
    });
}

int kk_weight_norm(const float* v, const float* g, int64_t rows, int64_t per_row, float* w) {
    if (!v || !g || !w || rows < 0 || per_row < 0) return KK_ERR_INVALID;
    weight_norm(v, g, rows, per_row, w);
    return KK_OK;
}

int kk_voice_load(const char* const* paths, int n, float** pack, int64_t* rows, char* err, size_t errlen) {
    if (!paths || n <= 0 || !pack || !rows) return KK_ERR_INVALID;
    *pack = nullptr, *rows = 0;
    return guard(err, errlen, [&] {
        std::vector<HostTensor> packs;
        for (int i = 0; i < n; i++) {
            check(paths[i] != nullptr, "null voice path");
            try {
                packs.push_back(read_voice_pack(paths[i]));
            } catch (const std::runtime_error& e) {
                fail(KK_ERR_INVALID, e.what());
            }
            check(packs.back().shape == packs[0].shape, "voice packs have different shapes");
        }
        const size_t m = packs[0].data.size();
        float* out = (float*)std::malloc(sizeof(float) * std::max<size_t>(m, 1));
        if (!out) throw std::bad_alloc();
        if (n == 1) {
            std::memcpy(out, packs[0].data.data(), sizeof(float) * m);
        } else {
            // the element-wise mean of the packs, summed in order in f32 (src/engine.rs:127-130)
            const float fn = (float)n;
            for (size_t i = 0; i < m; i++) {
                float s = 0.f;
                for (int p = 0; p < n; p++) s += packs[p].data[i];
                out[i] = s / fn;
            }
        }
        *pack = out;
        *rows = packs[0].shape[0];
    });
}

void kk_voice_free(float* pack) { std::free(pack); }

int kk_voice_ref_s(const float* pack, int64_t rows, int64_t n_phoneme_chars, const float** ref_s) {
    // Voice::ref_s (src/engine.rs:54-59): row n - 1 of the pack, 256 values
    if (!pack || !ref_s || n_phoneme_chars < 1 || n_phoneme_chars > rows) return KK_ERR_INVALID;
    *ref_s = pack + (n_phoneme_chars - 1) * 256;
    return KK_OK;
}

int kk_upload_model(kk_ctx* ctx, const kk_tensor* tensors, int n, char* err, size_t errlen) {
    if (!ctx || (!tensors && n > 0)) return KK_ERR_INVALID;
    return guard(err, errlen, [&] {
        use_device(ctx);
        load_model(ctx, tensors, n);
    });
}

int kk_plan_create(kk_ctx* ctx, const kk_decoder_item* items, int n, kk_plan** out, char* err, size_t errlen) {
    if (!ctx || !out) return KK_ERR_INVALID;
    *out = nullptr;
    return guard(err, errlen, [&] {
        use_device(ctx);
        *out = create_decoder_plan(ctx, items, n);
    });
}

int kk_plan_create_full(kk_ctx* ctx, const kk_item* items, int n, kk_plan** out, char* err, size_t errlen) {
    if (!ctx || !out) return KK_ERR_INVALID;
    *out = nullptr;
    return guard(err, errlen, [&] {
        use_device(ctx);
        auto p = std::make_unique<kk_plan>();
        p->ctx = ctx;
        init_full_plan(p.get(), items, n);
        *out = register_plan(ctx, std::move(p));
    });
}

int kk_plan_durations(const kk_plan* plan, int item, const int64_t** dur, int32_t* n_tok) {
    if (!plan || !dur || !n_tok || plan->kind != PLAN_FULL || item < 0 || item >= plan->nb) return KK_ERR_INVALID;
    *dur = plan->pred[item].data();
    *n_tok = (int32_t)plan->pred[item].size();
    return KK_OK;
}

int kk_plan_create_generator(kk_ctx* ctx, const kk_generator_item* items, int n, kk_plan** out, char* err,
                             size_t errlen) {
    if (!ctx || !out) return KK_ERR_INVALID;
    *out = nullptr;
    return guard(err, errlen, [&] {
        use_device(ctx);
        *out = create_generator_plan(ctx, items, n);
    });
}

int kk_snake_block_noalloc(kk_ctx* ctx, const char* prefix, float* x, int64_t rows, const int64_t* start,
                           const int64_t* len, int n, const float* const* ref_s, char* err, size_t errlen) {
    if (!ctx) return KK_ERR_INVALID;
    return guard(err, errlen, [&] { snake_block_noalloc(ctx, prefix, x, rows, start, len, n, ref_s); });
}

int kk_plan_create_snake(kk_ctx* ctx, const char* prefix, const float* const* x, const int64_t* t,
                         const float* const* ref_s, int n, int gap, kk_plan** out, char* err, size_t errlen) {
    if (!ctx || !out) return KK_ERR_INVALID;
    *out = nullptr;
    return guard(err, errlen, [&] {
        use_device(ctx);
        *out = create_snake_plan(ctx, prefix, x, t, ref_s, n, gap);
    });
}

int kk_plan_run(kk_plan* plan, int until, char* err, size_t errlen) {
    if (!plan) return KK_ERR_INVALID;
    if (!plan->ctx) {
        set_err(err, errlen, "plan outlived its context");
        return KK_ERR_STATE;
    }
    return guard(err, errlen, [&] { run_plan(plan, until); });
}

int kk_plan_sync(kk_plan* plan, char* err, size_t errlen) {
    if (!plan) return KK_ERR_INVALID;
    if (!plan->ctx) {
        set_err(err, errlen, "plan outlived its context");
        return KK_ERR_STATE;
    }
    return guard(err, errlen, [&] {
        use_device(plan->ctx);
        drain_and_check_abort(plan);
    });
}

// Each item's result into `out` (see kk_plan_fetch).  Audio: one copy of the whole packed sample
// layout into a pinned block of the output pool; the items point into it.
// blk: a pinned block already taken for the plan's samples with out[] pointing into it (the
// one-shot entries: the run may have issued the copies itself, early_issued), or null.
static void fetch_plan(kk_plan* plan, kk_output* out, float* blk = nullptr) {
    use_device(plan->ctx);
    check(plan->last_until >= KK_STAGE_ALL || plan->kind == PLAN_SNAKE, "plan has not run to the end");
    hipStream_t s = plan->ctx->stream;
    if (plan->kind == PLAN_SNAKE) {
        KK_HIP(hipStreamSynchronize(s));
        for (int b = 0; b < plan->nb; b++) {
            const int64_t t = plan->ds.len[b];
            out[b].n_samples = t * plan->sc;
            out[b].audio = (float*)std::malloc(sizeof(float) * out[b].n_samples);
            if (!out[b].audio) throw std::bad_alloc();
            tap_rows(plan->B[0].p, plan->sc, plan->ds.start[b], t, plan->sc, out[b].audio);
        }
        return;
    }
    const size_t bytes = sizeof(float) * 600 * (size_t)plan->ln;
    if (!blk) {
        blk = (float*)out_block_take(bytes, plan->nb);
        for (int b = 0; b < plan->nb; b++) out[b] = kk_output{blk + 600 * plan->a[b], 600 * plan->nfr[b]};
    }
    // ids-level plans: the run checked (and run again on the one-CU recurrences if a pair gave up)
    // before its audio is copied; the one-shot run's early copies are issued again by that rerun
    if (plan->kind == PLAN_FULL) drain_and_check_abort(plan);
    if (!plan->early_issued) KK_HIP(hipMemcpyAsync(blk, plan->audio.p, bytes, hipMemcpyDeviceToHost, s));
    KK_HIP(hipStreamSynchronize(s));
    if (plan->early_issued) {
        KK_HIP(hipEventSynchronize(plan->out_ev[kk_plan::kOutGroups]));
        plan->early_issued = false;
    }
}

// The one-shot entries take the output block before the run, so that the run can copy each group
// of items' samples into it as soon as they are done (out[] points into it from here on: a failure
// releases it through kk_output_free after the streams are drained).
static float* take_early_block(kk_plan* p, kk_output* out) {
    float* blk = (float*)out_block_take(sizeof(float) * 600 * (size_t)p->ln, p->nb);
    for (int b = 0; b < p->nb; b++) out[b] = kk_output{blk + 600 * p->a[b], 600 * p->nfr[b]};
    p->early_out = blk;
    p->early_issued = false;
    return blk;
}

int kk_plan_fetch(kk_plan* plan, kk_output* out, char* err, size_t errlen) {
    if (!plan || !out) return KK_ERR_INVALID;
    if (!plan->ctx) {
        set_err(err, errlen, "plan outlived its context");
        return KK_ERR_STATE;
    }
    for (int b = 0; b < plan->nb; b++) out[b] = kk_output{nullptr, 0};
    int rc = guard(err, errlen, [&] { fetch_plan(plan, out); });
    if (rc != KK_OK) kk_output_free(out, plan->nb);
    return rc;
}

int kk_plan_fetch_pcm16(kk_plan* plan, int16_t* const* dst, int64_t* clipped, char* err, size_t errlen) {
    if (!plan || !dst) return KK_ERR_INVALID;
    if (!plan->ctx) {
        set_err(err, errlen, "plan outlived its context");
        return KK_ERR_STATE;
    }
    return guard(err, errlen, [&] {
        use_device(plan->ctx);
        check(plan->kind != PLAN_SNAKE, "a snake plan has no audio");
        check(plan->last_until >= KK_STAGE_ALL, "plan has not run to the end");
        for (int b = 0; b < plan->nb; b++) check(dst[b] != nullptr, "null destination for item " + std::to_string(b));
        hipStream_t s = plan->ctx->stream;
        if (plan->kind == PLAN_FULL) drain_and_check_abort(plan);
        KK_HIP(launch_zero(plan->pcm_clip.p, (int64_t)plan->nb * 8, s));
        KK_HIP(launch_pcm16(plan->audio.as<float>(), plan->audio_start.as<int64_t>(), plan->pcm_len.as<int64_t>(),
                            plan->ist_item.as<int64_t>(), plan->ist_s0.as<int64_t>(), plan->n_ist,
                            plan->pcm.as<int16_t>(), plan->pcm_clip.as<unsigned long long>(), s));
        KK_HIP(hipStreamSynchronize(s));
        for (int b = 0; b < plan->nb; b++)
            KK_HIP(hipMemcpy(dst[b], plan->pcm.as<int16_t>() + 600 * plan->a[b], sizeof(int16_t) * 600 * plan->nfr[b],
                             hipMemcpyDeviceToHost));
        if (clipped) {
            std::vector<unsigned long long> c(plan->nb);
            KK_HIP(hipMemcpy(c.data(), plan->pcm_clip.p, sizeof(unsigned long long) * plan->nb, hipMemcpyDeviceToHost));
            for (int b = 0; b < plan->nb; b++) clipped[b] = (int64_t)c[b];
        }
    });
}

// Pinned host allocations made by kk_host_alloc: [base, base + bytes) by base.
static std::mutex g_pinned_mu;
static std::map<uintptr_t, size_t> g_pinned;

static bool is_pinned(const void* p, size_t bytes) {
    std::lock_guard<std::mutex> lock(g_pinned_mu);
    const uintptr_t a = (uintptr_t)p;
    auto it = g_pinned.upper_bound(a);
    if (it == g_pinned.begin()) return false;
    --it;
    return a >= it->first && a + bytes <= it->first + it->second;
}

int kk_host_alloc(kk_ctx* ctx, size_t bytes, void** out, char* err, size_t errlen) {
    if (!ctx || !out) return KK_ERR_INVALID;
    *out = nullptr;
    return guard(err, errlen, [&] {
        use_device(ctx);
        check(bytes > 0, "kk_host_alloc of 0 bytes");
        void* p = nullptr;
        KK_HIP(hipHostMalloc(&p, bytes, hipHostMallocDefault));
        std::lock_guard<std::mutex> lock(g_pinned_mu);
        g_pinned[(uintptr_t)p] = bytes;
        *out = p;
    });
}

void kk_host_free(void* p) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> lock(g_pinned_mu);
        auto it = g_pinned.find((uintptr_t)p);
        if (it == g_pinned.end()) return;  // not ours: left alone
        g_pinned.erase(it);
    }
    (void)hipHostFree(p);
}

int kk_plan_item_samples(const kk_plan* plan, int item, int64_t* offset, int64_t* count) {
    if (!plan || !offset || !count || item < 0 || item >= plan->nb || plan->kind == PLAN_SNAKE) return KK_ERR_INVALID;
    *offset = 600 * plan->a[item];
    *count = 600 * plan->nfr[item];
    return KK_OK;
}

// The PCM_16 encoding of the whole sample layout and its copies into pinned dst / clipped (or null).
static void enqueue_pcm16_fetch(kk_plan* plan, int16_t* dst, int64_t* clipped) {
    hipStream_t s = plan->ctx->stream;
    KK_HIP(launch_zero(plan->pcm_clip.p, (int64_t)plan->nb * 8, s));
    KK_HIP(launch_pcm16(plan->audio.as<float>(), plan->audio_start.as<int64_t>(), plan->pcm_len.as<int64_t>(),
                        plan->ist_item.as<int64_t>(), plan->ist_s0.as<int64_t>(), plan->n_ist, plan->pcm.as<int16_t>(),
                        plan->pcm_clip.as<unsigned long long>(), s));
    KK_HIP(hipMemcpyAsync(dst, plan->pcm.p, sizeof(int16_t) * 600 * (size_t)plan->ln, hipMemcpyDeviceToHost, s));
    if (clipped)
        KK_HIP(hipMemcpyAsync(clipped, plan->pcm_clip.p, sizeof(int64_t) * plan->nb, hipMemcpyDeviceToHost, s));
}

int kk_plan_fetch_pcm16_async(kk_plan* plan, int16_t* dst, int64_t* clipped, char* err, size_t errlen) {
    if (!plan || !dst) return KK_ERR_INVALID;
    if (!plan->ctx) {
        set_err(err, errlen, "plan outlived its context");
        return KK_ERR_STATE;
    }
    return guard(err, errlen, [&] {
        use_device(plan->ctx);
        check(plan->kind != PLAN_SNAKE, "a snake plan has no audio");
        check(plan->last_until >= KK_STAGE_ALL, "plan has not run to the end");
        check(!plan->fetch_pending, "the previous asynchronous fetch has not been waited for");
        const size_t pcm_bytes = sizeof(int16_t) * 600 * (size_t)plan->ln;
        check(is_pinned(dst, pcm_bytes), "dst must be " + std::to_string(pcm_bytes) +
                                             " bytes of pinned memory from kk_host_alloc");
        check(!clipped || is_pinned(clipped, sizeof(int64_t) * plan->nb),
              "clipped must be pinned memory from kk_host_alloc");
        hipStream_t s = plan->ctx->stream;
        if (!plan->fetch_ev) KK_HIP(hipEventCreateWithFlags(&plan->fetch_ev, hipEventDisableTiming));
        enqueue_pcm16_fetch(plan, dst, clipped);
        // ids-level plans: the run's abort flag comes back with the samples; kk_plan_fetch_wait checks it
        if (plan->kind == PLAN_FULL && plan->abort_host)
            KK_HIP(hipMemcpyAsync(plan->abort_host, plan->u_lstmx.p, sizeof(uint64_t), hipMemcpyDeviceToHost, s));
        KK_HIP(hipEventRecord(plan->fetch_ev, s));
        plan->fetch_dst = dst, plan->fetch_clipped = clipped;
        plan->fetch_pending = true;
    });
}

int kk_plan_fetch_wait(kk_plan* plan, char* err, size_t errlen) {
    if (!plan) return KK_ERR_INVALID;
    if (!plan->ctx) {
        set_err(err, errlen, "plan outlived its context");
        return KK_ERR_STATE;
    }
    return guard(err, errlen, [&] {
        if (!plan->fetch_pending) return;
        use_device(plan->ctx);
        plan->fetch_pending = false;
        KK_HIP(hipEventSynchronize(plan->fetch_ev));
        if (plan->kind == PLAN_FULL && plan->abort_host && *plan->abort_host != 0 && !plan->lstm_single) {
            // a two-CU pair of the run gave up: the run again on the one-CU recurrences (see
            // drain_and_check_abort), its samples into the same destination
            plan->lstm_single = true;
            run_plan(plan, plan->last_until);
            enqueue_pcm16_fetch(plan, plan->fetch_dst, plan->fetch_clipped);
            drain_aborted(plan);
        }
        if (plan->kind == PLAN_FULL) check_lstm_abort(plan);
    });
}

int kk_encode_pcm16(kk_ctx* ctx, const float* audio, int64_t n, int16_t* out, int64_t* clipped, char* err,
                    size_t errlen) {
    if (!ctx || n < 0 || (n > 0 && (!audio || !out))) return KK_ERR_INVALID;
    return guard(err, errlen, [&] {
        use_device(ctx);
        DevBuf a, o, len, clip;
        a.upload(audio, (size_t)n);
        o.alloc((size_t)n * sizeof(int16_t));
        const int64_t nn[1] = {n};
        len.upload(nn, 1);
        clip.alloc(sizeof(unsigned long long));
        KK_HIP(launch_zero(clip.p, 8, ctx->stream));
        KK_HIP(launch_pcm16(a.as<float>(), nullptr, len.as<int64_t>(), nullptr, nullptr, ceil_div(n, kIstftSamples),
                            o.as<int16_t>(), clip.as<unsigned long long>(), ctx->stream));
        KK_HIP(hipStreamSynchronize(ctx->stream));
        if (n) KK_HIP(hipMemcpy(out, o.p, sizeof(int16_t) * n, hipMemcpyDeviceToHost));
        unsigned long long c = 0;
        KK_HIP(hipMemcpy(&c, clip.p, sizeof(c), hipMemcpyDeviceToHost));
        if (clipped) *clipped = (int64_t)c;
    });
}

int kk_wav_header(int format, uint32_t sample_rate, uint64_t data_bytes, uint8_t* out, char* err, size_t errlen) {
    if (!out) return KK_ERR_INVALID;
    return guard(err, errlen, [&] {
        check(format == KK_WAV_PCM16 || format == KK_WAV_FLOAT32, "unknown WAV format");
        // check_riff_size (src/wav.rs:34-40): the RIFF size field is 36 + data in 32 bits
        check(data_bytes <= (uint64_t)UINT32_MAX - 36,
              "the audio (" + std::to_string(data_bytes) + " bytes) exceeds the 4 GiB limit of a WAV file");
        const uint16_t bits = format == KK_WAV_PCM16 ? 16 : 32, tag = format == KK_WAV_PCM16 ? 1 : 3;
        auto put = [&](int at, const void* v, int n) { std::memcpy(out + at, v, n); };
        auto u32 = [&](int at, uint32_t v) {
            for (int i = 0; i < 4; i++) out[at + i] = (uint8_t)(v >> (8 * i));
        };
        auto u16 = [&](int at, uint16_t v) { out[at] = (uint8_t)v, out[at + 1] = (uint8_t)(v >> 8); };
        put(0, "RIFF", 4);
        u32(4, (uint32_t)(36 + data_bytes));
        put(8, "WAVEfmt ", 8);
        u32(16, 16);
        u16(20, tag);
        u16(22, 1);
        u32(24, sample_rate);
        u32(28, sample_rate * bits / 8);
        u16(32, bits / 8);
        u16(34, bits);
        put(36, "data", 4);
        u32(40, (uint32_t)data_bytes);
    });
}

int kk_plan_tap(kk_plan* plan, const char* name, int item, float* dst, int64_t count, char* err, size_t errlen) {
    if (!plan || !name || !dst) return KK_ERR_INVALID;
    if (!plan->ctx) {
        set_err(err, errlen, "plan outlived its context");
        return KK_ERR_STATE;
    }
    return guard(err, errlen, [&] {
        use_device(plan->ctx);
        check(item >= 0 && item < plan->nb, "item out of range");
        check(plan->kind != PLAN_SNAKE, "snake plans have no taps");
        drain_and_check_abort(plan);
        const std::string n(name);
        const int64_t N = plan->nfr[item], a = plan->a[item];
        auto need = [&](int64_t c) { check(count == c, "tap " + n + " holds " + std::to_string(c) + " values"); };
        const bool full = plan->kind == PLAN_FULL;
        auto full_only = [&] { check(full, n + " exists in ids-level plans only"); };
        const int64_t T = full ? plan->ntok[item] : 0, ts = full ? plan->tstart[item] : 0;
        if (n == "bert") {
            full_only(), need(768 * T);
            tap_rows(plan->u_h.p, 768, ts, T, 768, dst);
        } else if (n == "d") {
            full_only(), need(640 * T);
            tap_rows(plan->u_x.p, 640, ts, T, 640, dst);
        } else if (n == "logits") {
            full_only(), need(50 * T);
            tap_rows(plan->u_logits.p, Runner::kLogitsLd, ts, T, 50, dst);
        } else if (n == "t_en") {
            full_only(), need(512 * T);
            tap_rows(plan->t_en.p, 512, ts, T, 512, dst);
        } else if (n == "shared") {
            full_only(), need(512 * N);
            tap_rows(plan->u_sh.p, 512, a, N, 512, dst);
        } else if (n == "f0" || n == "n") {
            full_only(), need(2 * N);
            KK_HIP(hipMemcpy(dst, (n == "f0" ? plan->f0 : plan->en).as<float>() + 2 * a, sizeof(float) * 2 * N,
                             hipMemcpyDeviceToHost));
        } else if (n == "asr") {
            check(plan->kind == PLAN_DECODER || full, "asr exists in decoder and ids-level plans only");
            need(512 * N);
            tap_rows(plan->xcat.p, kXcatLd, a, N, 512, dst);
        } else if (n == "decoder") {
            need(512 * 2 * N);
            tap_rows(plan->dec_out.p, 512, 2 * a, 2 * N, 512, dst);
        } else if (n == "har") {
            check(plan->tap_source, "tap har needs KOKORO_HIP_TEST_TAP_SOURCE=1 at plan creation");
            need(600 * N);
            KK_HIP(hipMemcpy(dst, plan->har.as<float>() + 600 * a, sizeof(float) * 600 * N, hipMemcpyDeviceToHost));
        } else if (n == "spec") {
            need(22 * (120 * N + 1));
            tap_rows(plan->spec.p, kSpecLd, 120 * a, 120 * N + 1, 22, dst);
        } else if (n == "gen0") {
            // stage 0's output as ups.1's bf16 operand (leaky ReLU 0.1 applied), widened to f32
            check(plan->last_until == KK_STAGE_GEN0, "gen0 is valid after a run until KK_STAGE_GEN0");
            need(256 * 20 * N);
            tap_rows_bf16(plan->B[2].p, 256, 20 * a, 20 * N, 256, dst);
        } else if (n == "post") {
            need(22 * (120 * N + 1));
            tap_rows(plan->post.p, kPostLd, 120 * a, 120 * N + 1, 22, dst);
        } else if (n == "audio") {
            need(600 * N);
            KK_HIP(hipMemcpy(dst, plan->audio.as<float>() + 600 * a, sizeof(float) * 600 * N, hipMemcpyDeviceToHost));
        } else {
            fail(KK_ERR_INVALID, "unknown tap " + n);
        }
    });
}

int kk_plan_get_info(const kk_plan* plan, kk_plan_info* info) {
    if (!plan || !info) return KK_ERR_INVALID;
    info->n_items = plan->nb;
    info->ln = plan->ln;
    int64_t fr = 0;
    for (auto v : plan->nfr) fr += v;
    info->frames = fr;
    info->samples = plan->kind == PLAN_SNAKE ? 0 : 600 * fr;
    info->conv_flop = plan->conv_flop;
    info->snake_flop = plan->snake_flop;
    info->device_bytes = plan->dev_bytes;
    info->launches = plan->launches;
    return KK_OK;
}

void kk_plan_free(kk_plan* plan) {
    if (!plan) return;
    if (plan->ctx) {  // an orphan's device memory went with its context (kk_close)
        (void)hipSetDevice(plan->ctx->device);
        (void)hipStreamSynchronize(plan->ctx->stream);
        // a run that failed between a fork and its join may leave work on the side streams
        for (auto ss : plan->ctx->side) (void)hipStreamSynchronize(ss);
        plan->drop_events();
        plan->ctx->plans.erase(plan);
    }
    delete plan;
}

int kk_forward_decoder_batch(kk_ctx* ctx, const kk_decoder_item* items, int n, kk_output* out, char* err,
                             size_t errlen) {
    if (!ctx || !out || n < 0) return KK_ERR_INVALID;
    for (int b = 0; b < n; b++) out[b] = kk_output{nullptr, 0};
    int rc = guard(err, errlen, [&] {
        use_device(ctx);
        // the one-shot plan is kept: its device buffers serve the next batch that fits
        if (!ctx->oneshot) {
            ctx->oneshot = new kk_plan();
            ctx->oneshot->ctx = ctx;
        }
        try {
            // KOKORO_HIP_TIMING=1: host-side phase times of this call on stderr (diagnostics)
            static const bool timing = env_i64("KOKORO_HIP_TIMING", 0) != 0;
            const auto t0 = std::chrono::steady_clock::now();
            init_decoder_plan(ctx->oneshot, items, n, true);
            float* blk = take_early_block(ctx->oneshot, out);
            const auto t1 = std::chrono::steady_clock::now();
            run_plan(ctx->oneshot, KK_STAGE_ALL);
            const auto t2 = std::chrono::steady_clock::now();
            if (timing) KK_HIP(hipStreamSynchronize(ctx->stream));
            const auto t3 = std::chrono::steady_clock::now();
            fetch_plan(ctx->oneshot, out, blk);
            ctx->oneshot->early_out = nullptr;
            const auto t4 = std::chrono::steady_clock::now();
            if (timing) {
                auto ms = [](auto a, auto b) { return std::chrono::duration<double, std::milli>(b - a).count(); };
                std::fprintf(stderr, "kk_forward_decoder_batch: plan %.3f ms (staged %.2f MB), enqueue %.3f ms, "
                             "device %.3f ms, fetch %.3f ms\n", ms(t0, t1), ctx->stage.used / 1e6, ms(t1, t2),
                             ms(t2, t3), ms(t3, t4));
            }
        } catch (...) {
            // a failure (device memory exhausted above all) releases the cached buffers, so that a
            // caller splitting the batch (src/engine.rs:229-234) has the whole device again
            drop_oneshot(ctx);
            throw;
        }
    });
    if (rc != KK_OK) kk_output_free(out, n);
    return rc;
}

int kk_forward_batch(kk_ctx* ctx, const kk_item* items, int n, kk_result* out, char* err, size_t errlen) {
    if (!ctx || !out || n < 0) return KK_ERR_INVALID;
    for (int b = 0; b < n; b++) out[b] = kk_result{nullptr, 0, nullptr, 0};
    std::vector<kk_output> audio(std::max(n, 0), kk_output{nullptr, 0});
    int rc = guard(err, errlen, [&] {
        use_device(ctx);
        if (!ctx->oneshot) {
            ctx->oneshot = new kk_plan();
            ctx->oneshot->ctx = ctx;
        }
        try {
            static const bool timing = env_i64("KOKORO_HIP_TIMING", 0) != 0;
            const auto t0 = std::chrono::steady_clock::now();
            init_full_plan(ctx->oneshot, items, n);  // the token phase runs here
            float* blk = take_early_block(ctx->oneshot, audio.data());
            const auto t1 = std::chrono::steady_clock::now();
            run_plan(ctx->oneshot, KK_STAGE_ALL, true);
            if (timing) KK_HIP(hipStreamSynchronize(ctx->stream));
            const auto t2 = std::chrono::steady_clock::now();
            fetch_plan(ctx->oneshot, audio.data(), blk);
            ctx->oneshot->early_out = nullptr;
            for (int b = 0; b < n; b++) {
                const auto& d = ctx->oneshot->pred[b];
                out[b].pred_dur = (int64_t*)std::malloc(sizeof(int64_t) * d.size());
                if (!out[b].pred_dur) throw std::bad_alloc();
                std::memcpy(out[b].pred_dur, d.data(), sizeof(int64_t) * d.size());
                out[b].n_tok = (int32_t)d.size();
            }
            for (int b = 0; b < n; b++) out[b].audio = audio[b].audio, out[b].n_samples = audio[b].n_samples;
            const auto t3 = std::chrono::steady_clock::now();
            if (timing) {
                auto ms = [](auto a, auto b) { return std::chrono::duration<double, std::milli>(b - a).count(); };
                std::fprintf(stderr, "kk_forward_batch: tokens + durations %.3f ms, frames %.3f ms, fetch %.3f ms\n",
                             ms(t0, t1), ms(t1, t2), ms(t2, t3));
            }
        } catch (...) {
            drop_oneshot(ctx);
            throw;
        }
    });
    if (rc != KK_OK) {
        kk_output_free(audio.data(), n);
        for (int b = 0; b < n; b++) {
            std::free(out[b].pred_dur);
            out[b] = kk_result{nullptr, 0, nullptr, 0};
        }
    }
    return rc;
}

void kk_result_free(kk_result* out, int n) {
    if (!out) return;
    for (int b = 0; b < n; b++) {
        kk_output o{out[b].audio, out[b].n_samples};
        kk_output_free(&o, 1);
        std::free(out[b].pred_dur);
        out[b] = kk_result{nullptr, 0, nullptr, 0};
    }
}

void kk_output_free(kk_output* out, int n) {
    if (!out) return;
    for (int b = 0; b < n; b++) {
        if (out[b].audio && !out_block_release(out[b].audio)) std::free(out[b].audio);
        out[b].audio = nullptr;
        out[b].n_samples = 0;
    }
}

int kk_set_profiling(kk_ctx* ctx, int on) {
    if (!ctx) return KK_ERR_INVALID;
    ctx->profiling = on != 0;
    return KK_OK;
}

int kk_profile_read(kk_ctx* ctx, kk_profile_entry* out, int max, int* n_out, char* err, size_t errlen) {
    if (!ctx || !out || !n_out) return KK_ERR_INVALID;
    return guard(err, errlen, [&] {
        use_device(ctx);
        KK_HIP(hipStreamSynchronize(ctx->stream));
        kk_profile_entry acc[PC_COUNT];
        for (int i = 0; i < PC_COUNT; i++) {
            std::memset(&acc[i], 0, sizeof(acc[i]));
            std::snprintf(acc[i].name, sizeof(acc[i].name), "%s", kProfNames[i]);
        }
        for (auto& r : ctx->prof) {
            float ms = 0.f;
            KK_HIP(hipEventElapsedTime(&ms, r.e0, r.e1));
            acc[r.cls].launches++;
            acc[r.cls].ms += ms;
            acc[r.cls].flop += r.flop;
            acc[r.cls].bytes += r.bytes;
            ctx->event_pool.push_back(r.e0);
            ctx->event_pool.push_back(r.e1);
        }
        ctx->prof.clear();
        int k = 0;
        for (int i = 0; i < PC_COUNT && k < max; i++)
            if (acc[i].launches > 0) out[k++] = acc[i];
        *n_out = k;
    });
}

int kk_profile_launches(kk_ctx* ctx, kk_launch_record* out, int max, int* n_out, char* err, size_t errlen) {
    if (!ctx || (!out && max > 0) || !n_out) return KK_ERR_INVALID;
    return guard(err, errlen, [&] {
        use_device(ctx);
        KK_HIP(hipStreamSynchronize(ctx->stream));
        int k = 0;
        for (auto& r : ctx->prof) {
            if (k < max) {
                kk_launch_record& o = out[k];
                std::memset(&o, 0, sizeof(o));
                std::snprintf(o.name, sizeof(o.name), "%s", r.label.c_str());
                std::snprintf(o.cls, sizeof(o.cls), "%s", kProfNames[r.cls]);
                float ms = 0.f;
                KK_HIP(hipEventElapsedTime(&ms, r.e0, r.e1));
                o.ms = ms, o.flop = r.flop, o.bytes = r.bytes;
            }
            k++;
        }
        *n_out = k;
    });
}

}  // extern "C"
