"""Independent torch-CPU restatement of the decoder + iSTFTNet generator, built from library routines
(F.conv1d, F.conv_transpose1d, F.instance_norm, F.interpolate, torch.stft / torch.istft), in float64.

Test infrastructure: it pins the C oracle (oracle/kk_oracle.c) from a second, structurally different
implementation that follows the upstream model definition the reference restates (StyleTTS2
AdainResBlk1d / iSTFTNet AdaINResBlock1, SineGen, TorchSTFT; docs/truth-pack/OQ_INDEX.md OQ-8,
OQ-9), so a wrong padding, dilation, weight orientation or op order in the oracle shows up here.
In float32 (set_dtype) it is also the torch-CPU functional baseline that bench.py times beside the
GPU: the op sequence upstream kokoro runs on a CPU, one item at a time.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

DT = torch.float64


def set_dtype(dt):
    """Arithmetic type of every op below (float64 to pin the oracle, float32 for the CPU baseline)."""
    global DT
    DT = dt


def T(a):
    return torch.as_tensor(np.asarray(a), dtype=DT)


ROUND_OPERANDS = False
ROUND_ONLY = None  # with ROUND_OPERANDS: None (every layer) or the layer-name prefixes that round
ROUND_EXCEPT = ()  # layer-name prefixes that do not round
ROUND_FP16 = ()    # layer-name prefixes that round to fp16 instead of bf16


class bf16_operands:
    """Within: conv() and linear() round their input and weight to bf16 first (the GPU's MFMA
    operands, and the reference's GLinear / BF16 convs, src/gpu.rs:280-301), accumulating in DT.
    only / skip / fp16: layer-name prefixes that select where it rounds (for measurements of which
    rounding points matter)."""

    def __init__(self, only=None, skip=(), fp16=()):
        self.only, self.skip, self.fp16 = only, tuple(skip), tuple(fp16)

    def __enter__(self):
        global ROUND_OPERANDS, ROUND_ONLY, ROUND_EXCEPT, ROUND_FP16
        ROUND_OPERANDS, ROUND_ONLY, ROUND_EXCEPT, ROUND_FP16 = True, self.only, self.skip, self.fp16

    def __exit__(self, *a):
        global ROUND_OPERANDS, ROUND_ONLY, ROUND_EXCEPT, ROUND_FP16
        ROUND_OPERANDS, ROUND_ONLY, ROUND_EXCEPT, ROUND_FP16 = False, None, (), ()


def _rb(t, prefix=""):
    if not ROUND_OPERANDS or prefix.startswith(ROUND_EXCEPT or ("\0",)):
        return t
    if ROUND_ONLY is not None and not prefix.startswith(tuple(ROUND_ONLY)):
        return t
    fmt = torch.float16 if ROUND_FP16 and prefix.startswith(ROUND_FP16) else torch.bfloat16
    return t.to(torch.float32).to(fmt).to(DT)


def conv(w, prefix, x, stride=1, pad=0, dil=1, bias=True):
    b = T(w[prefix + ".bias"]) if bias else None
    return F.conv1d(_rb(x, prefix)[None], _rb(T(w[prefix + ".weight"]), prefix), b, stride=stride, padding=pad,
                    dilation=dil)[0]


def adain(w, prefix, x, s):
    """AdaIN1d: (1 + gamma) * InstanceNorm1d(affine)(x) + beta, gamma/beta = fc(s)."""
    c = x.shape[0]
    h = F.linear(T(s[:128]), T(w[prefix + ".fc.weight"]), T(w[prefix + ".fc.bias"]))
    n = F.instance_norm(x[None], weight=T(w[prefix + ".norm.weight"]), bias=T(w[prefix + ".norm.bias"]), eps=1e-5)[0]
    return (1 + h[:c, None]) * n + h[c:, None]


def resblk(w, p, x, s, upsample=False):
    """StyleTTS2 AdainResBlk1d: (residual + shortcut) / sqrt(2)."""
    din = x.shape[0]
    r = F.leaky_relu(adain(w, p + ".norm1", x, s), 0.2)
    if upsample:
        r = F.conv_transpose1d(r[None], T(w[p + ".pool.weight"]), T(w[p + ".pool.bias"]), stride=2, padding=1,
                               output_padding=1, groups=din)[0]
    r = conv(w, p + ".conv1", r, pad=1)
    r = F.leaky_relu(adain(w, p + ".norm2", r, s), 0.2)
    r = conv(w, p + ".conv2", r, pad=1)
    sc = x
    if upsample:
        sc = F.interpolate(sc[None], scale_factor=2, mode="nearest")[0]
    if p + ".conv1x1.weight" in w:
        sc = conv(w, p + ".conv1x1", sc, bias=False)
    return (r + sc) / math.sqrt(2)


def snake_block(w, p, x, s):
    """iSTFTNet AdaINResBlock1 with Snake activations, dilations 1, 3, 5."""
    k = w[p + ".convs1.0.weight"].shape[2]
    for i, d in enumerate((1, 3, 5)):
        a1 = T(w[f"{p}.alpha1.{i}"]).reshape(-1, 1)
        a2 = T(w[f"{p}.alpha2.{i}"]).reshape(-1, 1)
        xt = adain(w, f"{p}.adain1.{i}", x, s)
        xt = xt + (1 / a1) * torch.sin(a1 * xt) ** 2
        xt = conv(w, f"{p}.convs1.{i}", xt, pad=(k * d - d) // 2, dil=d)
        xt = adain(w, f"{p}.adain2.{i}", xt, s)
        xt = xt + (1 / a2) * torch.sin(a2 * xt) ** 2
        xt = conv(w, f"{p}.convs2.{i}", xt, pad=(k - 1) // 2)
        x = xt + x
    return x


def decoder(w, asr, f0, en, s):
    asr, f0, en = T(asr), T(f0), T(en)
    f0n = conv(w, "decoder.F0_conv", f0[None], stride=2, pad=1)
    nn_ = conv(w, "decoder.N_conv", en[None], stride=2, pad=1)
    x = resblk(w, "decoder.encode", torch.cat([asr, f0n, nn_]), s)
    ar = conv(w, "decoder.asr_res.0", asr)
    for i in range(4):
        x = resblk(w, f"decoder.decode.{i}", torch.cat([x, ar, f0n, nn_]), s, upsample=i == 3)
    return x


def sine_source(w, f0c, rand_ini, noise):
    """SineGen._f02sine + SourceModuleHnNSF with the reference's fixed noise (9 harmonics, sr 24 kHz,
    upsample 300, sine_amp 0.1, noise_std 0.003, voiced threshold 10)."""
    f0c = T(f0c)
    l = f0c.shape[0]
    s = 300 * l
    f0_up = F.interpolate(f0c[None, None], scale_factor=300, mode="nearest")[0, 0]  # [S]
    harm = torch.arange(1, 10, dtype=DT)
    rad = torch.remainder(f0_up[:, None] * harm[None, :] / 24000.0, 1.0)  # [S, 9]
    ri = T(rand_ini).clone()
    ri[0] = 0
    rad[0, :] = rad[0, :] + ri
    rad_d = F.interpolate(rad.T[None], scale_factor=1 / 300, mode="linear", align_corners=False)[0].T  # [L, 9]
    phase = torch.cumsum(rad_d, dim=0) * 2 * math.pi
    phase = F.interpolate(phase.T[None] * 300, scale_factor=300, mode="linear", align_corners=False)[0].T  # [S, 9]
    sines = torch.sin(phase) * 0.1
    uv = (f0_up > 10).to(DT)[:, None]
    noise_amp = uv * 0.003 + (1 - uv) * 0.1 / 3
    sw = sines * uv + noise_amp * T(noise).reshape(s, 9)
    lw = T(w["decoder.generator.m_source.l_linear.weight"]).reshape(9)
    lb = T(w["decoder.generator.m_source.l_linear.bias"]).reshape(())
    return torch.tanh(sw @ lw + lb)


def stft(x):
    """TorchSTFT.transform: n_fft 20, hop 5, periodic Hann, center, reflect -> (magnitude, phase)."""
    win = torch.hann_window(20, periodic=True, dtype=DT)
    X = torch.stft(T(x), n_fft=20, hop_length=5, win_length=20, window=win, center=True, pad_mode="reflect",
                   return_complex=True)
    return X.abs(), torch.angle(X)


def istft(post):
    """exp(magnitude), sin(phase), then torch.istft (TorchSTFT.inverse)."""
    post = T(post)
    mag = torch.exp(post[:11])
    ph = torch.sin(post[11:])
    win = torch.hann_window(20, periodic=True, dtype=DT)
    return torch.istft(mag * torch.exp(1j * ph), n_fft=20, hop_length=5, win_length=20, window=win, center=True)


def generator(w, x, f0, s, rand_ini, noise, taps=None, spec=None):
    """Generator forward; `spec` overrides the source + STFT output (to pin the glue separately
    from the ill-conditioned phases of near-zero STFT bins)."""
    g = "decoder.generator"
    x = T(x)
    if spec is None:
        har = sine_source(w, f0, rand_ini, noise)
        mag, ph = stft(har)
        spec = torch.cat([mag, ph])  # [22, 120N + 1]
    else:
        spec = T(spec)
    if taps is not None:
        taps["spec"] = spec
    for i in range(2):
        x = F.leaky_relu(x, 0.1)
        if i == 0:
            xs = conv(w, f"{g}.noise_convs.0", spec, stride=6, pad=3)
        else:
            xs = conv(w, f"{g}.noise_convs.1", spec)
        xs = snake_block(w, f"{g}.noise_res.{i}", xs, s)
        stride, pad = (10, 5) if i == 0 else (6, 3)
        x = F.conv_transpose1d(x[None], T(w[f"{g}.ups.{i}.weight"]), T(w[f"{g}.ups.{i}.bias"]), stride=stride,
                               padding=pad)[0]
        if i == 1:
            x = F.pad(x[None], (1, 0), mode="reflect")[0]
        x = x + xs
        acc = None
        for j in range(3):
            r = snake_block(w, f"{g}.resblocks.{3 * i + j}", x, s)
            acc = r if acc is None else acc + r
        x = acc / 3
        if taps is not None:
            taps[f"gen{i}"] = x
    x = F.leaky_relu(x, 0.01)
    post = conv(w, f"{g}.conv_post", x, pad=3)
    if taps is not None:
        taps["post"] = post
    return istft(post)


# ------------------------------------------------------------------ upstream stages (ids -> F0, N, t_en)
# The reference runs these on its GPU engine (src/gpu_batch.rs:179-297); the host-side pieces are the
# ALBERT embedding lookup (src/albert.rs:70-81) and the duration rounding (src/model.rs:90-100).

HEADS, HEAD_DIM = 12, 64


def linear(w, prefix, x):
    """Linear on row-major x [t, din] (src/nn.rs:7-23; GLinear::fwd src/gpu.rs:280-301)."""
    b = T(w[prefix + ".bias"]) if prefix + ".bias" in w else None
    return F.linear(_rb(x, prefix), _rb(T(w[prefix + ".weight"]), prefix), b)


def gelu_new(x):
    """kernels/kokoro.cu:84-90: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    return 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))


def albert_embeddings(w, ids):
    """Albert::embeddings (src/albert.rs:70-81): (word + token_type[0]) + position, LayerNorm 1e-12."""
    ids = torch.as_tensor(np.asarray(ids, np.int64))
    e = (T(w["bert.embeddings.word_embeddings.weight"])[ids] + T(w["bert.embeddings.token_type_embeddings.weight"])[0])
    e = e + T(w["bert.embeddings.position_embeddings.weight"])[: len(ids)]
    return F.layer_norm(e, (e.shape[1],), T(w["bert.embeddings.LayerNorm.weight"]),
                        T(w["bert.embeddings.LayerNorm.bias"]), eps=1e-12)


def albert(w, ids):
    """albert_b (src/gpu_batch.rs:423-455): one shared post-LN layer applied 12 times; per head
    softmax(q k^T / 8) v over the item's own tokens (src/gpu_batch.rs:433-441)."""
    L = "bert.encoder.albert_layer_groups.0.albert_layers.0"
    h = linear(w, "bert.encoder.embedding_hidden_mapping_in", albert_embeddings(w, ids))
    t = h.shape[0]
    for _ in range(12):
        q, k, v = (linear(w, f"{L}.attention.{n}", h).reshape(t, HEADS, HEAD_DIM).transpose(0, 1)
                   for n in ("query", "key", "value"))
        p = torch.softmax(q @ k.transpose(1, 2) * HEAD_DIM ** -0.5, dim=-1)   # [heads, t, t]
        ctx = (p @ v).transpose(0, 1).reshape(t, HEADS * HEAD_DIM)
        a = F.layer_norm(linear(w, f"{L}.attention.dense", ctx) + h, (h.shape[1],),
                         T(w[f"{L}.attention.LayerNorm.weight"]), T(w[f"{L}.attention.LayerNorm.bias"]), eps=1e-12)
        f = gelu_new(linear(w, f"{L}.ffn", a))
        h = F.layer_norm(linear(w, f"{L}.ffn_output", f) + a, (h.shape[1],),
                         T(w[f"{L}.full_layer_layer_norm.weight"]), T(w[f"{L}.full_layer_layer_norm.bias"]), eps=1e-12)
    return h


def lstm_dir(w, prefix, sfx, x, reverse):
    """One direction of torch.nn.LSTM (gates i, f, g, o; lstm_seq_batched kernels/kokoro.cu:404-455:
    gate = (W_ih x + b_ih) + (W_hh h + b_hh), c = f c + i g, h = o tanh(c))."""
    wih, whh = T(w[f"{prefix}.weight_ih_l0{sfx}"]), T(w[f"{prefix}.weight_hh_l0{sfx}"])
    bih, bhh = T(w[f"{prefix}.bias_ih_l0{sfx}"]), T(w[f"{prefix}.bias_hh_l0{sfx}"])
    hd = whh.shape[1]
    gx = F.linear(_rb(x, prefix), _rb(wih, prefix), bih)  # W_ih on the GLinear route (bf16 operands on the GPU)
    h = torch.zeros(hd, dtype=DT)
    c = torch.zeros(hd, dtype=DT)
    out = torch.zeros(x.shape[0], hd, dtype=DT)
    order = range(x.shape[0] - 1, -1, -1) if reverse else range(x.shape[0])
    for t in order:
        g = gx[t] + (whh @ h + bhh)
        i, f, gg, o = torch.sigmoid(g[:hd]), torch.sigmoid(g[hd:2 * hd]), torch.tanh(g[2 * hd:3 * hd]), torch.sigmoid(g[3 * hd:])
        c = f * c + i * gg
        h = o * torch.tanh(c)
        out[t] = h
    return out


def bilstm(w, prefix, x):
    """BiLstm (src/nn.rs:168-190): [t, din] -> [t, 2H], forward then reverse direction."""
    return torch.cat([lstm_dir(w, prefix, "", x, False), lstm_dir(w, prefix, "_reverse", x, True)], dim=1)


def text_encoder(w, ids):
    """text_encoder_b (src/gpu_batch.rs:457-481): embedding, 3 x (Conv1d k5 p2, LayerNorm over the
    channels with gamma / beta eps 1e-5, leaky ReLU 0.2), BiLSTM.  Returns t_en [t, 512]."""
    ids = torch.as_tensor(np.asarray(ids, np.int64))
    x = T(w["text_encoder.embedding.weight"])[ids].T  # [512, t]
    for i in range(3):
        y = conv(w, f"text_encoder.cnn.{i}.0", x, pad=2).T  # [t, 512]
        y = F.layer_norm(y, (y.shape[1],), T(w[f"text_encoder.cnn.{i}.1.gamma"]), T(w[f"text_encoder.cnn.{i}.1.beta"]),
                         eps=1e-5)
        x = F.leaky_relu(y, 0.2).T
    return bilstm(w, "text_encoder.lstm", x.T)


def ada_layer_norm(w, prefix, h, s):
    """adaln_rows_seg (kernels/kokoro.cu:337-373): (1 + gamma) LayerNorm(h) + beta, eps 1e-5, no
    affine; gamma, beta = fc(s) (src/gpu_batch.rs:225-231)."""
    gb = F.linear(T(s), T(w[prefix + ".weight"]), T(w[prefix + ".bias"]))
    d = h.shape[1]
    return (1 + gb[:d]) * F.layer_norm(h, (d,), eps=1e-5) + gb[d:]


def duration_encoder(w, d_en, s_pro):
    """src/gpu_batch.rs:216-233: x = [d_en | s]; 3 x (BiLSTM, AdaLayerNorm, [h | s]).  [t, 640]."""
    s = T(s_pro)
    srow = s[None].expand(d_en.shape[0], -1)
    x = torch.cat([d_en, srow], dim=1)
    for i in range(3):
        h = bilstm(w, f"predictor.text_encoder.lstms.{2 * i}", x)
        h = ada_layer_norm(w, f"predictor.text_encoder.lstms.{2 * i + 1}.fc", h, s)
        x = torch.cat([h, srow], dim=1)
    return x


def durations(logits, speed):
    """durations_from_logits (src/model.rs:90-100): round-half-even(sum sigmoid / speed), >= 1."""
    s = torch.sigmoid(torch.as_tensor(logits, dtype=DT)).sum(dim=1) / speed
    return np.maximum(np.round(s.numpy()).astype(np.int64), 1)


def f0n(w, d, dur, s_pro, taps=None):
    """src/gpu_batch.rs:265-294: en = d's rows repeated by the durations, shared BiLSTM, then the F0
    and N stacks (AdainResBlk1d 512->512, 512->256 upsampled, 256->256; Conv1d k1 -> 1) at 2N."""
    src = np.repeat(np.arange(len(dur)), dur)
    en = d[torch.as_tensor(src)]
    sh = bilstm(w, "predictor.shared", en)
    if taps is not None:
        taps["shared"] = sh
    return f0n_stacks(w, sh, s_pro)


def f0n_stacks(w, sh, s_pro):
    """The F0 and N stacks on the shared LSTM's output sh [N, 512] (src/gpu_batch.rs:282-292)."""
    sh = torch.as_tensor(sh, dtype=DT).T  # [512, N]
    out = []
    for name in ("F0", "N"):
        h = resblk(w, f"predictor.{name}.0", sh, s_pro)
        h = resblk(w, f"predictor.{name}.1", h, s_pro, upsample=True)
        h = resblk(w, f"predictor.{name}.2", h, s_pro)
        out.append(conv(w, f"predictor.{name}_proj", h)[0])
    return out[0], out[1]


def upstream(w, ids, ref_s, speed=1.0, taps=None, dur=None):
    """forward_batch up to the decoder for one item (src/gpu_batch.rs:179-297): returns
    (durations, t_en [512, t], F0 [2N], N [2N]); `dur` overrides the predicted durations."""
    ref_s = np.asarray(ref_s)
    s_pro = ref_s[128:]
    bert = albert(w, ids)
    d_en = linear(w, "bert_encoder", bert)
    d = duration_encoder(w, d_en, s_pro)
    xl = bilstm(w, "predictor.lstm", d)
    logits = linear(w, "predictor.duration_proj.linear_layer", xl)
    pred = durations(logits, speed) if dur is None else np.asarray(dur, np.int64)
    f0, n = f0n(w, d, pred, s_pro, taps)
    t_en = text_encoder(w, ids)
    if taps is not None:
        taps.update(bert=bert, d_en=d_en, d=d, xl=xl, logits=logits, t_en=t_en, f0=f0, n=n)
    return pred, t_en.T, f0, n
