"""Tensor inventory of the Kokoro-82M decoder + iSTFTNet generator and its seeded random init.

Names follow the checkpoint's state-dict keys with weight_norm already resolved, exactly as the
reference's host structs hold them after `Weights::conv_weight` (src/weights.rs:62-70).  Shapes
follow `Decoder::load` / `Generator::load` (src/vocoder.rs:54-111) and the layer loaders of
src/nn.rs:25-166.

Random init (no checkpoint is available offline): every tensor is drawn from its own stream,
seeded by (base seed, FNV-1a of its name), so a tensor's values do not depend on which other
tensors exist.
- Conv1d / Linear weights and biases: U(-1/sqrt(fan_in), 1/sqrt(fan_in)), fan_in = Cin * k.
- ConvTranspose1d: fan_in = Cin * k / stride (the number of inputs each output sums).
- InstanceNorm affine: weight U(0.8, 1.2), bias U(-0.1, 0.1) (non-identity so that the affine
  path is exercised; the reference applies it, docs/truth-pack/OQ_INDEX.md:17 OQ-8).
- Snake alpha: U(0.5, 1.5).
- conv_post scaled by 0.1 so exp(magnitude) stays O(1).
"""
from __future__ import annotations

import numpy as np

STYLE_DIM = 128
HIDDEN = 512
GEN = "decoder.generator"
KERNELS = (3, 7, 11)
DILATIONS = (1, 3, 5)


def _conv(spec, prefix, cin, cout, k, bias=True, kind="conv", stride=1):
    spec.append((f"{prefix}.weight", (cout, cin, k), kind, cin * k))
    if bias:
        spec.append((f"{prefix}.bias", (cout,), kind, cin * k))


def _adain(spec, prefix, c):
    spec.append((f"{prefix}.fc.weight", (2 * c, STYLE_DIM), "conv", STYLE_DIM))
    spec.append((f"{prefix}.fc.bias", (2 * c,), "conv", STYLE_DIM))
    spec.append((f"{prefix}.norm.weight", (c,), "norm_w", 0))
    spec.append((f"{prefix}.norm.bias", (c,), "norm_b", 0))


def _resblk(spec, prefix, din, dout, upsample):
    """AdainResBlk1d::load (src/nn.rs:119-140)."""
    _conv(spec, f"{prefix}.conv1", din, dout, 3)
    _conv(spec, f"{prefix}.conv2", dout, dout, 3)
    _adain(spec, f"{prefix}.norm1", din)
    _adain(spec, f"{prefix}.norm2", dout)
    if din != dout:
        _conv(spec, f"{prefix}.conv1x1", din, dout, 1, bias=False)
    if upsample:
        spec.append((f"{prefix}.pool.weight", (din, 1, 3), "conv", 3))
        spec.append((f"{prefix}.pool.bias", (din,), "conv", 3))


def _snake(spec, prefix, c, k):
    """AdaInResBlock1::load (src/nn.rs:154-165)."""
    for i in range(3):
        _conv(spec, f"{prefix}.convs1.{i}", c, c, k)
        _conv(spec, f"{prefix}.convs2.{i}", c, c, k)
        _adain(spec, f"{prefix}.adain1.{i}", c)
        _adain(spec, f"{prefix}.adain2.{i}", c)
        spec.append((f"{prefix}.alpha1.{i}", (1, c, 1), "alpha", 0))
        spec.append((f"{prefix}.alpha2.{i}", (1, c, 1), "alpha", 0))


def tensor_spec():
    """[(name, shape, init kind, fan_in)] for the decoder + generator."""
    spec = []
    _resblk(spec, "decoder.encode", 514, 1024, False)
    for i in range(3):
        _resblk(spec, f"decoder.decode.{i}", 1090, 1024, False)
    _resblk(spec, "decoder.decode.3", 1090, 512, True)
    _conv(spec, "decoder.F0_conv", 1, 1, 3)
    _conv(spec, "decoder.N_conv", 1, 1, 3)
    _conv(spec, "decoder.asr_res.0", 512, 64, 1)
    spec.append((f"{GEN}.m_source.l_linear.weight", (1, 9), "conv", 9))
    spec.append((f"{GEN}.m_source.l_linear.bias", (1,), "conv", 9))
    _conv(spec, f"{GEN}.noise_convs.0", 22, 256, 12)
    _conv(spec, f"{GEN}.noise_convs.1", 22, 128, 1)
    _snake(spec, f"{GEN}.noise_res.0", 256, 7)
    _snake(spec, f"{GEN}.noise_res.1", 128, 11)
    # ConvTranspose1d weights are [Cin, Cout, K] (src/nn.rs:184-195)
    spec.append((f"{GEN}.ups.0.weight", (512, 256, 20), "convt", 512 * 20 // 10))
    spec.append((f"{GEN}.ups.0.bias", (256,), "convt", 512 * 20 // 10))
    spec.append((f"{GEN}.ups.1.weight", (256, 128, 12), "convt", 256 * 12 // 6))
    spec.append((f"{GEN}.ups.1.bias", (128,), "convt", 256 * 12 // 6))
    for i in range(6):
        _snake(spec, f"{GEN}.resblocks.{i}", 256 if i < 3 else 128, KERNELS[i % 3])
    _conv(spec, f"{GEN}.conv_post", 128, 22, 7, kind="post")
    return spec


# ------------------------------------------------------------------ upstream stages
N_TOKEN = 178
ALBERT_EMB, ALBERT_HID, ALBERT_FFN, ALBERT_POS = 128, 768, 2048, 512
ALBERT_LAYER = "bert.encoder.albert_layer_groups.0.albert_layers.0"
LSTM_H = 256
MAX_DUR = 50


def _linear(spec, prefix, din, dout, bias=True, kind="conv"):
    spec.append((f"{prefix}.weight", (dout, din), kind, din))
    if bias:
        spec.append((f"{prefix}.bias", (dout,), kind, din))


def _lstm(spec, prefix, din, h=LSTM_H):
    """BiLstm::load (src/nn.rs:178-189): torch.nn.LSTM names, gate order i, f, g, o."""
    for sfx in ("", "_reverse"):
        spec.append((f"{prefix}.weight_ih_l0{sfx}", (4 * h, din), "lstm", h))
        spec.append((f"{prefix}.weight_hh_l0{sfx}", (4 * h, h), "lstm", h))
        spec.append((f"{prefix}.bias_ih_l0{sfx}", (4 * h,), "lstm", h))
        spec.append((f"{prefix}.bias_hh_l0{sfx}", (4 * h,), "lstm", h))


def upstream_spec():
    """[(name, shape, init kind, fan_in)] for ALBERT, bert_encoder, the text encoder and the prosody
    predictor (src/albert.rs:36-67, src/model.rs:21-88, src/model.rs:122-141)."""
    spec = []
    spec.append(("bert.embeddings.word_embeddings.weight", (N_TOKEN, ALBERT_EMB), "emb", 0))
    spec.append(("bert.embeddings.position_embeddings.weight", (ALBERT_POS, ALBERT_EMB), "emb", 0))
    spec.append(("bert.embeddings.token_type_embeddings.weight", (2, ALBERT_EMB), "emb", 0))
    spec.append(("bert.embeddings.LayerNorm.weight", (ALBERT_EMB,), "norm_w", 0))
    spec.append(("bert.embeddings.LayerNorm.bias", (ALBERT_EMB,), "norm_b", 0))
    _linear(spec, "bert.encoder.embedding_hidden_mapping_in", ALBERT_EMB, ALBERT_HID)
    for nm in ("query", "key", "value", "dense"):
        _linear(spec, f"{ALBERT_LAYER}.attention.{nm}", ALBERT_HID, ALBERT_HID)
    spec.append((f"{ALBERT_LAYER}.attention.LayerNorm.weight", (ALBERT_HID,), "norm_w", 0))
    spec.append((f"{ALBERT_LAYER}.attention.LayerNorm.bias", (ALBERT_HID,), "norm_b", 0))
    _linear(spec, f"{ALBERT_LAYER}.ffn", ALBERT_HID, ALBERT_FFN)
    _linear(spec, f"{ALBERT_LAYER}.ffn_output", ALBERT_FFN, ALBERT_HID)
    spec.append((f"{ALBERT_LAYER}.full_layer_layer_norm.weight", (ALBERT_HID,), "norm_w", 0))
    spec.append((f"{ALBERT_LAYER}.full_layer_layer_norm.bias", (ALBERT_HID,), "norm_b", 0))
    _linear(spec, "bert_encoder", ALBERT_HID, HIDDEN)
    # text encoder (src/model.rs:29-44)
    spec.append(("text_encoder.embedding.weight", (N_TOKEN, HIDDEN), "emb", 0))
    for i in range(3):
        _conv(spec, f"text_encoder.cnn.{i}.0", HIDDEN, HIDDEN, 5)
        spec.append((f"text_encoder.cnn.{i}.1.gamma", (HIDDEN,), "norm_w", 0))
        spec.append((f"text_encoder.cnn.{i}.1.beta", (HIDDEN,), "norm_b", 0))
    _lstm(spec, "text_encoder.lstm", HIDDEN)
    # prosody predictor (src/model.rs:60-88)
    cin = HIDDEN + STYLE_DIM
    for i in range(3):
        _lstm(spec, f"predictor.text_encoder.lstms.{2 * i}", cin)
        _linear(spec, f"predictor.text_encoder.lstms.{2 * i + 1}.fc", STYLE_DIM, 2 * HIDDEN)
    _lstm(spec, "predictor.lstm", cin)
    spec.append(("predictor.duration_proj.linear_layer.weight", (MAX_DUR, HIDDEN), "dur_w", HIDDEN))
    spec.append(("predictor.duration_proj.linear_layer.bias", (MAX_DUR,), "dur_bias", 0))
    _lstm(spec, "predictor.shared", cin)
    for name in ("F0", "N"):
        _resblk(spec, f"predictor.{name}.0", HIDDEN, HIDDEN, False)
        _resblk(spec, f"predictor.{name}.1", HIDDEN, HIDDEN // 2, True)
        _resblk(spec, f"predictor.{name}.2", HIDDEN // 2, HIDDEN // 2, False)
    spec.append(("predictor.F0_proj.weight", (1, HIDDEN // 2, 1), "conv", HIDDEN // 2))
    spec.append(("predictor.F0_proj.bias", (1,), "f0_bias", 0))
    _conv(spec, "predictor.N_proj", HIDDEN // 2, 1, 1)
    return spec


def random_upstream_weights(seed=0):
    """{name: float32 array} for the upstream stages (same init rule as random_weights)."""
    return {name: init_tensor(name, shape, kind, fan_in, seed) for name, shape, kind, fan_in in upstream_spec()}


def random_model_weights(seed=0):
    """Decoder + generator and the upstream stages: the whole Kokoro-82M model."""
    w = random_weights(seed)
    w.update(random_upstream_weights(seed))
    return w


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for byte in s.encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def mix_seed(seed: int, index: int) -> int:
    """splitmix64 finalizer of seed ^ index * golden (src/engine.rs:141-146)."""
    m = 0xFFFFFFFFFFFFFFFF
    z = (seed ^ ((index * 0x9E3779B97F4A7C15) & m)) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def init_tensor(name, shape, kind, fan_in, seed):
    rng = np.random.default_rng(mix_seed(seed, fnv1a64(name)))
    n = int(np.prod(shape))
    if kind in ("conv", "convt", "post"):
        bound = 1.0 / np.sqrt(fan_in)
        v = rng.uniform(-bound, bound, n)
        if kind == "post":
            v = v * 0.1
    elif kind == "norm_w":
        v = rng.uniform(0.8, 1.2, n)
    elif kind == "norm_b":
        v = rng.uniform(-0.1, 0.1, n)
    elif kind == "alpha":
        v = rng.uniform(0.5, 1.5, n)
    elif kind == "lstm":
        # torch.nn.LSTM's default: U(-1/sqrt(H), 1/sqrt(H))
        bound = 1.0 / np.sqrt(fan_in)
        v = rng.uniform(-bound, bound, n)
    elif kind == "emb":
        v = rng.standard_normal(n)
    elif kind == "dur_w":
        # a row shared by the 50 outputs (3x the Linear default) plus the default per row: the 50
        # logits of a token move together, so that the durations vary from token to token (about
        # 2 to 12 frames) instead of averaging out in the sum of 50 sigmoids
        bound = 1.0 / np.sqrt(fan_in)
        common = rng.uniform(-3 * bound, 3 * bound, shape[1])
        v = (common[None, :] + rng.uniform(-bound, bound, shape)).reshape(-1)
    elif kind == "f0_bias":
        # a voiced F0 curve (Hz) around which the stack's output varies
        v = rng.uniform(120.0, 200.0, n)
    elif kind == "dur_bias":
        # about 5 frames per token on average over N(0, 1) styles (sigmoid(-2.2) * 50 = 5.0 before the
        # shared row of the weight moves it)
        v = -2.2 + rng.uniform(-0.1, 0.1, n)
    else:
        raise ValueError(kind)
    return v.astype(np.float32).reshape(shape)


def random_weights(seed=0, prefixes=None):
    """{name: float32 array} for every tensor (optionally only names under `prefixes`)."""
    out = {}
    for name, shape, kind, fan_in in tensor_spec():
        if prefixes and not any(name.startswith(p) for p in prefixes):
            continue
        out[name] = init_tensor(name, shape, kind, fan_in, seed)
    return out


def param_count():
    return sum(int(np.prod(s)) for _, s, _, _ in tensor_spec())
