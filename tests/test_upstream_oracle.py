"""Pins of the upstream oracle (oracle/torch_ref.py: ALBERT, the text encoder, the duration encoder,
the LSTMs, the durations, the F0 / N stacks), run on the CPU.

Each restated stage is checked against an implementation that does not share its code:
- ALBERT against transformers' AlbertModel (the model class upstream kokoro's PL-BERT is, with
  hidden_act gelu_new, one shared layer, post-LN; src/albert.rs:1-2) loaded with the same weights;
- the BiLSTM against torch.nn.LSTM(bidirectional=True) (gate order, the reverse direction, both
  biases);
- gelu_new against transformers' NewGELU and torch's tanh-approximate GELU;
- AdaLayerNorm against closed forms (zero projection = plain LayerNorm; gamma = -1 kills the
  normalized part), so a dropped "1 +" or swapped gamma / beta fails;
- the text encoder's LayerNorm over channels against F.layer_norm on the transposed tensor and the
  conv stack against nn.Conv1d modules;
- the duration rule against the library's kk_durations_from_logits (ties at .5 included);
- the duration expansion of the F0 / N input against the library's src_row table.
Negative controls plant a mistake in the oracle's inputs and check that the comparison sees it.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import torch_ref as R

torch.set_num_threads(4)


@pytest.fixture(scope="module")
def w():
    from kokoro_hip import model_spec
    return model_spec.random_model_weights(seed=0)


def _ids(rng, n):
    return np.concatenate([[0], rng.integers(0, 178, n), [0]]).astype(np.int64)


def test_albert_vs_transformers(w):
    from transformers import AlbertConfig, AlbertModel
    cfg = AlbertConfig(vocab_size=178, embedding_size=128, hidden_size=768, num_attention_heads=12,
                       intermediate_size=2048, num_hidden_layers=12, num_hidden_groups=1, inner_group_num=1,
                       hidden_act="gelu_new", max_position_embeddings=512, type_vocab_size=2, layer_norm_eps=1e-12,
                       hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0)
    cfg._attn_implementation = "eager"
    m = AlbertModel(cfg, add_pooling_layer=False).double().eval()
    sd = {k[len("bert."):]: torch.from_numpy(np.asarray(v, np.float64)) for k, v in w.items() if k.startswith("bert.")}
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all("position_ids" in k or "token_type_ids" in k for k in missing), missing
    rng = np.random.default_rng(3)
    for n in (5, 37):
        ids = _ids(rng, n)
        with torch.no_grad():
            ref = m(input_ids=torch.from_numpy(ids)[None], attention_mask=torch.ones(1, len(ids), dtype=torch.long))
        got = R.albert(w, ids)
        err = (got - ref.last_hidden_state[0]).abs().max().item()
        assert err < 1e-9, err
    # negative control: a wrong position offset (positions from 1) is seen
    w2 = dict(w)
    w2["bert.embeddings.position_embeddings.weight"] = np.roll(w["bert.embeddings.position_embeddings.weight"], -1, 0)
    assert (R.albert(w2, ids) - ref.last_hidden_state[0]).abs().max().item() > 1e-3


def test_bilstm_vs_torch_lstm(w):
    lstm = torch.nn.LSTM(640, 256, bidirectional=True, batch_first=True).double()
    p = "predictor.text_encoder.lstms.0"
    sd = {k[len(p) + 1:]: torch.from_numpy(np.asarray(v, np.float64)) for k, v in w.items() if k.startswith(p + ".")}
    lstm.load_state_dict(sd)
    x = torch.from_numpy(np.random.default_rng(4).standard_normal((19, 640)))
    with torch.no_grad():
        ref = lstm(x[None])[0][0]
    got = R.bilstm(w, p, x)
    assert (got - ref).abs().max().item() < 1e-12
    # negative control: gates in the order i, g, f, o instead of i, f, g, o
    w2 = dict(w)
    for sfx in ("", "_reverse"):
        for nm in ("weight_ih_l0", "weight_hh_l0", "bias_ih_l0", "bias_hh_l0"):
            a = np.asarray(w[f"{p}.{nm}{sfx}"])
            w2[f"{p}.{nm}{sfx}"] = np.concatenate([a[:256], a[512:768], a[256:512], a[768:]])
    assert (R.bilstm(w2, p, x) - ref).abs().max().item() > 1e-2


def test_gelu_new():
    from transformers.activations import NewGELUActivation
    x = torch.linspace(-8, 8, 2001, dtype=torch.float64)
    assert (R.gelu_new(x) - NewGELUActivation()(x)).abs().max().item() < 1e-15
    assert (R.gelu_new(x) - F.gelu(x, approximate="tanh")).abs().max().item() < 1e-14
    # not the erf GELU
    assert (R.gelu_new(x) - F.gelu(x)).abs().max().item() > 1e-4


def test_ada_layer_norm_closed_forms():
    rng = np.random.default_rng(5)
    h = torch.from_numpy(rng.standard_normal((7, 512)) * 3 + 1)
    s = rng.standard_normal(128)
    zero = {"fc.weight": np.zeros((1024, 128)), "fc.bias": np.zeros(1024)}
    got = R.ada_layer_norm(zero, "fc", h, s)
    assert (got - F.layer_norm(h, (512,), eps=1e-5)).abs().max().item() < 1e-12
    # gamma = -1, beta = b: the normalized part vanishes, every row is b
    b = rng.standard_normal(512)
    kill = {"fc.weight": np.zeros((1024, 128)), "fc.bias": np.concatenate([-np.ones(512), b])}
    got = R.ada_layer_norm(kill, "fc", h, s)
    assert (got - torch.from_numpy(b)[None]).abs().max().item() < 1e-12
    # the row statistics: mean 0, variance var / (var + eps) per row before the style
    n = R.ada_layer_norm(zero, "fc", h, s)
    assert n.mean(1).abs().max().item() < 1e-12


def test_text_encoder_vs_modules(w):
    """The text encoder as torch modules (Embedding, Conv1d, LayerNorm over the channel axis,
    LeakyReLU, LSTM) -- the structure of upstream kokoro's TextEncoder -- against the oracle."""
    rng = np.random.default_rng(6)
    ids = _ids(rng, 23)
    emb = torch.nn.Embedding(178, 512).double()
    emb.weight.data = torch.from_numpy(np.asarray(w["text_encoder.embedding.weight"], np.float64))
    x = emb(torch.from_numpy(ids))[None].transpose(1, 2)  # [1, 512, t]
    for i in range(3):
        conv = torch.nn.Conv1d(512, 512, 5, padding=2).double()
        conv.weight.data = torch.from_numpy(np.asarray(w[f"text_encoder.cnn.{i}.0.weight"], np.float64))
        conv.bias.data = torch.from_numpy(np.asarray(w[f"text_encoder.cnn.{i}.0.bias"], np.float64))
        ln = torch.nn.LayerNorm(512, eps=1e-5).double()
        ln.weight.data = torch.from_numpy(np.asarray(w[f"text_encoder.cnn.{i}.1.gamma"], np.float64))
        ln.bias.data = torch.from_numpy(np.asarray(w[f"text_encoder.cnn.{i}.1.beta"], np.float64))
        x = conv(x)
        x = ln(x.transpose(1, 2)).transpose(1, 2)
        x = F.leaky_relu(x, 0.2)
    lstm = torch.nn.LSTM(512, 256, bidirectional=True, batch_first=True).double()
    p = "text_encoder.lstm"
    lstm.load_state_dict({k[len(p) + 1:]: torch.from_numpy(np.asarray(v, np.float64))
                          for k, v in w.items() if k.startswith(p + ".")})
    with torch.no_grad():
        ref = lstm(x.transpose(1, 2))[0][0]
        got = R.text_encoder(w, ids)
    assert (got - ref).abs().max().item() < 1e-12


def test_durations_vs_library():
    from kokoro_hip import api
    rng = np.random.default_rng(8)
    lg = rng.standard_normal((40, 50)) * 2 - 2.5
    for speed in (1.0, 0.8, 1.3):
        want = api.durations_from_logits(lg.astype(np.float32), speed)
        got = R.durations(lg.astype(np.float32).astype(np.float64), speed)
        s = torch.sigmoid(torch.from_numpy(lg.astype(np.float32).astype(np.float64))).sum(1).numpy() / speed
        near = np.abs(s - np.floor(s) - 0.5) < 1e-4  # f32 and f64 sums may round differently there
        assert np.array_equal(want[~near], got[~near])
    # ties: sum exactly 2.5 -> 2, 3.5 -> 4 (half to even), and the clamp at 1
    assert list(R.durations(np.full((1, 50), -100.0), 1.0)) == [1]
    lg = np.full((2, 50), -1000.0)
    lg[0, :5] = 1000.0  # sum 5 -> 5 at speed 2 -> 2.5 -> 2
    lg[1, :7] = 1000.0  # 7 / 2 = 3.5 -> 4
    assert list(R.durations(lg, 2.0)) == [2, 4]


def test_expansion_matches_library_src_row(w):
    """f0n's frame rows (np.repeat of the token rows) are the library's src_row table of one item."""
    from kokoro_hip import api
    dur = np.array([3, 1, 4, 1, 5], np.int64)
    sr = api.layout_src_row([dur], [0], [0], int(dur.sum()) + 2)
    assert np.array_equal(sr[: dur.sum()], np.repeat(np.arange(len(dur)), dur))


def test_upstream_shapes_and_taps(w):
    rng = np.random.default_rng(9)
    ids = _ids(rng, 11)
    s = rng.standard_normal(256).astype(np.float32)
    taps = {}
    pred, t_en, f0, n = R.upstream(w, ids, s, taps=taps)
    N = int(pred.sum())
    assert t_en.shape == (512, 13) and f0.shape == (2 * N,) and n.shape == (2 * N,)
    assert taps["d"].shape == (13, 640) and taps["logits"].shape == (13, 50)
    # the style half of the duration encoder's output is ref_s[128:256] on every row
    assert np.allclose(taps["d"][:, 512:].numpy(), s[None, 128:])
    # a forced duration table replaces the prediction
    pred2, _, f02, _ = R.upstream(w, ids, s, dur=np.full(13, 2))
    assert list(pred2) == [2] * 13 and f02.shape == (52,)
