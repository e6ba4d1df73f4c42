"""The CPU oracle against the committed golden vectors (tests/golden/golden_v1.npz, written by the
float64 torch restatement from library routines; see tests/golden/make_golden.py)."""
import os

import numpy as np
import pytest

from conftest import snr_db
from oracle import oracle as O

G = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_v1.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(G, allow_pickle=False)


def test_golden_conv_and_convt(g):
    y = O.conv1d(g["conv_x"], g["conv_w"], g["conv_b"], 1, 25, 5)
    assert np.abs(y - g["conv_y"]).max() < 1e-5 * np.abs(g["conv_y"]).max()
    y = O.conv_transpose1d(g["convt_x"], g["convt_w"], g["convt_b"], 10, 5)
    assert np.abs(y - g["convt_y"]).max() < 1e-5 * np.abs(g["convt_y"]).max()


def test_golden_stft_istft(g):
    s = O.stft20(g["stft_x"])
    assert np.abs(s[:11] - g["stft_mag"]).max() < 1e-5
    strong = g["stft_mag"] > 1e-3
    assert np.abs(np.angle(np.exp(1j * (s[11:] - g["stft_phase"]))))[strong].max() < 1e-4
    a = O.istft20(g["istft_post"])
    assert np.abs(a - g["istft_y"]).max() < 1e-5 * np.abs(g["istft_y"]).max()


def test_golden_source(g, weights):
    har = O.sine_source(g["src_f0"], g["src_rand_ini"], g["src_noise"],
                        weights["decoder.generator.m_source.l_linear.weight"],
                        weights["decoder.generator.m_source.l_linear.bias"][0])
    assert np.abs(har - g["src_har"]).max() < 5e-4


def test_golden_blocks(g, oracle_model):
    x = g["snake_x"]
    y = oracle_model.snake_block("decoder.generator.resblocks.0", x, g["snake_style"])
    assert snr_db(g["snake_y"] - x, y - x) > 90
    y = oracle_model.resblk("decoder.encode", g["encode_x"], g["snake_style"], 1024)
    assert snr_db(g["encode_y"], y) > 90


def test_golden_generator_glue(g, oracle_model):
    """Generator stages from the golden spectrum (noise convs, Snake blocks, ConvTs, reflect pad,
    resblock means, conv_post, iSTFT)."""
    audio, post = oracle_model.generator_from_spec(g["gen_x"], g["gen_spec"], g["gen_style"])
    assert snr_db(g["gen_post"], post) > 70
    assert snr_db(g["gen_audio"], audio) > 70
    assert np.abs(audio - g["gen_audio"]).max() < 1e-4
