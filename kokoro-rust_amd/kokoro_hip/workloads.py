"""Seeded synthetic workloads for the decoder + generator path (no corpus or checkpoint offline).

One item carries what the reference's `forward_batch` holds for it when the decoder starts
(src/gpu_batch.rs:244-297): integer durations per token, the text-encoder features of its tokens
(`t_en`, [512, T_tok]), the F0 and energy curves at 2N (the predictor's outputs), `ref_s` (256
values; the decoder uses the first 128, src/gpu_batch.rs:206-213) and its noise source
(ItemNoise::Counter(seed), src/gpu_batch.rs:14-17).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class DecoderItem:
    dur: np.ndarray          # int64 [T_tok], each >= 1
    t_en: np.ndarray         # float32 [512, T_tok]
    f0: np.ndarray           # float32 [2N]
    energy: np.ndarray       # float32 [2N]
    ref_s: np.ndarray        # float32 [256]
    seed: int                # noise counter seed
    rand_ini: np.ndarray | None = None   # fixed noise replay (ItemNoise::Fixed)
    sine: np.ndarray | None = None

    @property
    def n_frames(self) -> int:
        return int(self.dur.sum())

    @property
    def n_samples(self) -> int:
        return 600 * self.n_frames


def smooth_curve(rng, n, lo, hi, knots=None):
    """Smooth random curve in [lo, hi]: cubic-ish interpolation of random knots."""
    knots = knots or max(4, n // 40)
    xs = np.linspace(0, n - 1, knots)
    ys = rng.uniform(0.0, 1.0, knots)
    t = np.arange(n)
    y = np.interp(t, xs, ys)
    # two passes of a short moving average keep it smooth at the knots
    k = max(1, n // (4 * knots))
    if k > 1:
        ker = np.ones(k) / k
        y = np.convolve(np.pad(y, k, mode="edge"), ker, mode="same")[k:-k]
        y = np.convolve(np.pad(y, k, mode="edge"), ker, mode="same")[k:-k]
    return (lo + (hi - lo) * y).astype(np.float32)


def random_durations(rng, n_frames, lo=1, hi=9):
    """Integer durations >= 1 that sum to n_frames exactly."""
    d = []
    s = 0
    while s < n_frames:
        v = int(rng.integers(lo, hi + 1))
        v = min(v, n_frames - s)
        d.append(v)
        s += v
    return np.asarray(d, dtype=np.int64)


def make_item(rng, n_frames, seed, unvoiced_frac=0.1):
    dur = random_durations(rng, n_frames)
    t_tok = len(dur)
    t_en = rng.standard_normal((512, t_tok)).astype(np.float32)
    l2 = 2 * n_frames
    f0 = smooth_curve(rng, l2, 100.0, 300.0)
    if unvoiced_frac > 0 and l2 >= 20:
        # a few unvoiced spans (F0 below the 10 Hz voicing threshold, src/kernels sine_har_source)
        n_spans = max(1, int(unvoiced_frac * l2 / 20))
        for _ in range(n_spans):
            a = int(rng.integers(0, l2 - 10))
            b = min(l2, a + int(rng.integers(5, 20)))
            f0[a:b] = rng.uniform(0.0, 5.0)
    energy = smooth_curve(rng, l2, -1.0, 1.0)
    ref_s = rng.standard_normal(256).astype(np.float32)
    return DecoderItem(dur=dur, t_en=t_en, f0=f0, energy=energy, ref_s=ref_s, seed=int(seed))


def config3_items(seed=3, batch=32, lo=100, hi=800):
    """batch 32 ragged, N ~ U[lo, hi] decoder frames per item."""
    rng = np.random.default_rng(seed)
    ns = rng.integers(lo, hi + 1, batch)
    return [make_item(rng, int(n), seed=int(rng.integers(0, 2**63))) for n in ns]


def small_items(seed, ns):
    rng = np.random.default_rng(seed)
    return [make_item(rng, int(n), seed=int(rng.integers(0, 2**63))) for n in ns]


def config1_generator_input(seed=1, n_frames=100):
    """generator-only forward, x [512, 2N] ~ N(0,1), F0 smooth in 100-300 Hz."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((512, 2 * n_frames)).astype(np.float32)
    f0 = smooth_curve(rng, 2 * n_frames, 100.0, 300.0)
    style = rng.standard_normal(128).astype(np.float32)
    return x, f0, style, int(rng.integers(0, 2**63))


def config2_snake_items(seed=2, batch=16, lo=500, hi=2000, channels=256):
    """one AdaINResBlock1 (256 ch, k 7) on 16 ragged items of T ~ U[500, 2000]."""
    rng = np.random.default_rng(seed)
    ts = rng.integers(lo, hi + 1, batch)
    xs = [rng.standard_normal((channels, int(t))).astype(np.float32) for t in ts]
    styles = [rng.standard_normal(128).astype(np.float32) for _ in ts]
    return xs, styles


def config5_items(seed=5, batch=128, g_lo=80, g_hi=4000):
    """128 items, generator frames G log-uniform in [80, 4000] (N = G / 2)."""
    rng = np.random.default_rng(seed)
    gs = np.exp(rng.uniform(np.log(g_lo), np.log(g_hi), batch))
    ns = np.maximum(1, (gs / 2).astype(np.int64))
    return [make_item(rng, int(n), seed=int(rng.integers(0, 2**63))) for n in ns]


# ------------------------------------------------------------------ ids-level items (the whole forward)
@dataclass
class IdsItem:
    """BatchItem (src/gpu_batch.rs:19-24): input_ids with the two boundary tokens, ref_s, speed, noise."""
    ids: np.ndarray          # int64 [n_ids], each in [0, 178)
    ref_s: np.ndarray        # float32 [256]
    seed: int
    speed: float = 1.0
    rand_ini: np.ndarray | None = None
    sine: np.ndarray | None = None


def make_ids_item(rng, n_phonemes, seed, speed=1.0):
    """n_phonemes ids uniform over the vocabulary, wrapped in the boundary token 0; ref_s ~ N(0, 1)."""
    ids = np.concatenate([[0], rng.integers(0, 178, n_phonemes), [0]]).astype(np.int64)
    return IdsItem(ids=ids, ref_s=rng.standard_normal(256).astype(np.float32), seed=int(seed), speed=speed)


def config4_items(seed=4, batch=64, lo=20, hi=510):
    """batch 64, phoneme ids uniform over vocab 178, lengths uniform 20-510."""
    rng = np.random.default_rng(seed)
    return [make_ids_item(rng, int(rng.integers(lo, hi + 1)), 4000 + b) for b in range(batch)]


def small_ids_items(seed, ns, speed=1.0):
    rng = np.random.default_rng(seed)
    return [make_ids_item(rng, n, 7000 + b, speed) for b, n in enumerate(ns)]
