"""Pins of the CPU oracle (oracle/kk_oracle.c), run on the CPU.

Every oracle function is checked against something that does not share its code: published
known-answer values (splitmix64), closed forms (durations, layout tables, Box-Muller, Snake),
library routines (torch.nn.functional conv / instance_norm / interpolate, torch.stft / istft), and
an independent float64 torch restatement of the whole decoder and generator (oracle/torch_ref.py).
Negative controls plant a mistake on the CPU and check that the comparison catches it.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import torch_ref as R
from conftest import snr_db
from oracle import oracle as O

torch.set_num_threads(4)
M64 = (1 << 64) - 1


# ------------------------------------------------------------------ noise (src/vocoder.rs:17-41)


def splitmix64_stream(state, n):
    """Textbook stateful splitmix64 (Vigna): state += golden; mix."""
    out = []
    for _ in range(n):
        state = (state + 0x9E3779B97F4A7C15) & M64
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        out.append(z ^ (z >> 31))
    return out


def test_splitmix64_known_answers():
    # published first outputs of splitmix64 from state 0
    assert O.splitmix_at(0, 0) == 0xE220A8397B1DCDAF
    assert O.splitmix_at(0, 1) == 0x6E789E6AA1B965F4
    assert O.splitmix_at(0, 2) == 0x06C45D188009454F
    rng = np.random.default_rng(1)
    for seed in [int(v) for v in rng.integers(0, 2**63, 4)] + [M64]:
        ref = splitmix64_stream(seed, 40)
        assert [O.splitmix_at(seed, i) for i in range(40)] == ref


def test_rand_ini_and_box_muller():
    seed = 0x1234ABCD9876
    ri = O.rand_ini(seed)
    want = np.array([(O.splitmix_at(seed, h) >> 40) / 16777216.0 for h in range(9)], np.float32)
    assert np.array_equal(ri, want)
    n = 1001
    z = O.gen_noise(seed, n)
    xs = [O.splitmix_at(seed, 1024 + i) for i in range((n + 1) // 2)]
    u1 = np.array([((x >> 40) + 1) / 16777216.0 for x in xs])
    u2 = np.array([((x >> 16) & 0xFFFFFF) / 16777216.0 for x in xs])
    r = np.sqrt(-2 * np.log(u1))
    ref = np.empty(2 * len(xs))
    ref[0::2], ref[1::2] = r * np.cos(2 * np.pi * u2), r * np.sin(2 * np.pi * u2)
    assert np.abs(z - ref[:n]).max() < 2e-5
    assert abs(z.mean()) < 0.1 and abs(z.std() - 1) < 0.1


# ------------------------------------------------------------------ host rules (bit-exact)


def test_durations_ties_and_clamp():
    t = 6
    logits = np.zeros((t, 50), np.float32)  # sigmoid(0) = 0.5 exactly: sum = 25
    for speed, want in [(1.0, 25), (2.0, 12), (10.0, 2), (20.0, 1), (100.0, 1), (25 / 3.5, 4)]:
        d = O.durations_from_logits(logits, speed)
        assert (d == want).all(), (speed, d)
    logits[:] = -80.0  # sigmoid underflows to ~0 -> clamp to 1
    assert (O.durations_from_logits(logits, 1.0) == 1).all()
    rng = np.random.default_rng(3)
    lg = rng.normal(0, 3, (200, 50)).astype(np.float32)
    s = np.zeros(200, np.float32)
    for j in range(50):
        s = s + (np.float32(1) / (np.float32(1) + np.exp(-lg[:, j])))
    ref = np.maximum(1, np.round(s / np.float32(1.3)).astype(np.int64))  # np.round: half to even
    assert np.array_equal(O.durations_from_logits(lg, 1.3), ref)


def test_layout_closed_form():
    rng = np.random.default_rng(4)
    nfs = rng.integers(1, 50, 7)
    a, ln = O.layout_frames(nfs, gap=2)
    assert ln == int(nfs.sum()) + 2 * len(nfs)
    assert np.array_equal(a, np.concatenate([[0], np.cumsum(nfs + 2)[:-1]]))
    for f, add in [(1, 0), (2, 0), (20, 0), (120, 1)]:
        l = f * ln + (1 if add else 0)
        col = O.layout_col_item(l, a * f, nfs * f + add)
        brute = np.full(l, -1, np.int32)
        for b in range(len(nfs)):
            brute[a[b] * f: a[b] * f + nfs[b] * f + add] = b
        assert np.array_equal(col, brute)
        # every gap is at least the widest conv reach of its domain (docs/design/BATCHING.md:23-24)
        assert (col < 0).sum() >= len(nfs) * (2 * f - add)
    # stage-1 item starts are aligned to the stride-6 noise conv
    assert ((a * 120) % 6 == 0).all()
    with pytest.raises(ValueError):
        O.layout_col_item(10, [0, 5], [6, 3])   # overlap
    with pytest.raises(ValueError):
        O.layout_col_item(10, [0, 8], [3, 3])   # overflow


def test_src_row_closed_form():
    rng = np.random.default_rng(5)
    durs = [rng.integers(1, 6, int(n)) for n in rng.integers(1, 12, 5)]
    tstart = np.concatenate([[0], np.cumsum([len(d) + 2 for d in durs])[:-1]])
    a, ln = O.layout_frames([d.sum() for d in durs])
    sr = O.layout_src_row(durs, tstart, a, ln)
    want = np.full(ln, -1, np.int32)
    for b, d in enumerate(durs):
        want[a[b]: a[b] + d.sum()] = tstart[b] + np.repeat(np.arange(len(d)), d)
    assert np.array_equal(sr, want)


def test_bf16_fp16_rounding():
    rng = np.random.default_rng(6)
    x = np.concatenate([rng.normal(0, 3, 5000), rng.normal(0, 1e-6, 100), [0.0, -0.0, 1.0, 65504.0, 1e-7]])
    x = x.astype(np.float32)
    L = O.lib()
    got = np.array([L.ko_bf16_round(float(v)) for v in x], np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, want)
    import ctypes as C
    L.ko_fp16_round.argtypes = [C.c_float]
    L.ko_fp16_round.restype = C.c_float
    got16 = np.array([L.ko_fp16_round(float(v)) for v in x], np.float32)
    assert np.array_equal(got16, x.astype(np.float16).astype(np.float32))


# ------------------------------------------------------------------ layers vs library routines


@pytest.mark.parametrize("cin,cout,k,stride,pad,dil,t", [
    (5, 7, 3, 1, 1, 1, 40), (9, 4, 7, 1, 9, 3, 33), (22, 6, 12, 6, 3, 1, 121), (8, 3, 1, 1, 0, 1, 17),
    (6, 6, 11, 1, 25, 5, 90), (1, 1, 3, 2, 1, 1, 20)])
def test_conv1d_vs_torch(cin, cout, k, stride, pad, dil, t):
    rng = np.random.default_rng(cin * 100 + k)
    x = rng.standard_normal((cin, t)).astype(np.float32)
    w = rng.standard_normal((cout, cin, k)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    y = O.conv1d(x, w, b, stride, pad, dil)
    ref = F.conv1d(R.T(x)[None], R.T(w), R.T(b), stride=stride, padding=pad, dilation=dil)[0].numpy()
    assert y.shape == ref.shape
    assert np.abs(y - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("cin,cout,k,stride,pad,t", [(6, 4, 20, 10, 5, 13), (5, 3, 12, 6, 3, 21), (2, 2, 3, 2, 1, 9)])
def test_conv_transpose1d_vs_torch(cin, cout, k, stride, pad, t):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((cin, t)).astype(np.float32)
    w = rng.standard_normal((cin, cout, k)).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    y = O.conv_transpose1d(x, w, b, stride, pad)
    ref = F.conv_transpose1d(R.T(x)[None], R.T(w), R.T(b), stride=stride, padding=pad)[0].numpy()
    assert y.shape == ref.shape
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


def test_adain_vs_instance_norm():
    rng = np.random.default_rng(8)
    c, t = 12, 77
    x = (rng.standard_normal((c, t)) * 3 + 5).astype(np.float32)  # offset mean: shifted sums matter
    nw, nb = rng.uniform(0.8, 1.2, c).astype(np.float32), rng.uniform(-0.1, 0.1, c).astype(np.float32)
    fw = (rng.standard_normal((2 * c, 128)) * 0.05).astype(np.float32)
    fb = (rng.standard_normal(2 * c) * 0.05).astype(np.float32)
    s = rng.standard_normal(128).astype(np.float32)
    w = {"p.norm.weight": nw, "p.norm.bias": nb, "p.fc.weight": fw, "p.fc.bias": fb}
    mean, rstd = O.chan_stats(x)
    gb = O.style_fc(fw, fb, s)
    ref_gb = F.linear(R.T(s), R.T(fw), R.T(fb)).numpy()
    assert np.abs(gb - ref_gb).max() < 1e-6
    ref = R.adain(w, "p", R.T(x), s)
    y_leaky = O.adain_apply(x, mean, rstd, nw, nb, gb, mode=0, slope=0.2)
    assert np.abs(y_leaky - F.leaky_relu(ref, 0.2).numpy()).max() < 2e-5
    alpha = rng.uniform(0.5, 1.5, c).astype(np.float32)
    y_snake = O.adain_apply(x, mean, rstd, nw, nb, gb, mode=1, alpha=alpha)
    a = R.T(alpha)[:, None]
    assert np.abs(y_snake - (ref + torch.sin(a * ref) ** 2 / a).numpy()).max() < 2e-5


# ------------------------------------------------------------------ source, STFT, iSTFT


def test_stft_vs_torch():
    rng = np.random.default_rng(9)
    x = np.tanh(rng.standard_normal(600)).astype(np.float32)
    out = O.stft20(x)
    mag, ph = R.stft(x)
    assert out.shape == (22, 121)
    assert np.abs(out[:11] - mag.numpy()).max() < 2e-6 * mag.max().item()
    dphi = np.angle(np.exp(1j * (out[11:] - ph.numpy())))
    sig = mag.numpy() > 1e-3
    assert np.abs(dphi[sig]).max() < 1e-4


def test_istft_vs_torch():
    rng = np.random.default_rng(10)
    post = (rng.standard_normal((22, 61)) * 0.5).astype(np.float32)
    a = O.istft20(post)
    ref = R.istft(post).numpy()
    assert a.shape == ref.shape == (300,)
    assert np.abs(a - ref).max() < 1e-5 * np.abs(ref).max()


def test_sine_source_vs_interpolate_cumsum(weights):
    rng = np.random.default_rng(11)
    from kokoro_hip import workloads
    f0 = workloads.smooth_curve(rng, 40, 100, 300)
    f0[10:14] = 0.0  # an unvoiced span
    seed = 77
    ri, nz = O.rand_ini(seed), O.gen_noise(seed, 300 * 40 * 9)
    har = O.sine_source(f0, ri, nz, weights["decoder.generator.m_source.l_linear.weight"],
                        weights["decoder.generator.m_source.l_linear.bias"][0])
    ref = R.sine_source(weights, f0, ri, nz).numpy()
    # f32 phases of up to ~2e3 rad carry ~1e-4 rad of rounding; the source is O(0.3)
    assert np.abs(har - ref).max() < 5e-4
    assert snr_db(ref, har) > 60


# ------------------------------------------------------------------ blocks and whole path vs torch


def test_snake_blocks_vs_torch(weights, oracle_model):
    rng = np.random.default_rng(12)
    for p, c, t in [("decoder.generator.resblocks.0", 256, 50), ("decoder.generator.noise_res.1", 128, 90)]:
        x = rng.standard_normal((c, t)).astype(np.float32)
        s = rng.standard_normal(256).astype(np.float32)
        y = oracle_model.snake_block(p, x, s)
        ref = R.snake_block(weights, p, R.T(x), s).numpy()
        assert snr_db(ref - x, y - x) > 90, p


def test_decoder_blocks_vs_torch(weights, oracle_model):
    rng = np.random.default_rng(13)
    s = rng.standard_normal(256).astype(np.float32)
    x = rng.standard_normal((514, 9)).astype(np.float32)
    y = oracle_model.resblk("decoder.encode", x, s, 1024)
    assert snr_db(R.resblk(weights, "decoder.encode", R.T(x), s).numpy(), y) > 90
    x = rng.standard_normal((1090, 7)).astype(np.float32)
    y = oracle_model.resblk("decoder.decode.3", x, s, 512, upsample=True)
    assert y.shape == (512, 14)
    assert snr_db(R.resblk(weights, "decoder.decode.3", R.T(x), s, upsample=True).numpy(), y) > 90


@pytest.fixture(scope="module")
def small_item():
    from kokoro_hip import workloads
    return workloads.small_items(14, [4])[0]


def test_decoder_vs_torch(weights, oracle_model, small_item):
    it = small_item
    asr = O.expand_tokens(it.t_en, it.dur)
    x = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
    ref = R.decoder(weights, asr, it.f0, it.energy, it.ref_s).numpy()
    assert x.shape == (512, 2 * it.n_frames)
    assert snr_db(ref, x) > 90


def test_generator_vs_torch(weights, oracle_model, small_item):
    it = small_item
    rng = np.random.default_rng(15)
    x = rng.standard_normal((512, 2 * it.n_frames)).astype(np.float32)
    ri, nz = O.item_noise(it)
    audio, spec, post = oracle_model.generator(x, it.f0, it.ref_s, ri, nz, taps=True)
    # source + STFT: magnitudes to f32 rounding; phases where the bin carries energy (the phase of a
    # near-zero bin is ill-conditioned: the f32 source of the reference moves it, and a zero
    # imaginary part can land on either side of the atan2 branch cut)
    taps = {}
    R.generator(weights, x, it.f0, it.ref_s, ri, nz, taps)
    ts = taps["spec"].numpy()
    assert np.abs(spec[:11] - ts[:11]).max() < 1e-4
    strong = ts[:11] > 1e-2 * ts[:11].max()
    assert np.abs(np.angle(np.exp(1j * (spec[11:] - ts[11:]))))[strong].max() < 1e-3
    # the generator glue from the same spectrum
    taps = {}
    ref = R.generator(weights, x, it.f0, it.ref_s, ri, nz, taps, spec=spec).numpy()
    assert audio.shape == ref.shape == (600 * it.n_frames,)
    assert snr_db(taps["post"].numpy(), post) > 70
    assert snr_db(ref, audio) > 70
    assert np.abs(audio - ref).max() < 1e-4


def test_negative_controls(weights, oracle_model, small_item):
    """Plant mistakes on the CPU: each must move the output past the parity bars."""
    it = small_item
    rng = np.random.default_rng(16)
    x = rng.standard_normal((512, 2 * it.n_frames)).astype(np.float32)
    ri, nz = O.item_noise(it)
    a = oracle_model.generator(x, it.f0, it.ref_s, ri, nz)
    # a neighbour's noise stream
    a_noise = oracle_model.generator(x, it.f0, it.ref_s, ri, O.gen_noise(it.seed ^ 1, nz.size))
    assert snr_db(a, a_noise) < 40
    # another item's style
    a_style = oracle_model.generator(x, it.f0, rng.standard_normal(256).astype(np.float32), ri, nz)
    assert snr_db(a, a_style) < 40
    # one perturbed weight tensor: 1% random noise on a Snake block's convs2 (its output feeds the
    # residual directly; a uniform scale of convs1 would be undone by the instance norm after it)
    w2 = dict(weights)
    key = "decoder.generator.resblocks.4.convs2.1.weight"
    w2[key] = (weights[key] * (1 + 0.01 * rng.standard_normal(weights[key].shape))).astype(np.float32)
    a_w = O.Model(w2).generator(x, it.f0, it.ref_s, ri, nz)
    assert snr_db(a, a_w) < 60 and snr_db(a, a_w) > 20
    # a zero-padding (mask) mistake: a neighbour's samples leaking into the first frames
    x_leak = x.copy()
    x_leak[:, 0] += 1.0
    a_leak = oracle_model.generator(x_leak, it.f0, it.ref_s, ri, nz)
    assert snr_db(a, a_leak) < 44


def test_two_frame_items_are_ill_conditioned(oracle_model):
    """The error-budget fact behind the GPU tests' two-frame rule: a two-column InstanceNorm turns
    operand rounding into O(1) changes, with bf16 and with fp16 operands alike, while one-, three-,
    four- and five-frame items stay well inside the bar (the seeds of the GPU tests' tiny items)."""
    from kokoro_hip import workloads

    def snr(r, x):
        r = r.astype(np.float64)
        return 10 * np.log10((r ** 2).sum() / ((r - x) ** 2).sum())

    for ns, seed in [([2, 1], 66), ([1, 3, 2], 67), ([5, 4], 66)]:
        for it in workloads.small_items(seed, ns):
            asr = O.expand_tokens(it.t_en, it.dur)
            x = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
            with O.operand_formats(0xff, 0):
                xb = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
            with O.operand_formats(0xff, O.GROUP_DECODER):
                xf = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
            if it.n_frames == 2:
                assert snr(x, xb) < 25.0 and snr(x, xf) < 25.0
            else:
                assert snr(x, xb) >= 35.0 and snr(x, xf) >= snr(x, xb)
