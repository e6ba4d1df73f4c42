"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Two bars per waveform-level check:
- against the fp32 oracle: the north-star tolerance, max-abs <= 2e-3 and SNR >= 40 dB;
- against the oracle with its MFMA-layer operands rounded to bf16 (the GPU's own rounding points):
  a tight bar that an indexing, masking or layout mistake cannot pass (SNR >= 50 dB for one Snake
  block and for the decoder, >= 44 dB end to end: only accumulation order and bf16 rounding ties
  differ, and those ties compound through the layers in series -- two emulations that differ by a
  single fp16 rounding point of the increments already land 54.6-55 dB apart on one 256-channel
  Snake block; a masking or indexing error lands near 0-20 dB).
Integer and index work (duration expansion) is compared bit for bit.
"""
import numpy as np
import pytest

from conftest import snr_db

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


def test_snake_block_ragged(gpu_ctx, oracle_model):
    from kokoro_hip import api
    from oracle import oracle as O
    rng = np.random.default_rng(21)
    ts = [57, 130, 96]
    xs = [rng.standard_normal((256, t)).astype(np.float32) for t in ts]
    styles = [rng.standard_normal(256).astype(np.float32) for _ in ts]
    _print("snake block resblocks.1, T =", ts)
    with api.Plan.snake(gpu_ctx, "decoder.generator.resblocks.1", xs, styles, gap=40) as plan:
        plan.run()
        outs = plan.fetch()
    for x, s, y in zip(xs, styles, outs):
        ref = oracle_model.snake_block("decoder.generator.resblocks.1", x, s)
        with O.bf16_emulation():
            emu = oracle_model.snake_block("decoder.generator.resblocks.1", x, s)
        d_ref, d_emu = y - x, emu - x  # compare the block's increment, not the pass-through input
        _print("  fp32 snr", snr_db(ref - x, d_ref), "emu snr", snr_db(d_emu, d_ref), "maxabs", np.abs(y - ref).max())
        assert snr_db(d_emu, d_ref) >= 50.0
        assert snr_db(ref - x, d_ref) >= 40.0


def test_snake_block_128(gpu_ctx, oracle_model):
    from kokoro_hip import api
    from oracle import oracle as O
    rng = np.random.default_rng(22)
    ts = [300, 141]
    xs = [rng.standard_normal((128, t)).astype(np.float32) for t in ts]
    styles = [rng.standard_normal(256).astype(np.float32) for _ in ts]
    with api.Plan.snake(gpu_ctx, "decoder.generator.noise_res.1", xs, styles, gap=40) as plan:
        plan.run()
        outs = plan.fetch()
    for x, s, y in zip(xs, styles, outs):
        with O.bf16_emulation():
            emu = oracle_model.snake_block("decoder.generator.noise_res.1", x, s)
        _print("  128ch k11 emu snr", snr_db(emu - x, y - x))
        assert snr_db(emu - x, y - x) >= 50.0


@pytest.fixture(scope="module")
def decoder_run(gpu_ctx, oracle_model):
    from kokoro_hip import api, workloads
    from oracle import oracle as O
    items = workloads.small_items(31, [9, 23, 14])
    _print("decoder batch, N =", [it.n_frames for it in items])
    with api.Plan.decoder(gpu_ctx, items) as plan:
        plan.run()
        audio = plan.fetch()
        taps = []
        for b, it in enumerate(items):
            n = it.n_frames
            taps.append({"asr": plan.tap("asr", b, (512, n)), "decoder": plan.tap("decoder", b, (512, 2 * n)),
                         "spec": plan.tap("spec", b, (22, 120 * n + 1)),
                         "post": plan.tap("post", b, (22, 120 * n + 1))})
    refs, emus = [], []
    for it in items:
        refs.append(O.synth_item(oracle_model, it, taps=True))
        with O.bf16_emulation():
            emus.append(O.synth_item(oracle_model, it, taps=True))
    return items, audio, taps, refs, emus


def test_duration_expansion_bit_exact(decoder_run):
    from oracle import oracle as O
    items, _, taps, _, _ = decoder_run
    for it, tp in zip(items, taps):
        assert np.array_equal(tp["asr"], O.expand_tokens(it.t_en, it.dur))


def test_decoder_output(decoder_run, oracle_model):
    from oracle import oracle as O
    items, _, taps, _, _ = decoder_run
    for it, tp in zip(items, taps):
        asr = O.expand_tokens(it.t_en, it.dur)
        ref = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
        with O.bf16_emulation():
            emu = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
        _print("  decoder fp32 snr", snr_db(ref, tp["decoder"]), "emu snr", snr_db(emu, tp["decoder"]))
        assert snr_db(emu, tp["decoder"]) >= 50.0
        assert snr_db(ref, tp["decoder"]) >= 40.0


def test_source_spectrum(decoder_run):
    """Harmonic source + STFT from identical F0 and noise: magnitudes to f32 rounding, phases
    compared on the circle (a sign flip of a zero imaginary part moves atan2 between +pi and -pi)."""
    items, _, taps, refs, _ = decoder_run
    for tp, (_, spec, _) in zip(taps, refs):
        g = tp["spec"]
        mag_err = np.abs(g[:11] - spec[:11]).max() / max(np.abs(spec[:11]).max(), 1e-6)
        dphi = np.angle(np.exp(1j * (g[11:].astype(np.float64) - spec[11:])))
        weight = spec[:11] > 1e-4 * spec[:11].max()
        _print("  spec mag rel err", mag_err, "phase err", np.abs(dphi[weight]).max())
        assert mag_err < 1e-4
        assert np.abs(dphi[weight]).max() < 1e-3


def test_end_to_end_audio(decoder_run):
    items, audio, taps, refs, emus = decoder_run
    for it, a, (ref, _, _), (emu, _, _) in zip(items, audio, refs, emus):
        assert a.shape == (600 * it.n_frames,)
        _print("  audio fp32 snr", snr_db(ref, a), "maxabs", np.abs(a - ref).max(), "emu snr", snr_db(emu, a))
        assert np.abs(a - ref).max() <= 2e-3
        assert snr_db(ref, a) >= 40.0
        assert snr_db(emu, a) >= 44.0


def test_generator_only(gpu_ctx, oracle_model):
    from kokoro_hip import api, workloads
    from oracle import oracle as O
    x, f0, style, seed = workloads.config1_generator_input(seed=5, n_frames=12)
    with api.Plan.generator(gpu_ctx, [x], [f0], [style], [seed]) as plan:
        plan.run()
        (a,) = plan.fetch()
    ref = oracle_model.generator(x, f0, style, O.rand_ini(seed), O.gen_noise(seed, 600 * 12 * 9))
    _print("  generator-only fp32 snr", snr_db(ref, a), "maxabs", np.abs(a - ref).max())
    assert np.abs(a - ref).max() <= 2e-3
    assert snr_db(ref, a) >= 40.0


def test_plan_outliving_its_context(weights):
    """A plan freed after its context is closed releases nothing twice and reports KK_ERR_STATE
    (Engine ownership: src/engine.rs owns GpuKokoro; a caller may drop them in any order)."""
    from kokoro_hip import api, workloads
    ctx = api.Context(0)
    ctx.upload_model(weights)
    plan = api.Plan.decoder(ctx, workloads.small_items(41, [3]))
    ctx.close()
    with pytest.raises(api.KKError) as e:
        plan.run()
    assert e.value.code == -4
    plan.free()
