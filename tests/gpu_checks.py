"""GPU-side comparison helpers shared by the GPU test modules (not a test module itself)."""
import numpy as np

from conftest import snr_db


def _print(*a):
    print(*a, flush=True)


# Items of exactly two decoder frames: the decoder's InstanceNorm then runs over two columns, which
# normalize to +-d / sqrt(d^2 + 4 eps) whatever their difference d, so a channel whose two values lie
# within ~sqrt(eps) of each other turns operand rounding into an O(1) change.  Measured on the
# oracle (tests use the same seeds): with bf16 operands the decoder lands 14-16 dB and the audio
# 29-30 dB from fp32; fp16 operands do not fix it (15-18 and 30-32 dB).  One- and three-frame and
# longer items meet the full bar end to end (audio 43-44 dB).  Two-frame items are checked stage by
# stage: the decoder against the emulation's own deviation, the generator from the GPU's decoder
# output at the full bar.
ILL_CONDITIONED_N = (2,)


def unstable_phase_bins(spec_gpu, spec_ref):
    """Spectral bins whose phase input to the generator differs between two spectra by more than
    1e-2 rad (raw, not wrapped: the generator reads the phase values themselves).  Two kinds occur,
    both set by rounding, in the reference against upstream torch as here: atan2's branch cut (a bin
    with a ~0 imaginary part and a negative real part reads +pi on one side and -pi on the other),
    and the real DC / Nyquist bins of a frame whose sum cancels to ~1e-8, which read 0 or pi by
    that sum's sign."""
    return int((np.abs(np.asarray(spec_gpu[11:], np.float64) - spec_ref[11:]) > 1e-2).sum())


def check_vs_oracle(ctx, oracle_model, items, label):
    """Runs the items and compares each with the oracle.

    - Duration expansion: bit-exact.
    - Source spectrum: magnitudes to f32 rounding, phases on the circle where a bin carries energy.
    - Audio with the north-star bar (max-abs <= 2e-3, SNR >= 40 dB): end to end against the oracle,
      or against the oracle's generator run from the GPU's own spectrum when a bin's phase is set by
      rounding (unstable_phase_bins: atan2's branch cut -- the first and last frame of every item are
      symmetric under the reflect padding, so all their bins are real -- and real DC / Nyquist bins
      whose sum cancels); the generator sees such a phase jump as an input change, in the reference
      against upstream torch as here.
    - Two-frame items (ILL_CONDITIONED_N): the decoder output within 6 dB of the bf16-emulated
      oracle's own distance from fp32, and the audio against the oracle's generator run from the
      GPU's decoder output and spectrum.
    Returns the number of items compared end to end and the audio."""
    from kokoro_hip import api
    from oracle import oracle as O
    with api.Plan.decoder(ctx, items) as plan:
        plan.run()
        outs = plan.fetch()
        taps = [{"asr": plan.tap("asr", b, (512, it.n_frames)), "dec": plan.tap("decoder", b, (512, 2 * it.n_frames)),
                 "spec": plan.tap("spec", b, (22, 120 * it.n_frames + 1))} for b, it in enumerate(items)]
    end_to_end = 0
    for it, a, tp in zip(items, outs, taps):
        assert a.shape == (600 * it.n_frames,) and np.isfinite(a).all()
        asr = O.expand_tokens(it.t_en, it.dur)
        assert np.array_equal(asr, tp["asr"])
        g = tp["spec"]
        ref, spec, _ = O.synth_item(oracle_model, it, taps=True)
        mag_err = np.abs(g[:11] - spec[:11]).max() / max(np.abs(spec[:11]).max(), 1e-6)
        dphi = np.angle(np.exp(1j * (g[11:].astype(np.float64) - spec[11:])))
        energetic = spec[:11] > 1e-4 * spec[:11].max()
        flips = unstable_phase_bins(g, spec)
        assert mag_err < 1e-4 and np.abs(dphi[energetic]).max() < 1e-3
        note = ""
        if it.n_frames in ILL_CONDITIONED_N:
            x = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
            with O.bf16_emulation():
                xe = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
            d_gpu, d_emu = snr_db(x, tp["dec"]), snr_db(x, xe)
            note = f" decoder snr {d_gpu:.1f} (emulation {d_emu:.1f}); generator from the GPU decoder and spectrum"
            assert d_gpu >= min(d_emu, 40.0) - 6.0
            ref, _ = oracle_model.generator_from_spec(tp["dec"], g, it.ref_s)
        elif flips:
            note = " (generator from the GPU spectrum)"
            x = oracle_model.decoder(asr, it.f0, it.energy, it.ref_s)
            ref, _ = oracle_model.generator_from_spec(x, g, it.ref_s)
        else:
            end_to_end += 1
        _print(f"  {label} N {it.n_frames}: mag err {mag_err:.3g} phase err {np.abs(dphi[energetic]).max():.3g} "
               f"phase-unstable bins {flips} audio snr {snr_db(ref, a):.2f} maxabs {np.abs(a - ref).max():.3g}{note}")
        assert np.abs(a - ref).max() <= 2e-3
        assert snr_db(ref, a) >= 40.0
    return end_to_end, outs


