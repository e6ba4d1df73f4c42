"""Properties of the HIP path that hold at any size, through the C ABI.

- Determinism: the same inputs give byte-identical audio run after run, through a reused plan and
  through the one-shot entry (src/gpu_batch.rs contract: tests/bf16x_regression.rs:34-45).
- Per-item independence: an item's audio does not depend on its neighbours or its position in the
  batch (docs/design/BATCHING.md:26-42): bit for bit, alone, first, last, between other items.
  Tiles never span items and statistics combine per item in a fixed order, so nothing else may
  differ.
- Fixed noise (ItemNoise::Fixed, src/gpu_batch.rs:14-17, 319-350): caller-provided rand_ini and
  sine noise replace the counter stream, against the oracle on the same arrays.
- Edge sizes: one-frame and two-frame items (the smallest domains: 2 generator frames, 121 stage-1
  columns) and one long item.
Oracle comparisons use the north-star bar (max-abs <= 2e-3, SNR >= 40 dB) on the audio and check
the source spectrum on its own (see gpu_checks.check_vs_oracle for the one ill-conditioned step).
"""
import numpy as np
import pytest

from conftest import snr_db
from gpu_checks import ILL_CONDITIONED_N, check_vs_oracle

pytestmark = pytest.mark.gpu


def _print(*a):
    print(*a, flush=True)


def _run(ctx, items):
    from kokoro_hip import api
    with api.Plan.decoder(ctx, items) as plan:
        plan.run()
        return plan.fetch()


def test_rerun_and_one_shot_bit_identical(gpu_ctx):
    """Runs of one plan repeat bit for bit, with another plan's run and a stage run between them."""
    from kokoro_hip import api, workloads
    items = workloads.small_items(61, [11, 5, 17])
    with api.Plan.decoder(gpu_ctx, items) as plan:
        runs = []
        for i in range(4):
            plan.run()
            runs.append(plan.fetch())
            if i == 2:
                _run(gpu_ctx, workloads.small_items(60, [6, 9]))
                plan.run(until="gen0")
    c = gpu_ctx.forward_decoder_batch(items)
    for r in runs[1:] + [c]:
        for x, y in zip(runs[0], r):
            assert np.array_equal(x, y)


def test_concurrent_chains_match_serial(gpu_ctx):
    """The resblock chains on three streams (the default) and in one stream (per-launch profiling
    runs them serially) give the same bits: stage 0's output and the audio."""
    from kokoro_hip import api, workloads
    items = workloads.small_items(65, [14, 3, 22, 8])
    outs = []
    for prof in (False, True, False):
        gpu_ctx.set_profiling(prof)
        try:
            with api.Plan.decoder(gpu_ctx, items) as plan:
                plan.run(until="gen0")  # stage 0's chains
                taps = [plan.tap("gen0", b, (256, 20 * it.n_frames)) for b, it in enumerate(items)]
                plan.run()
                outs.append((taps, plan.fetch()))
        finally:
            gpu_ctx.set_profiling(False)
    for taps, audio in outs[1:]:
        for x, y in zip(outs[0][0], taps):
            assert np.array_equal(x, y)
        for x, y in zip(outs[0][1], audio):
            assert np.array_equal(x, y)


def test_item_independent_of_batch(gpu_ctx):
    from kokoro_hip import workloads
    a, b, c, d = workloads.small_items(62, [13, 4, 21, 9])
    alone = _run(gpu_ctx, [a])[0]
    _print("item alone:", alone.shape)
    for batch, pos in [([a, b, c], 0), ([c, b, a], 2), ([d, a, c], 1), ([b, a], 1)]:
        out = _run(gpu_ctx, batch)[pos]
        assert np.array_equal(out, alone), f"position {pos} of {len(batch)}"


def test_fixed_noise_vs_oracle(gpu_ctx, oracle_model):
    """Caller-provided noise against the oracle on the same arrays (at least one item end to end)."""
    from kokoro_hip import workloads
    rng = np.random.default_rng(63)
    items = workloads.small_items(63, [8, 15])
    for it in items:
        it.rand_ini = rng.uniform(-1.0, 1.0, 9).astype(np.float32)
        it.sine = rng.standard_normal(600 * it.n_frames * 9).astype(np.float32)
    end_to_end, outs = check_vs_oracle(gpu_ctx, oracle_model, items, "fixed noise")
    assert end_to_end >= 1
    # the counter stream is not used: a different seed changes nothing
    items[0].seed ^= 0x5555
    again = _run(gpu_ctx, items)
    assert np.array_equal(again[0], outs[0])


@pytest.mark.parametrize("ns", [[1], [2, 1], [1, 3, 2], [5, 4]])
def test_tiny_items_vs_oracle(gpu_ctx, oracle_model, ns):
    from kokoro_hip import workloads
    check_vs_oracle(gpu_ctx, oracle_model, workloads.small_items(64 + len(ns), ns), "tiny")


def test_long_item_vs_oracle(gpu_ctx, oracle_model):
    """One 600-frame item (15 s of audio) between two short ones."""
    from kokoro_hip import workloads
    check_vs_oracle(gpu_ctx, oracle_model, workloads.small_items(67, [7, 600, 3]), "long")


def test_one_shot_reuses_memory(gpu_ctx, monkeypatch):
    """kk_forward_decoder_batch keeps its device buffers between calls and does not clear them: every
    value a run reads must have been written earlier in the same run.  With the poison hook every
    buffer is filled with NaN bytes before each call, so a read of anything stale or unwritten
    (a gap row, a pad channel, a previous batch's data) would reach the audio.  Batches of growing
    and shrinking layouts, one after another, must equal fresh plans bit for bit."""
    from kokoro_hip import workloads
    batches = [workloads.small_items(71, [30, 7, 44]), workloads.small_items(72, [5, 61]),
               workloads.small_items(73, [12, 3, 25, 9, 1]), workloads.small_items(74, [2])]
    fresh = [_run(gpu_ctx, b) for b in batches]
    for poison in ("1", None):
        if poison:
            monkeypatch.setenv("KOKORO_HIP_TEST_POISON", poison)
        else:
            monkeypatch.delenv("KOKORO_HIP_TEST_POISON", raising=False)
        for i, (b, f) in enumerate(zip(batches, fresh)):
            out = gpu_ctx.forward_decoder_batch(b)
            for j, (x, y) in enumerate(zip(f, out)):
                assert np.isfinite(y).all() and np.array_equal(x, y), f"poison {poison} batch {i} item {j}"
    _print("  one-shot reuse: 4 batches x 2 passes bit-identical to fresh plans")


def test_gap_mask_negative_control(gpu_ctx, oracle_model, monkeypatch):
    """The reference proves its batch tests detect padding contamination by switching gap masking
    off (KOKORO_BATCH_NEGCTL_NOMASK, src/gpu_batch.rs:62-66; tests/bf16x_regression.rs:47-55).  The
    same hook here makes every convolution read an item's neighbours and gaps as its own rows; the
    checks this suite relies on must then fail: the batch's audio changes, an item in the batch no
    longer equals its run alone (with masking), and items fall below the oracle bar.  Unmasked,
    convolutions also read rows no kernel of the run wrote (gaps, and conv_post's bf16 operand rows
    over stale f32 words), so that audio may hold non-finite values: they count as different, and
    as failing the bar."""
    from kokoro_hip import workloads
    from oracle import oracle as O
    items = workloads.small_items(75, [9, 14, 6])
    masked = _run(gpu_ctx, items)
    alone = _run(gpu_ctx, [items[1]])[0]
    assert np.array_equal(alone, masked[1])
    monkeypatch.setenv("KOKORO_BATCH_NEGCTL_NOMASK", "1")
    unmasked = _run(gpu_ctx, items)
    monkeypatch.delenv("KOKORO_BATCH_NEGCTL_NOMASK")
    assert all(np.isfinite(a).all() for a in masked)
    assert not np.array_equal(alone, unmasked[1])
    failing = 0
    for it, a, u in zip(items, masked, unmasked):
        ref = O.synth_item(oracle_model, it)
        ok_m = np.abs(a - ref).max() <= 2e-3 and snr_db(ref, a) >= 40.0
        ok_u = np.abs(u - ref).max() <= 2e-3 and snr_db(ref, u) >= 40.0
        _print(f"  N {it.n_frames}: masked snr {snr_db(ref, a):.1f} maxabs {np.abs(a - ref).max():.3g} | "
               f"unmasked snr {snr_db(ref, u):.1f} maxabs {np.abs(u - ref).max():.3g}")
        failing += not ok_u
    assert failing >= 1
