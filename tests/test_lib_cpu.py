"""The HIP library on the CPU: it loads, exports every entry point include/kokoro_hip.h declares,
and its host-side rules (durations, ragged layout, expansion table) equal the oracle's bit for bit.
No compute call is made here (there is no GPU in this container)."""
import os
import re

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    src = open(os.path.join(ROOT, "include", "kokoro_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(kk_[a-z_0-9]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    from kokoro_hip import api
    L = api.lib()
    syms = header_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing
    assert set(syms) == set(api.EXPORTS)


def test_identity():
    from kokoro_hip import api
    assert "gfx950" in api.identity() and "bf16" in api.identity()


def test_durations_bit_exact():
    from kokoro_hip import api
    rng = np.random.default_rng(1)
    for speed in (0.8, 1.0, 1.3, 2.0):
        lg = rng.normal(0, 4, (300, 50)).astype(np.float32)
        assert np.array_equal(api.durations_from_logits(lg, speed), O.durations_from_logits(lg, speed))
    z = np.zeros((4, 50), np.float32)
    assert list(api.durations_from_logits(z, 2.0)) == [12] * 4  # 12.5 -> 12 (ties to even)
    # Rust's saturating `as i64` (src/model.rs:96): a NaN sum -> 0 -> clamped to 1; a sum past 2^63
    # (a tiny speed) -> i64::MAX; -inf logits give a sum of 0 -> 1
    odd = np.zeros((3, 50), np.float32)
    odd[0, 7] = np.nan
    odd[2, :] = -np.inf
    for speed in (1.0, 1e-30):
        got = api.durations_from_logits(odd, speed)
        assert np.array_equal(got, O.durations_from_logits(odd, speed))
    assert list(api.durations_from_logits(odd, 1.0)) == [1, 25, 1]
    assert list(api.durations_from_logits(odd, 1e-30)) == [1, 2**63 - 1, 1]


def test_layout_bit_exact():
    from kokoro_hip import api
    rng = np.random.default_rng(2)
    for _ in range(5):
        nfs = rng.integers(1, 900, int(rng.integers(1, 40)))
        a1, l1 = api.layout_frames(nfs)
        a2, l2 = O.layout_frames(nfs)
        assert l1 == l2 and np.array_equal(a1, a2)
        for f, add in [(1, 0), (2, 0), (20, 0), (120, 1)]:
            l = f * l1 + add
            assert np.array_equal(api.layout_col_item(l, a1 * f, nfs * f + add),
                                  O.layout_col_item(l, a1 * f, nfs * f + add))
        durs = [rng.integers(1, 8, int(rng.integers(1, 30))) for _ in range(len(nfs))]
        tstart = np.concatenate([[0], np.cumsum([len(d) + 2 for d in durs])[:-1]])
        a, ln = O.layout_frames([d.sum() for d in durs])
        assert np.array_equal(api.layout_src_row(durs, tstart, a, ln), O.layout_src_row(durs, tstart, a, ln))


def test_layout_errors():
    from kokoro_hip import api
    with pytest.raises(api.KKError):
        api.layout_col_item(10, [0, 5], [6, 3])
    with pytest.raises(api.KKError):
        api.durations_from_logits(np.zeros((2, 50), np.float32), 0.0)


def test_weight_spec_shapes():
    """The tensor table is the decoder + generator of Kokoro-82M (src/vocoder.rs:54-111)."""
    from kokoro_hip import model_spec
    spec = {n: s for n, s, _, _ in model_spec.tensor_spec()}
    assert spec["decoder.generator.ups.0.weight"] == (512, 256, 20)
    assert spec["decoder.generator.ups.1.weight"] == (256, 128, 12)
    assert spec["decoder.generator.resblocks.5.convs1.2.weight"] == (128, 128, 11)
    assert spec["decoder.decode.3.pool.weight"] == (1090, 1, 3)
    assert spec["decoder.generator.conv_post.weight"] == (22, 128, 7)
    assert 53.0e6 < model_spec.param_count() < 53.6e6
