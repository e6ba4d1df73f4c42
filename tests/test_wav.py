"""Output formats (src/wav.rs): the PCM_16 rule and the canonical WAV header.

CPU: the oracle's restatement pinned independently -- the header against Python's `wave` module
(a library writer of the same canonical PCM header) and field by field for float32, the PCM_16
rule against hand-derived values of the reference's own test line (src/wav.rs:207-213) and
against Python's built-in round() (round half to even) on exact ties; then the library's header
(host code, no GPU) against the oracle, including the 4 GiB limit (src/wav.rs:234-242).
GPU: the device encoder, on edge values and on a plan's audio, bit-exact against the oracle."""
import io
import struct
import wave

import numpy as np
import pytest

from oracle import oracle as O

MAX_DATA = 0xFFFFFFFF - 36


def _ties(n=64):
    """f32 samples whose f32 product with 32767 is exactly k + 0.5 (found by brute force)."""
    out = []
    for k in range(-32000, 32000, 97):
        s = np.float32((k + 0.5) / 32767.0)
        for cand in (s, np.nextafter(s, np.float32(2)), np.nextafter(s, np.float32(-2))):
            if float(np.float32(cand) * np.float32(32767.0)) == k + 0.5:
                out.append(np.float32(cand))
                break
        if len(out) >= n:
            break
    return np.array(out, np.float32)


def test_oracle_header_matches_python_wave():
    for n, sr in [(0, 24000), (1, 24000), (12345, 22050), (600 * 7, 48000)]:
        buf = io.BytesIO()
        with wave.open(buf, "wb") as w:
            w.setnchannels(1), w.setsampwidth(2), w.setframerate(sr)
            w.writeframes(b"\0\0" * n)
        assert O.wav_header(0, sr, 2 * n) == buf.getvalue()[:44]


def test_oracle_float32_header_fields():
    h = O.wav_header(1, 24000, 4000)
    riff, size, wavefmt, fmtlen, tag, ch, sr, br, align, bits, data, dbytes = struct.unpack("<4sI8sIHHIIHH4sI", h)
    assert (riff, size, wavefmt, fmtlen) == (b"RIFF", 4036, b"WAVEfmt ", 16)
    assert (tag, ch, sr, br, align, bits, data, dbytes) == (3, 1, 24000, 96000, 4, 32, b"data", 4000)
    # riff_size_limit_is_enforced_not_wrapped (src/wav.rs:234-242)
    assert struct.unpack("<I", O.wav_header(0, 24000, MAX_DATA)[4:8])[0] == 0xFFFFFFFF
    for bad in (MAX_DATA + 1, 0xFFFFFFFF + 10):
        with pytest.raises(ValueError):
            O.wav_header(0, 24000, bad)


def test_oracle_pcm16_rule():
    # the reference test's clipping line (src/wav.rs:210), by hand:
    # 0.25 * 32767 = 8191.75 -> 8192; -1.5 and 1.5 clip to -32768 / 32767; 0; -0.3333 * 32767 = -10921.2 -> -10921
    out, clipped = O.encode_pcm16([0.25, -1.5, 1.5, 0.0, -0.3333])
    assert list(out) == [8192, -32768, 32767, 0, -10921] and clipped == 2
    # +-1 and the bounds: -32768 is inside the range (-1.0000305 * 32767 rounds to -32768)
    out, clipped = O.encode_pcm16([1.0, -1.0, -1.0000305, 1.0000153, -1.0000459])
    assert list(out) == [32767, -32767, -32768, 32767, -32768] and clipped == 2
    # NaN counts and stores 0; infinities count and clamp
    out, clipped = O.encode_pcm16([np.nan, np.inf, -np.inf])
    assert list(out) == [0, 32767, -32768] and clipped == 3
    # exact ties go to the even neighbour (Python's round() is round-half-even on the exact value)
    t = _ties()
    assert len(t) >= 32
    out, _ = O.encode_pcm16(t)
    assert list(out) == [round(float(x * np.float32(32767.0))) for x in t]


def test_library_header_equals_oracle():
    from kokoro_hip import api
    for fmt in (api.WAV_PCM16, api.WAV_FLOAT32):
        for sr, nb in [(24000, 0), (24000, 1200), (16000, 77), (24000, MAX_DATA)]:
            assert api.wav_header(fmt, sr, nb) == O.wav_header(fmt, sr, nb)
        with pytest.raises(api.KKError):
            api.wav_header(fmt, 24000, MAX_DATA + 1)
    with pytest.raises(api.KKError):
        api.wav_header(7, 24000, 10)


def _edge_samples():
    rng = np.random.default_rng(71)
    lines = [np.sin(np.arange(1000, dtype=np.float32) * np.float32(0.01)) * np.float32(0.5),
             np.array([0.25, -1.5, 1.5, 0.0, -0.3333], np.float32),
             ((np.arange(777) % 17).astype(np.float32) - 8.0) / np.float32(9.0)]  # src/wav.rs:207-213
    edge = np.array([1.0, -1.0, -1.0000305, 1.0000153, -1.0000459, 0.0, -0.0, np.nan, np.inf, -np.inf, 3e38,
                     -3e38, 1e-30, 0.5 / 32767, -0.5 / 32767], np.float32)
    return np.concatenate(lines + [edge, _ties(), rng.normal(0, 0.6, 5000).astype(np.float32)])


@pytest.mark.gpu
def test_device_pcm16_bit_exact(gpu_ctx):
    a = _edge_samples()
    for n in (len(a), 513, 1, 0):
        got, clipped = gpu_ctx.encode_pcm16(a[:n])
        want, wclip = O.encode_pcm16(a[:n])
        assert np.array_equal(got, want) and clipped == wclip, n


@pytest.mark.gpu
def test_plan_fetch_pcm16(gpu_ctx):
    from kokoro_hip import api, workloads
    items = workloads.small_items(72, [9, 3, 14])
    with api.Plan.decoder(gpu_ctx, items) as plan:
        plan.run()
        audio = plan.fetch()
        pcm, clipped = plan.fetch_pcm16()
    for a, p, c in zip(audio, pcm, clipped):
        want, wclip = O.encode_pcm16(a)
        assert p.shape == a.shape and np.array_equal(p, want) and c == wclip


@pytest.mark.gpu
def test_plan_fetch_pcm16_async(gpu_ctx):
    """The asynchronous fetch into pinned memory: the same bits as the synchronous fetch, gap samples
    0, and a run of the next batch enqueued before the wait does not disturb the copy."""
    from kokoro_hip import api, workloads
    items = workloads.small_items(73, [5, 11, 2])
    other = workloads.small_items(74, [12, 4, 9])  # a different batch of the same shape
    with api.Plan.decoder(gpu_ctx, items) as plan, api.Plan.decoder(gpu_ctx, other) as plan2:
        plan.run()
        pcm, clipped = plan.fetch_pcm16()
        ln = plan.info()["ln"]
        dst = gpu_ctx.host_alloc(600 * ln, np.int16)
        clip = gpu_ctx.host_alloc(len(items), np.int64)
        try:
            dst.array[:] = 12345
            plan.fetch_pcm16_async(dst, clip)
            plan.run()  # the next batch on the same plan, enqueued before the wait
            plan2.run()
            plan.fetch_wait()
            got = dst.array.copy()
            covered = np.zeros(got.size, bool)
            for b in range(len(items)):
                off, cnt = plan.item_samples(b)
                assert cnt == pcm[b].size
                assert np.array_equal(got[off:off + cnt], pcm[b]), b
                covered[off:off + cnt] = True
            assert not got[~covered].any()  # gap samples
            assert np.array_equal(clip.array, clipped)
            # a second fetch without a wait is refused; one into pageable memory too
            plan.fetch_pcm16_async(dst)
            with pytest.raises(api.KKError, match="not been waited"):
                plan.fetch_pcm16_async(dst)
            plan.fetch_wait()
            plan.fetch_wait()  # nothing pending: a no-op
            pageable = api.PinnedArray.__new__(api.PinnedArray)
            host = np.zeros(600 * ln, np.int16)
            pageable.ptr = api.C.c_void_p(host.ctypes.data)
            with pytest.raises(api.KKError, match="pinned"):
                plan.fetch_pcm16_async(pageable)
        finally:
            dst.free()
            clip.free()
