"""ctypes front end of the CPU oracle (oracle/kk_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
"""
from __future__ import annotations

import ctypes as C
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# KK_ORACLE_LIB: another build of the same source (the sanitizer test loads an ASan + UBSan build)
LIB_PATH = os.environ.get("KK_ORACLE_LIB") or os.path.join(HERE, "libkk_oracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run oracle/build_oracle.py)")
        L = C.CDLL(LIB_PATH)
        L.ko_set_bf16_emulation.argtypes = [C.c_int]
        L.ko_set_operand_formats.argtypes = [C.c_int, C.c_int]
        L.ko_weight_norm.argtypes = [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64, C.c_void_p]
        L.ko_weight_norm.restype = None
        L.ko_set_threads.argtypes = [C.c_int]
        L.ko_bf16_round.argtypes = [C.c_float]
        L.ko_bf16_round.restype = C.c_float
        L.ko_layout_frames.argtypes = [_i64p, C.c_int, C.c_int, _i64p, C.POINTER(C.c_int64)]
        L.ko_layout_col_item.argtypes = [C.c_int64, _i64p, _i64p, C.c_int, _i32p]
        L.ko_layout_src_row.argtypes = [C.POINTER(C.c_void_p), _i64p, C.c_int, _i64p, _i64p, C.c_int64, _i32p]
        L.ko_durations_from_logits.argtypes = [_f32p, C.c_int, C.c_float, _i64p]
        L.ko_conv1d.argtypes = [_f32p, C.c_int, C.c_int, _f32p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_int, _f32p, C.c_int]
        L.ko_conv_transpose1d.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                          _f32p, C.c_int]
        L.ko_chan_stats.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _f32p]
        L.ko_style_fc.argtypes = [_f32p, _f32p, C.c_int, _f32p, _f32p]
        L.ko_adain_apply.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _f32p, _f32p, _f32p, _f32p, C.c_int, C.c_float,
                                     C.c_void_p, _f32p]
        L.ko_splitmix_at.argtypes = [C.c_uint64, C.c_uint64]
        L.ko_splitmix_at.restype = C.c_uint64
        L.ko_rand_ini.argtypes = [C.c_uint64, _f32p]
        L.ko_gen_noise.argtypes = [C.c_uint64, _f32p, C.c_int64]
        L.ko_sine_source.argtypes = [_f32p, C.c_int, _f32p, _f32p, _f32p, C.c_float, C.c_void_p, _f32p]
        L.ko_stft20.argtypes = [_f32p, C.c_int, _f32p, C.c_int]
        L.ko_istft20.argtypes = [_f32p, C.c_int, _f32p]
        L.ko_model_create.argtypes = [C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_void_p), _i64p,
                                      C.POINTER(C.c_void_p), C.c_char_p, C.c_size_t]
        L.ko_model_free.argtypes = [C.c_void_p]
        L.ko_decoder_forward.argtypes = [C.c_void_p, _f32p, _f32p, _f32p, _f32p, C.c_int, _f32p]
        L.ko_generator_forward.argtypes = [C.c_void_p, _f32p, _f32p, _f32p, C.c_int, _f32p, _f32p, _f32p,
                                           C.c_void_p, C.c_void_p]
        L.ko_generator_from_spec.argtypes = [C.c_void_p, _f32p, _f32p, _f32p, C.c_int, _f32p, C.c_void_p]
        L.ko_snake_block_forward.argtypes = [C.c_void_p, C.c_char_p, _f32p, C.c_int, _f32p, _f32p]
        L.ko_resblk_forward.argtypes = [C.c_void_p, C.c_char_p, _f32p, C.c_int, _f32p, _f32p]
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _chk(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} failed (rc={rc})")


GROUP_DECODER, GROUP_SNAKE, GROUP_POST, GROUP_UPS, GROUP_H16 = 1, 2, 4, 8, 16


class operand_formats:
    """Context manager: round the operands of the layer groups in `groups` (GROUP_*) to bf16, those
    also in `fp16_groups` to fp16 instead (error-budget analysis)."""

    def __init__(self, groups, fp16_groups=0):
        self.groups, self.fp16 = groups, fp16_groups

    def __enter__(self):
        lib().ko_set_operand_formats(self.groups, self.fp16)

    def __exit__(self, *a):
        lib().ko_set_bf16_emulation(0)


class bf16_emulation:
    """Context manager: round MFMA-layer operands to bf16 inside the oracle."""

    def __init__(self, on=True):
        self.on = on

    def __enter__(self):
        lib().ko_set_bf16_emulation(int(self.on))

    def __exit__(self, *a):
        lib().ko_set_bf16_emulation(0)


def weight_norm(v, g):
    """weight_norm (src/ops.rs:9-23) over the first dimension of v."""
    v = _f32(v)
    g = _f32(g).reshape(-1)
    w = np.empty_like(v)
    lib().ko_weight_norm(v.ctypes.data, g.ctypes.data, v.shape[0], v.size // max(v.shape[0], 1), w.ctypes.data)
    return w


def set_threads(n):
    lib().ko_set_threads(int(n))


# ------------------------------------------------------------------ layout


def layout_frames(nfs, gap=2):
    nfs = np.ascontiguousarray(nfs, dtype=np.int64)
    a = np.zeros(len(nfs), np.int64)
    ln = C.c_int64()
    _chk(lib().ko_layout_frames(nfs, len(nfs), gap, a, C.byref(ln)), "layout_frames")
    return a, int(ln.value)


def layout_col_item(l, start, length):
    start = np.ascontiguousarray(start, dtype=np.int64)
    length = np.ascontiguousarray(length, dtype=np.int64)
    out = np.zeros(l, np.int32)
    _chk(lib().ko_layout_col_item(l, start, length, len(start), out), "layout_col_item")
    return out


def layout_src_row(durs, tstart, a, ln):
    durs = [np.ascontiguousarray(d, dtype=np.int64) for d in durs]
    ptrs = (C.c_void_p * len(durs))(*[d.ctypes.data for d in durs])
    ntok = np.asarray([len(d) for d in durs], np.int64)
    out = np.zeros(ln, np.int32)
    _chk(lib().ko_layout_src_row(ptrs, ntok, len(durs), np.ascontiguousarray(tstart, np.int64),
                                 np.ascontiguousarray(a, np.int64), ln, out), "layout_src_row")
    return out


def durations_from_logits(logits, speed):
    logits = _f32(logits)
    t = logits.shape[0]
    out = np.zeros(t, np.int64)
    lib().ko_durations_from_logits(logits.reshape(-1), t, float(speed), out)
    return out


# ------------------------------------------------------------------ output formats (src/wav.rs)


def encode_pcm16(audio):
    """wav::encode, PCM_16 (src/wav.rs:63-80): v = (s * 32767).round_ties_even() in f32; a sample
    counts as clipped when v is outside [-32768, 32767] (NaN included); the stored value is v
    clamped, and NaN becomes 0 (Rust's saturating `as i16`).  Returns (int16 samples, clipped)."""
    a = np.asarray(audio, np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        v = np.rint(a * np.float32(32767.0))  # f32 product, round half to even
        inside = (v >= np.float32(-32768.0)) & (v <= np.float32(32767.0))
        out = np.where(np.isnan(v), np.float32(0.0), np.clip(v, -32768.0, 32767.0)).astype(np.int16)
    return out, int(np.count_nonzero(~inside))


def wav_header(fmt, sample_rate, data_bytes):
    """wav::header (src/wav.rs:43-61): canonical 44-byte mono RIFF/WAVE header, format tag 1
    (fmt 0, PCM_16) or 3 (fmt 1, float32); ValueError past check_riff_size (src/wav.rs:34-40)."""
    if data_bytes > 0xFFFFFFFF - 36:
        raise ValueError(f"the audio ({data_bytes} bytes) exceeds the 4 GiB limit of a WAV file")
    bits, tag = (16, 1) if fmt == 0 else (32, 3)
    return struct.pack("<4sI8sIHHIIHH4sI", b"RIFF", 36 + data_bytes, b"WAVEfmt ", 16, tag, 1, sample_rate,
                       sample_rate * bits // 8, bits // 8, bits, b"data", data_bytes)


# ------------------------------------------------------------------ primitives


def conv1d(x, w, b, stride=1, pad=0, dil=1):
    x, w = _f32(x), _f32(w)
    cin, t = x.shape
    cout, _, k = w.shape
    tout = (t + 2 * pad - dil * (k - 1) - 1) // stride + 1
    y = np.zeros((cout, tout), np.float32)
    bb = _f32(b) if b is not None else None
    _chk(lib().ko_conv1d(x, cin, t, w, bb.ctypes.data if bb is not None else None, cout, k, stride, pad, dil, y, tout),
         "conv1d")
    return y


def conv_transpose1d(x, w, b, stride, pad):
    x, w, b = _f32(x), _f32(w), _f32(b)
    cin, t = x.shape
    _, cout, k = w.shape
    tout = (t - 1) * stride + k - 2 * pad
    y = np.zeros((cout, tout), np.float32)
    _chk(lib().ko_conv_transpose1d(x, cin, t, w, b, cout, k, stride, pad, y, tout), "conv_transpose1d")
    return y


def chan_stats(x):
    x = _f32(x)
    c, t = x.shape
    m = np.zeros(c, np.float32)
    r = np.zeros(c, np.float32)
    lib().ko_chan_stats(x, c, t, m, r)
    return m, r


def style_fc(w, b, s):
    w, b, s = _f32(w), _f32(b), _f32(s)
    gb = np.zeros(w.shape[0], np.float32)
    lib().ko_style_fc(w, b, w.shape[0], s, gb)
    return gb


def adain_apply(x, mean, rstd, nw, nb, gb, mode, slope=0.2, alpha=None):
    x = _f32(x)
    c, t = x.shape
    y = np.zeros_like(x)
    al = _f32(alpha) if alpha is not None else None
    lib().ko_adain_apply(x, c, t, _f32(mean), _f32(rstd), _f32(nw), _f32(nb), _f32(gb), mode, slope,
                         al.ctypes.data if al is not None else None, y)
    return y


def splitmix_at(seed, ctr):
    return int(lib().ko_splitmix_at(seed, ctr))


def rand_ini(seed):
    out = np.zeros(9, np.float32)
    lib().ko_rand_ini(seed, out)
    return out


def gen_noise(seed, n):
    out = np.zeros(n, np.float32)
    lib().ko_gen_noise(seed, out, n)
    return out


def sine_source(f0c, rand_ini_, noise, lw, lb, want_phase=False):
    f0c = _f32(f0c)
    l = len(f0c)
    har = np.zeros(300 * l, np.float32)
    pp = np.zeros((9, l), np.float32) if want_phase else None
    _chk(lib().ko_sine_source(f0c, l, _f32(rand_ini_), _f32(noise), _f32(lw).reshape(-1), float(lb),
                              pp.ctypes.data if pp is not None else None, har), "sine_source")
    return (har, pp) if want_phase else har


def stft20(x):
    x = _f32(x)
    f = 1 + len(x) // 5
    out = np.zeros((22, f), np.float32)
    _chk(lib().ko_stft20(x, len(x), out, f), "stft20")
    return out


def istft20(post):
    post = _f32(post)
    f = post.shape[1]
    out = np.zeros(5 * (f - 1), np.float32)
    _chk(lib().ko_istft20(post, f, out), "istft20")
    return out


# ------------------------------------------------------------------ model


class Model:
    def __init__(self, weights: dict):
        names = list(weights.keys())
        self._arrs = [_f32(weights[n]).reshape(-1) for n in names]
        cn = (C.c_char_p * len(names))(*[n.encode() for n in names])
        ptrs = (C.c_void_p * len(names))(*[a.ctypes.data for a in self._arrs])
        numel = np.asarray([a.size for a in self._arrs], np.int64)
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = lib().ko_model_create(len(names), cn, ptrs, numel, C.byref(h), err, 512)
        if rc != 0:
            raise ValueError("oracle model: " + err.value.decode())
        self.h = h
        self._arrs = None  # the oracle copied every tensor
        self.l_w = _f32(weights["decoder.generator.m_source.l_linear.weight"]).reshape(-1)
        self.l_b = float(weights["decoder.generator.m_source.l_linear.bias"][0])

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.ko_model_free(self.h)
            self.h = None

    def decoder(self, asr, f0, en, style):
        asr = _f32(asr)
        n = asr.shape[1]
        out = np.zeros((512, 2 * n), np.float32)
        _chk(lib().ko_decoder_forward(self.h, asr, _f32(f0), _f32(en), _f32(style[:128]), n, out), "decoder")
        return out

    def generator(self, x, f0, style, rand_ini_, noise, taps=False):
        x = _f32(x)
        n = x.shape[1] // 2
        audio = np.zeros(600 * n, np.float32)
        spec = np.zeros((22, 120 * n + 1), np.float32) if taps else None
        post = np.zeros((22, 120 * n + 1), np.float32) if taps else None
        _chk(lib().ko_generator_forward(self.h, x, _f32(f0), _f32(style[:128]), n, _f32(rand_ini_), _f32(noise),
                                        audio, spec.ctypes.data if taps else None,
                                        post.ctypes.data if taps else None), "generator")
        return (audio, spec, post) if taps else audio

    def generator_from_spec(self, x, spec, style):
        x = _f32(x)
        n = x.shape[1] // 2
        audio = np.zeros(600 * n, np.float32)
        post = np.zeros((22, 120 * n + 1), np.float32)
        _chk(lib().ko_generator_from_spec(self.h, x, _f32(spec), _f32(style[:128]), n, audio, post.ctypes.data),
             "generator_from_spec")
        return audio, post

    def snake_block(self, prefix, x, style):
        x = _f32(x)
        out = np.zeros_like(x)
        _chk(lib().ko_snake_block_forward(self.h, prefix.encode(), x, x.shape[1], _f32(style[:128]), out),
             "snake_block")
        return out

    def resblk(self, prefix, x, style, dout, upsample=False):
        x = _f32(x)
        t = x.shape[1]
        out = np.zeros((dout, 2 * t if upsample else t), np.float32)
        _chk(lib().ko_resblk_forward(self.h, prefix.encode(), x, t, _f32(style[:128]), out), "resblk")
        return out


def expand_tokens(t_en, dur):
    """asr[:, f] = t_en[:, token of frame f] (src/gpu_batch.rs:265-297, per item)."""
    idx = np.repeat(np.arange(len(dur)), dur)
    return np.ascontiguousarray(t_en[:, idx])


def item_noise(item):
    n = item.n_frames
    if item.sine is not None:
        return _f32(item.rand_ini), _f32(item.sine)
    return rand_ini(item.seed), gen_noise(item.seed, 600 * n * 9)


def synth_item(model: Model, item, taps=False):
    """Decoder + generator for one DecoderItem -> audio [600 N] (and optional taps)."""
    asr = expand_tokens(item.t_en, item.dur)
    x = model.decoder(asr, item.f0, item.energy, item.ref_s)
    ri, nz = item_noise(item)
    return model.generator(x, item.f0, item.ref_s, ri, nz, taps=taps)
