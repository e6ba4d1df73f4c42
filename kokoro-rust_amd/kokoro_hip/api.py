"""ctypes binding of libkokoro_hip.so (the C ABI declared in include/kokoro_hip.h).

The library is the product; this module only marshals numpy arrays into the ABI's plain pointers.
It raises if the library is missing: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# KK_LIB: another build of the same sources (A/B measurements of two builds on one GPU box)
LIB_PATH = os.environ.get("KK_LIB") or os.path.join(os.path.dirname(HERE), "lib", "libkokoro_hip.so")

KK_OK = 0
KK_ERR_INVALID, KK_ERR_HIP, KK_ERR_OOM, KK_ERR_STATE = -1, -2, -3, -4
KK_NOISE_COUNTER = 0
KK_NOISE_FIXED = 1
STAGES = {"prosody": 0, "decoder": 1, "source": 2, "gen0": 3, "gen1": 4, "post": 5, "all": 6}
EXPORTS = [
    "kk_open", "kk_close", "kk_device_name", "kk_identity", "kk_upload_model", "kk_forward_decoder_batch",
    "kk_output_free", "kk_plan_create", "kk_plan_create_generator", "kk_plan_create_snake", "kk_plan_run",
    "kk_plan_sync", "kk_plan_fetch", "kk_plan_tap", "kk_plan_get_info", "kk_plan_free", "kk_set_profiling",
    "kk_profile_read", "kk_durations_from_logits", "kk_layout_frames", "kk_layout_col_item", "kk_layout_src_row",
    "kk_plan_fetch_pcm16", "kk_encode_pcm16", "kk_wav_header", "kk_host_alloc", "kk_host_free",
    "kk_plan_item_samples", "kk_plan_fetch_pcm16_async", "kk_plan_fetch_wait", "kk_snake_block_noalloc", "kk_profile_launches", "kk_checkpoint_open", "kk_checkpoint_count",
    "kk_checkpoint_entry", "kk_checkpoint_free", "kk_upload_checkpoint", "kk_weight_norm", "kk_voice_load",
    "kk_voice_free", "kk_voice_ref_s", "kk_forward_batch", "kk_result_free", "kk_plan_create_full",
    "kk_plan_durations",
]
NOALLOC_MAX_ROWS = 65536
NOALLOC_MAX_ITEMS = 64


class KKError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"kokoro_hip error {code}: {msg}")
        self.code = code


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.c_void_p), ("numel", C.c_int64)]


class DecoderItem(C.Structure):
    _fields_ = [("dur", C.c_void_p), ("n_tok", C.c_int32), ("t_en", C.c_void_p), ("f0", C.c_void_p),
                ("energy", C.c_void_p), ("ref_s", C.c_void_p), ("noise_kind", C.c_int32), ("seed", C.c_uint64),
                ("rand_ini", C.c_void_p), ("sine", C.c_void_p), ("sine_len", C.c_int64)]


class GeneratorItem(C.Structure):
    _fields_ = [("x", C.c_void_p), ("n_frames", C.c_int32), ("f0", C.c_void_p), ("ref_s", C.c_void_p),
                ("noise_kind", C.c_int32), ("seed", C.c_uint64), ("rand_ini", C.c_void_p), ("sine", C.c_void_p),
                ("sine_len", C.c_int64)]


class Output(C.Structure):
    _fields_ = [("audio", C.POINTER(C.c_float)), ("n_samples", C.c_int64)]


class Item(C.Structure):
    """kk_item: BatchItem (src/gpu_batch.rs:19-24)."""
    _fields_ = [("ids", C.c_void_p), ("n_ids", C.c_int32), ("ref_s", C.c_void_p), ("speed", C.c_float),
                ("noise_kind", C.c_int32), ("seed", C.c_uint64), ("rand_ini", C.c_void_p), ("sine", C.c_void_p),
                ("sine_len", C.c_int64)]


class Result(C.Structure):
    _fields_ = [("audio", C.POINTER(C.c_float)), ("n_samples", C.c_int64), ("pred_dur", C.POINTER(C.c_int64)),
                ("n_tok", C.c_int32)]


class PlanInfo(C.Structure):
    _fields_ = [("n_items", C.c_int64), ("ln", C.c_int64), ("frames", C.c_int64), ("samples", C.c_int64),
                ("conv_flop", C.c_double), ("snake_flop", C.c_double), ("device_bytes", C.c_int64),
                ("launches", C.c_int64)]


class LaunchRecord(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("cls", C.c_char * 32), ("ms", C.c_double), ("flop", C.c_double),
                ("bytes", C.c_double)]


class ProfileEntry(C.Structure):
    _fields_ = [("name", C.c_char * 32), ("launches", C.c_int64), ("ms", C.c_double), ("flop", C.c_double),
                ("bytes", C.c_double)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        vp, i32, i64, sz, cp = C.c_void_p, C.c_int, C.c_int64, C.c_size_t, C.c_char_p
        L.kk_open.argtypes = [i32, C.POINTER(vp), cp, sz]
        L.kk_close.argtypes = [vp]
        L.kk_close.restype = None
        L.kk_device_name.argtypes = [vp, cp, sz]
        L.kk_identity.restype = C.c_char_p
        L.kk_upload_model.argtypes = [vp, C.POINTER(Tensor), i32, cp, sz]
        L.kk_forward_decoder_batch.argtypes = [vp, C.POINTER(DecoderItem), i32, C.POINTER(Output), cp, sz]
        L.kk_output_free.argtypes = [C.POINTER(Output), i32]
        L.kk_output_free.restype = None
        L.kk_plan_create.argtypes = [vp, C.POINTER(DecoderItem), i32, C.POINTER(vp), cp, sz]
        L.kk_plan_create_generator.argtypes = [vp, C.POINTER(GeneratorItem), i32, C.POINTER(vp), cp, sz]
        L.kk_plan_create_snake.argtypes = [vp, cp, C.POINTER(vp), C.POINTER(C.c_int64), C.POINTER(vp), i32, i32,
                                           C.POINTER(vp), cp, sz]
        L.kk_plan_run.argtypes = [vp, i32, cp, sz]
        L.kk_plan_sync.argtypes = [vp, cp, sz]
        L.kk_plan_fetch.argtypes = [vp, C.POINTER(Output), cp, sz]
        L.kk_plan_tap.argtypes = [vp, cp, i32, vp, i64, cp, sz]
        L.kk_plan_fetch_pcm16.argtypes = [vp, C.POINTER(vp), vp, cp, sz]
        L.kk_encode_pcm16.argtypes = [vp, vp, i64, vp, vp, cp, sz]
        L.kk_host_alloc.argtypes = [vp, sz, C.POINTER(vp), cp, sz]
        L.kk_host_free.argtypes = [vp]
        L.kk_host_free.restype = None
        L.kk_plan_item_samples.argtypes = [vp, i32, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]
        L.kk_plan_fetch_pcm16_async.argtypes = [vp, vp, vp, cp, sz]
        L.kk_plan_fetch_wait.argtypes = [vp, cp, sz]
        L.kk_wav_header.argtypes = [i32, C.c_uint32, C.c_uint64, vp, cp, sz]
        L.kk_checkpoint_open.argtypes = [cp, C.POINTER(vp), cp, sz]
        L.kk_checkpoint_count.argtypes = [vp]
        L.kk_checkpoint_entry.argtypes = [vp, i32, C.POINTER(C.c_char_p), C.POINTER(C.POINTER(C.c_int64)),
                                          C.POINTER(C.c_int), C.POINTER(C.POINTER(C.c_float)), C.POINTER(C.c_int64)]
        L.kk_checkpoint_free.argtypes = [vp]
        L.kk_checkpoint_free.restype = None
        L.kk_upload_checkpoint.argtypes = [vp, vp, cp, sz]
        L.kk_weight_norm.argtypes = [vp, vp, i64, i64, vp]
        L.kk_voice_load.argtypes = [C.POINTER(cp), i32, C.POINTER(C.POINTER(C.c_float)), C.POINTER(C.c_int64), cp, sz]
        L.kk_voice_free.argtypes = [C.POINTER(C.c_float)]
        L.kk_voice_free.restype = None
        L.kk_voice_ref_s.argtypes = [C.POINTER(C.c_float), i64, i64, C.POINTER(C.POINTER(C.c_float))]
        L.kk_snake_block_noalloc.argtypes = [vp, cp, vp, i64, vp, vp, i32, C.POINTER(vp), cp, sz]
        L.kk_forward_batch.argtypes = [vp, C.POINTER(Item), i32, C.POINTER(Result), cp, sz]
        L.kk_result_free.argtypes = [C.POINTER(Result), i32]
        L.kk_result_free.restype = None
        L.kk_plan_create_full.argtypes = [vp, C.POINTER(Item), i32, C.POINTER(vp), cp, sz]
        L.kk_plan_durations.argtypes = [vp, i32, C.POINTER(C.POINTER(C.c_int64)), C.POINTER(C.c_int32)]
        L.kk_plan_get_info.argtypes = [vp, C.POINTER(PlanInfo)]
        L.kk_plan_free.argtypes = [vp]
        L.kk_plan_free.restype = None
        L.kk_set_profiling.argtypes = [vp, i32]
        L.kk_profile_read.argtypes = [vp, C.POINTER(ProfileEntry), i32, C.POINTER(C.c_int), cp, sz]
        L.kk_profile_launches.argtypes = [vp, C.POINTER(LaunchRecord), i32, C.POINTER(C.c_int), cp, sz]
        L.kk_durations_from_logits.argtypes = [vp, i32, C.c_float, vp]
        L.kk_layout_frames.argtypes = [vp, i32, vp]
        L.kk_layout_frames.restype = i64
        L.kk_layout_col_item.argtypes = [i64, vp, vp, i32, vp]
        L.kk_layout_src_row.argtypes = [C.POINTER(vp), vp, i32, vp, vp, i64, vp]
        _lib = L
    return _lib


def _err():
    return C.create_string_buffer(1024)


def _check(rc, err):
    if rc != KK_OK:
        raise KKError(rc, err.value.decode(errors="replace"))


def _p(a):
    return C.c_void_p(a.ctypes.data) if a is not None else C.c_void_p()


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def identity():
    return lib().kk_identity().decode()


WAV_PCM16, WAV_FLOAT32 = 0, 1


def wav_header(fmt, sample_rate, data_bytes):
    """wav::header (src/wav.rs:43-61): the canonical 44-byte mono header; KKError beyond 4 GiB."""
    out = np.zeros(44, np.uint8)
    err = _err()
    _check(lib().kk_wav_header(int(fmt), int(sample_rate), int(data_bytes), _p(out), err, len(err)), err)
    return out.tobytes()


# ------------------------------------------------------------------ checkpoints and voices


class Checkpoint:
    """kk_checkpoint_open: a torch.save model file read by the library (host only)."""

    def __init__(self, path):
        h = C.c_void_p()
        err = _err()
        _check(lib().kk_checkpoint_open(str(path).encode(), C.byref(h), err, len(err)), err)
        self.h = h

    def tensors(self):
        """{name: float32 array of its shape} (copies)."""
        out = {}
        for i in range(lib().kk_checkpoint_count(self.h)):
            nm, shp, nd, data, n = C.c_char_p(), C.POINTER(C.c_int64)(), C.c_int(), C.POINTER(C.c_float)(), C.c_int64()
            _check(lib().kk_checkpoint_entry(self.h, i, C.byref(nm), C.byref(shp), C.byref(nd), C.byref(data),
                                             C.byref(n)), _err())
            shape = tuple(shp[k] for k in range(nd.value))
            arr = np.ctypeslib.as_array(data, shape=(n.value,)).copy() if n.value else np.zeros(0, np.float32)
            out[nm.value.decode()] = arr.reshape(shape)
        return out

    def free(self):
        if getattr(self, "h", None):
            lib().kk_checkpoint_free(self.h)
            self.h = None

    def __del__(self):
        self.free()


def weight_norm(v, g):
    """kk_weight_norm over the first dimension of v."""
    v = _f32(v)
    g = _f32(g).reshape(-1)
    w = np.empty_like(v)
    rc = lib().kk_weight_norm(_p(v), _p(g), v.shape[0], v.size // max(v.shape[0], 1), _p(w))
    if rc != KK_OK:
        raise KKError(rc, "weight_norm")
    return w


def voice_load(paths):
    """kk_voice_load: the (mean) voice pack as float32 [rows, 256]."""
    enc = [str(p).encode() for p in paths]
    arr = (C.c_char_p * len(enc))(*enc)
    pack, rows = C.POINTER(C.c_float)(), C.c_int64()
    err = _err()
    _check(lib().kk_voice_load(arr, len(enc), C.byref(pack), C.byref(rows), err, len(err)), err)
    out = np.ctypeslib.as_array(pack, shape=(rows.value * 256,)).copy().reshape(rows.value, 256)
    lib().kk_voice_free(pack)
    return out


def voice_ref_s(pack, n_phoneme_chars):
    """kk_voice_ref_s on a [rows, 256] pack: its row n - 1."""
    pk = _f32(pack)
    ptr = pk.ctypes.data_as(C.POINTER(C.c_float))
    out = C.POINTER(C.c_float)()
    rc = lib().kk_voice_ref_s(ptr, pk.shape[0], int(n_phoneme_chars), C.byref(out))
    if rc != KK_OK:
        raise KKError(rc, "voice_ref_s")
    off = (C.addressof(out.contents) - pk.ctypes.data) // 4
    return pk.reshape(-1)[off:off + 256].copy()


# ------------------------------------------------------------------ host rules


def durations_from_logits(logits, speed):
    logits = _f32(logits)
    out = np.zeros(logits.shape[0], np.int64)
    rc = lib().kk_durations_from_logits(_p(logits), logits.shape[0], float(speed), _p(out))
    if rc != KK_OK:
        raise KKError(rc, "durations_from_logits")
    return out


def layout_frames(nfs):
    nfs = np.ascontiguousarray(nfs, np.int64)
    a = np.zeros(len(nfs), np.int64)
    ln = lib().kk_layout_frames(_p(nfs), len(nfs), _p(a))
    if ln < 0:
        raise KKError(int(ln), "layout_frames")
    return a, int(ln)


def layout_col_item(l, start, length):
    start = np.ascontiguousarray(start, np.int64)
    length = np.ascontiguousarray(length, np.int64)
    out = np.zeros(l, np.int32)
    rc = lib().kk_layout_col_item(l, _p(start), _p(length), len(start), _p(out))
    if rc != KK_OK:
        raise KKError(rc, "layout_col_item")
    return out


def layout_src_row(durs, tstart, a, ln):
    durs = [np.ascontiguousarray(d, np.int64) for d in durs]
    ptrs = (C.c_void_p * len(durs))(*[d.ctypes.data for d in durs])
    ntok = np.asarray([len(d) for d in durs], np.int32)
    out = np.zeros(ln, np.int32)
    tstart = np.ascontiguousarray(tstart, np.int64)
    a = np.ascontiguousarray(a, np.int64)
    rc = lib().kk_layout_src_row(ptrs, _p(ntok), len(durs), _p(tstart), _p(a), ln, _p(out))
    if rc != KK_OK:
        raise KKError(rc, "layout_src_row")
    return out


# ------------------------------------------------------------------ device objects


class Context:
    """Gpu::new + GpuKokoro::with_gpu (src/gpu.rs:81-105, 685-724) for the decoder + generator."""

    def __init__(self, ordinal=0):
        h = C.c_void_p()
        err = _err()
        _check(lib().kk_open(ordinal, C.byref(h), err, len(err)), err)
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().kk_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def device_name(self):
        buf = C.create_string_buffer(256)
        lib().kk_device_name(self.h, buf, 256)
        return buf.value.decode()

    def upload_model(self, weights: dict):
        names = list(weights.keys())
        arrs = [_f32(weights[n]).reshape(-1) for n in names]
        enc = [n.encode() for n in names]
        tab = (Tensor * len(names))(*[Tensor(e, a.ctypes.data, a.size) for e, a in zip(enc, arrs)])
        err = _err()
        _check(lib().kk_upload_model(self.h, tab, len(names), err, len(err)), err)

    def upload_checkpoint(self, ck):
        """kk_upload_checkpoint from a Checkpoint."""
        err = _err()
        _check(lib().kk_upload_checkpoint(self.h, ck.h, err, len(err)), err)

    def set_profiling(self, on):
        lib().kk_set_profiling(self.h, int(bool(on)))

    def profile_launches(self):
        """Per-launch records since the last profile_read: [(name, class, ms, flop, bytes)]."""
        n = C.c_int()
        err = _err()
        _check(lib().kk_profile_launches(self.h, None, 0, C.byref(n), err, len(err)), err)
        recs = (LaunchRecord * max(1, n.value))()
        _check(lib().kk_profile_launches(self.h, recs, n.value, C.byref(n), err, len(err)), err)
        return [(r.name.decode(), r.cls.decode(), r.ms, r.flop, r.bytes) for r in recs[: n.value]]

    def profile_read(self):
        ents = (ProfileEntry * 32)()
        n = C.c_int()
        err = _err()
        _check(lib().kk_profile_read(self.h, ents, 32, C.byref(n), err, len(err)), err)
        return {e.name.decode(): {"launches": e.launches, "ms": e.ms, "flop": e.flop, "bytes": e.bytes}
                for e in ents[: n.value]}

    # -------------------------------------------------------------- batch entry points
    def forward_decoder_batch(self, items):
        """kk_forward_decoder_batch: list of workloads.DecoderItem -> list of audio arrays."""
        arr, keep = _decoder_items(items)
        outs = (Output * len(items))()
        err = _err()
        _check(lib().kk_forward_decoder_batch(self.h, arr, len(items), outs, err, len(err)), err)
        res = [np.ctypeslib.as_array(o.audio, shape=(o.n_samples,)).copy() for o in outs]
        lib().kk_output_free(outs, len(items))
        del keep
        return res

    def forward_batch(self, items):
        """kk_forward_batch: list of workloads.IdsItem -> list of (audio, pred_dur)."""
        arr, keep = _items(items)
        outs = (Result * len(items))()
        err = _err()
        _check(lib().kk_forward_batch(self.h, arr, len(items), outs, err, len(err)), err)
        res = [(np.ctypeslib.as_array(o.audio, shape=(o.n_samples,)).copy(),
                np.ctypeslib.as_array(o.pred_dur, shape=(o.n_tok,)).copy()) for o in outs]
        lib().kk_result_free(outs, len(items))
        del keep
        return res

    def plan(self, items):
        return Plan.decoder(self, items)

    def snake_block_noalloc(self, prefix, x_ptr, rows, starts, lens, ref_ss):
        """kk_snake_block_noalloc: the Snake block in place on device memory at x_ptr (time-major f32
        [rows][C]), items at rows [starts[b], starts[b] + lens[b]); allocates nothing."""
        starts = np.ascontiguousarray(starts, np.int64)
        lens = np.ascontiguousarray(lens, np.int64)
        rss = [_f32(np.pad(np.asarray(r, np.float32), (0, max(0, 256 - len(r))))) for r in ref_ss]
        rp = (C.c_void_p * len(rss))(*[r.ctypes.data for r in rss])
        err = _err()
        _check(lib().kk_snake_block_noalloc(self.h, prefix.encode(), C.c_void_p(x_ptr), int(rows), _p(starts),
                                            _p(lens), len(lens), rp, err, len(err)), err)

    def prepare(self, items):
        """The items marshalled once into the ABI's structs, for repeated calls (timing)."""
        return PreparedBatch(items)

    def forward_prepared(self, pb):
        """kk_forward_decoder_batch on a PreparedBatch; the outputs stay in pb.outs (release with
        pb.release()).  Raises KKError on failure."""
        err = _err()
        _check(lib().kk_forward_decoder_batch(self.h, pb.arr, pb.n, pb.outs, err, len(err)), err)


    def forward_ids_prepared(self, pb):
        """kk_forward_batch on a PreparedIdsBatch; the results stay in pb.outs (release with
        pb.release()).  Raises KKError on failure."""
        err = _err()
        _check(lib().kk_forward_batch(self.h, pb.arr, pb.n, pb.outs, err, len(err)), err)

    def prepare_ids(self, items):
        """The ids-level items marshalled once into the ABI's structs, for repeated calls (timing)."""
        return PreparedIdsBatch(items)

    def host_alloc(self, count, dtype):
        """kk_host_alloc: a pinned host array of `count` elements of `dtype` (freed with .free())."""
        return PinnedArray(self, count, dtype)

    def encode_pcm16(self, audio):
        """kk_encode_pcm16: a host f32 array as PCM_16 (encoded on the device) and its clipped count."""
        a = _f32(audio).ravel()
        out = np.zeros(a.size, np.int16)
        clipped = np.zeros(1, np.int64)
        err = _err()
        _check(lib().kk_encode_pcm16(self.h, _p(a), a.size, _p(out), _p(clipped), err, len(err)), err)
        return out, int(clipped[0])


class PreparedBatch:
    def __init__(self, items):
        self.arr, self._keep = _decoder_items(items)
        self.n = len(items)
        self.outs = (Output * self.n)()

    def audio(self, b):
        o = self.outs[b]
        return np.ctypeslib.as_array(o.audio, shape=(o.n_samples,)).copy()

    def release(self):
        lib().kk_output_free(self.outs, self.n)


class PreparedIdsBatch:
    def __init__(self, items):
        self.arr, self._keep = _items(items)
        self.n = len(items)
        self.outs = (Result * self.n)()

    def audio(self, b):
        o = self.outs[b]
        return np.ctypeslib.as_array(o.audio, shape=(o.n_samples,)).copy()

    def pred_dur(self, b):
        o = self.outs[b]
        return np.ctypeslib.as_array(o.pred_dur, shape=(o.n_tok,)).copy()

    def release(self):
        lib().kk_result_free(self.outs, self.n)


class PinnedArray:
    """Pinned host memory from kk_host_alloc, viewed as a numpy array (`.array`)."""

    def __init__(self, ctx, count, dtype):
        dt = np.dtype(dtype)
        self.ptr = C.c_void_p()
        err = _err()
        _check(lib().kk_host_alloc(ctx.h, max(1, count) * dt.itemsize, C.byref(self.ptr), err, len(err)), err)
        buf = (C.c_char * (max(1, count) * dt.itemsize)).from_address(self.ptr.value)
        self.array = np.frombuffer(buf, dt, count)

    def free(self):
        if self.ptr:
            self.array = None
            lib().kk_host_free(self.ptr)
            self.ptr = C.c_void_p()


def _decoder_items(items):
    keep = []
    arr = (DecoderItem * len(items))()
    for i, it in enumerate(items):
        dur = np.ascontiguousarray(it.dur, np.int64)
        t_en, f0, en, rs = _f32(it.t_en), _f32(it.f0), _f32(it.energy), _f32(it.ref_s)
        keep += [dur, t_en, f0, en, rs]
        d = arr[i]
        d.dur, d.n_tok, d.t_en, d.f0, d.energy, d.ref_s = dur.ctypes.data, len(dur), t_en.ctypes.data, \
            f0.ctypes.data, en.ctypes.data, rs.ctypes.data
        if it.sine is not None:
            ri, sn = _f32(it.rand_ini), _f32(it.sine)
            keep += [ri, sn]
            d.noise_kind, d.rand_ini, d.sine, d.sine_len = KK_NOISE_FIXED, ri.ctypes.data, sn.ctypes.data, sn.size
        else:
            d.noise_kind, d.seed = KK_NOISE_COUNTER, int(it.seed) & 0xFFFFFFFFFFFFFFFF
    return arr, keep


def _items(items):
    keep = []
    arr = (Item * len(items))()
    for i, it in enumerate(items):
        ids = np.ascontiguousarray(it.ids, np.int64)
        rs = _f32(it.ref_s)
        keep += [ids, rs]
        d = arr[i]
        d.ids, d.n_ids, d.ref_s, d.speed = ids.ctypes.data, len(ids), rs.ctypes.data, float(it.speed)
        if getattr(it, "sine", None) is not None:
            ri, sn = _f32(it.rand_ini), _f32(it.sine)
            keep += [ri, sn]
            d.noise_kind, d.rand_ini, d.sine, d.sine_len = KK_NOISE_FIXED, ri.ctypes.data, sn.ctypes.data, sn.size
        else:
            d.noise_kind, d.seed = KK_NOISE_COUNTER, int(it.seed) & 0xFFFFFFFFFFFFFFFF
    return arr, keep


class Plan:
    def __init__(self, ctx, h, n, kind, n_samples=None):
        self.ctx, self.h, self.n, self.kind = ctx, h, n, kind
        self.n_samples = n_samples  # audio samples per item (decoder / generator plans)

    @classmethod
    def decoder(cls, ctx, items):
        arr, keep = _decoder_items(items)
        h = C.c_void_p()
        err = _err()
        _check(lib().kk_plan_create(ctx.h, arr, len(items), C.byref(h), err, len(err)), err)
        return cls(ctx, h, len(items), "decoder", [600 * it.n_frames for it in items])

    @classmethod
    def full(cls, ctx, items):
        """Ids-level plan (kk_plan_create_full): the token phase runs at creation."""
        arr, keep = _items(items)
        h = C.c_void_p()
        err = _err()
        _check(lib().kk_plan_create_full(ctx.h, arr, len(items), C.byref(h), err, len(err)), err)
        p = cls(ctx, h, len(items), "full")
        p.durations = [p.item_durations(b) for b in range(len(items))]
        p.n_samples = [600 * int(d.sum()) for d in p.durations]
        return p

    def item_durations(self, item):
        d, n = C.POINTER(C.c_int64)(), C.c_int32()
        _check(lib().kk_plan_durations(self.h, item, C.byref(d), C.byref(n)), _err())
        return np.ctypeslib.as_array(d, shape=(n.value,)).copy()

    @classmethod
    def generator(cls, ctx, xs, f0s, ref_ss, seeds):
        """Generator-only plan: x [512, 2N], f0 [2N], ref_s [>=128], counter seeds."""
        keep = []
        arr = (GeneratorItem * len(xs))()
        for i, (x, f0, rs, sd) in enumerate(zip(xs, f0s, ref_ss, seeds)):
            x, f0 = _f32(x), _f32(f0)
            rs = _f32(np.pad(np.asarray(rs, np.float32), (0, max(0, 256 - len(rs)))))
            keep += [x, f0, rs]
            g = arr[i]
            g.x, g.n_frames, g.f0, g.ref_s = x.ctypes.data, x.shape[1] // 2, f0.ctypes.data, rs.ctypes.data
            g.noise_kind, g.seed = KK_NOISE_COUNTER, int(sd) & 0xFFFFFFFFFFFFFFFF
        h = C.c_void_p()
        err = _err()
        _check(lib().kk_plan_create_generator(ctx.h, arr, len(xs), C.byref(h), err, len(err)), err)
        return cls(ctx, h, len(xs), "generator", [600 * (_f32(x).shape[1] // 2) for x in xs])

    @classmethod
    def snake(cls, ctx, prefix, xs, ref_ss, gap=40):
        xs = [_f32(x) for x in xs]
        rss = [_f32(np.pad(np.asarray(r, np.float32), (0, max(0, 256 - len(r))))) for r in ref_ss]
        xp = (C.c_void_p * len(xs))(*[x.ctypes.data for x in xs])
        rp = (C.c_void_p * len(xs))(*[r.ctypes.data for r in rss])
        ts = (C.c_int64 * len(xs))(*[x.shape[1] for x in xs])
        h = C.c_void_p()
        err = _err()
        _check(lib().kk_plan_create_snake(ctx.h, prefix.encode(), xp, ts, rp, len(xs), gap, C.byref(h), err,
                                          len(err)), err)
        p = cls(ctx, h, len(xs), "snake")
        p.shapes = [x.shape for x in xs]
        return p

    def run(self, until="all"):
        err = _err()
        _check(lib().kk_plan_run(self.h, STAGES[until] if isinstance(until, str) else int(until), err, len(err)),
               err)

    def sync(self):
        err = _err()
        _check(lib().kk_plan_sync(self.h, err, len(err)), err)

    def fetch(self):
        outs = (Output * self.n)()
        err = _err()
        _check(lib().kk_plan_fetch(self.h, outs, err, len(err)), err)
        res = [np.ctypeslib.as_array(o.audio, shape=(o.n_samples,)).copy() for o in outs]
        lib().kk_output_free(outs, self.n)
        if self.kind == "snake":
            res = [r.reshape(s) for r, s in zip(res, self.shapes)]
        return res

    def fetch_pcm16(self):
        """Each item's audio as PCM_16 (encoded on the device) and its clipped-sample count."""
        outs = [np.zeros(n, np.int16) for n in self.n_samples]
        ptrs = (C.c_void_p * self.n)(*[o.ctypes.data for o in outs])
        clipped = np.zeros(self.n, np.int64)
        err = _err()
        _check(lib().kk_plan_fetch_pcm16(self.h, ptrs, _p(clipped), err, len(err)), err)
        return outs, clipped

    def item_samples(self, item):
        """kk_plan_item_samples: (offset, count) of item `item` in the plan's sample layout."""
        off, cnt = C.c_int64(), C.c_int64()
        _check(lib().kk_plan_item_samples(self.h, item, C.byref(off), C.byref(cnt)), _err())
        return off.value, cnt.value

    def fetch_pcm16_async(self, dst, clipped=None):
        """kk_plan_fetch_pcm16_async into PinnedArrays (int16 of 600 ln, int64 of n_items)."""
        err = _err()
        _check(lib().kk_plan_fetch_pcm16_async(self.h, dst.ptr, clipped.ptr if clipped else None, err, len(err)),
               err)

    def fetch_wait(self):
        err = _err()
        _check(lib().kk_plan_fetch_wait(self.h, err, len(err)), err)

    def tap(self, name, item, shape):
        out = np.zeros(shape, np.float32)
        err = _err()
        _check(lib().kk_plan_tap(self.h, name.encode(), item, _p(out), out.size, err, len(err)), err)
        return out

    def info(self):
        inf = PlanInfo()
        lib().kk_plan_get_info(self.h, C.byref(inf))
        return {k: getattr(inf, k) for k, _ in PlanInfo._fields_}

    def free(self):
        if getattr(self, "h", None):
            lib().kk_plan_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.free()

    def __del__(self):
        self.free()
