"""kk_snake_block_noalloc, the entry point that allocates nothing (for callers that cannot call
hipMalloc), against the existing Snake-block entry (kk_plan_create_snake + kk_plan_run) on the same
inputs: bit-identical, on calls in a row over one device's shared scratch, the second smaller than
the first.  The caller's device buffer x is allocated here, by the test, through the HIP runtime the
library itself is bound to (torch's own initialization fails in a process where the library's
runtime came up first)."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class DeviceArray:
    """A device buffer from the library's own HIP runtime (test plumbing)."""
    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            # by soname: the copy already loaded for the library (a process that imported torch
            # first holds torch's build of this soname, and the library is bound to it)
            h = C.CDLL("libamdhip64.so.7")
            h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
            h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
            h.hipFree.argtypes = [C.c_void_p]
            h.hipDeviceSynchronize.argtypes = []
            cls._hip = h
        return cls._hip

    def __init__(self, host):
        self.host = np.ascontiguousarray(host)
        self.ptr = C.c_void_p()
        assert self.hip().hipMalloc(C.byref(self.ptr), self.host.nbytes) == 0
        assert self.hip().hipMemcpy(self.ptr, self.host.ctypes.data, self.host.nbytes, 1) == 0  # H2D

    def get(self):
        out = np.empty_like(self.host)
        assert self.hip().hipDeviceSynchronize() == 0
        assert self.hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, 2) == 0  # D2H
        return out

    def free(self):
        if self.ptr:
            self.hip().hipFree(self.ptr)
            self.ptr = C.c_void_p()


def _packed(xs, gap):
    starts, lens, r = [], [], 0
    for x in xs:
        starts.append(r)
        lens.append(x.shape[1])
        r += x.shape[1] + gap
    return starts, lens, r


def _noalloc(ctx, prefix, xs, styles, gap):
    c = xs[0].shape[0]
    starts, lens, rows = _packed(xs, gap)
    host = np.zeros((rows, c), np.float32)
    for s, x in zip(starts, xs):
        host[s:s + x.shape[1]] = x.T
    dev = DeviceArray(host)
    try:
        ctx.snake_block_noalloc(prefix, dev.ptr.value, rows, starts, lens, styles)
        out = dev.get()
    finally:
        dev.free()
    return [np.ascontiguousarray(out[s:s + x.shape[1]].T) for s, x in zip(starts, xs)]


@pytest.mark.parametrize("prefix,c", [("decoder.generator.resblocks.1", 256), ("decoder.generator.resblocks.5", 128)])
def test_noalloc_matches_snake_plan(gpu_ctx, prefix, c):
    from kokoro_hip import api
    rng = np.random.default_rng(95 + c)
    for call, ts in enumerate([[700, 1500, 300, 1200], [90, 400]]):  # the second call smaller
        xs = [rng.standard_normal((c, t)).astype(np.float32) for t in ts]
        styles = [rng.standard_normal(128).astype(np.float32) for _ in ts]
        with api.Plan.snake(gpu_ctx, prefix, xs, styles, gap=40) as plan:
            plan.run()
            ref = plan.fetch()
        got = _noalloc(gpu_ctx, prefix, xs, styles, gap=40)
        for b, (r, g) in enumerate(zip(ref, got)):
            assert np.isfinite(g).all() and np.array_equal(r, g), f"call {call} item {b}"
        print(f"  {prefix} call {call}: {len(ts)} items, {sum(ts)} columns, bit-identical", flush=True)


def test_noalloc_refuses_beyond_its_limits(gpu_ctx):
    """Refused on the host before any device work (the buffer is sized for the claimed rows all the
    same, so that nothing could reach past it)."""
    from kokoro_hip import api
    prefix = "decoder.generator.resblocks.1"
    styles = [np.zeros(128, np.float32)]
    rows = api.NOALLOC_MAX_ROWS + 1
    big = DeviceArray(np.zeros((rows, 256), np.float32))
    try:
        with pytest.raises(api.KKError) as e:
            gpu_ctx.snake_block_noalloc(prefix, big.ptr.value, rows, [0], [10], styles)
        assert e.value.code == -1 and "rows" in str(e.value)
        n = api.NOALLOC_MAX_ITEMS + 1
        with pytest.raises(api.KKError) as e:
            gpu_ctx.snake_block_noalloc(prefix, big.ptr.value, 4 * n, list(range(0, 4 * n, 4)), [2] * n, styles * n)
        assert e.value.code == -1 and "items" in str(e.value)
        assert not big.get().any()  # untouched
    finally:
        big.free()
