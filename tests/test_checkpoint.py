"""Real-weight hydration (src/torchpt.rs, src/weights.rs:62-84, src/ops.rs:9-23, src/engine.rs:54-59,
114-137) through the C ABI: the library's torch.save reader, weight_norm, the AdaIN affine
defaults and the voice packs.

The released kokoro-v1_0.pth and voices/*.pt are not available offline, so the archives here are
written by torch.save in the layout the released files have (a dict of per-submodule state dicts with
"module." prefixes, weight_g / weight_v pairs, the AdaIN InstanceNorm affine parameters absent; voice
packs [510, 1, 256]); what torch.load(weights_only=True) reads back from the same file is the truth
the reader is held to, bit for bit.
"""
import collections
import zipfile

import numpy as np
import pytest
import torch

from oracle import oracle as O


def _read(path):
    from kokoro_hip import api
    ck = api.Checkpoint(path)
    try:
        return ck.tensors()
    finally:
        ck.free()


def test_reads_what_torch_saves(tmp_path):
    g = torch.Generator().manual_seed(7)
    base = torch.randn(6, 10, generator=g)
    sd = collections.OrderedDict()
    sd["module.conv.weight_g"] = torch.rand(4, 1, 1, generator=g)
    sd["module.conv.weight_v"] = torch.randn(4, 3, 5, generator=g)
    sd["module.lin.weight"] = torch.randn(6, 4, generator=g).t()      # a transposed view
    sd["module.slice"] = base[2:5, 1:8]                                # offset and strides
    sd["module.shared"] = base[1]                                      # another view of one storage
    sd["module.scalar"] = torch.tensor(3.5)
    sd["module.empty"] = torch.zeros(0, 3)
    sd["plain.bias"] = torch.randn(300, generator=g)                   # no "module." prefix
    top = {"decoder": sd, "bert": collections.OrderedDict(x=torch.arange(5, dtype=torch.float32))}
    path = tmp_path / "m.pth"
    torch.save(top, path)
    ref = torch.load(path, weights_only=True)
    got = _read(path)
    want = {}
    for sub, d in ref.items():
        for k, t in d.items():
            want[f"{sub}.{k[7:] if k.startswith('module.') else k}"] = t.numpy()
    assert sorted(got) == sorted(want)
    for k, t in want.items():
        assert got[k].shape == t.shape and got[k].dtype == np.float32, k
        assert np.array_equal(got[k].reshape(-1).view(np.uint32), np.array(t).reshape(-1).view(np.uint32)), k


def _expect_refusal(path, words):
    from kokoro_hip import api
    with pytest.raises(api.KKError) as e:
        api.Checkpoint(path)
    assert e.value.code == -1 and any(w in str(e.value) for w in words), str(e.value)


def test_refuses_what_it_does_not_read(tmp_path):
    # float64 storage: another storage global
    p = tmp_path / "f64.pth"
    torch.save({"decoder": {"w": torch.zeros(3, dtype=torch.float64)}}, p)
    _expect_refusal(p, ["DoubleStorage"])
    # a Python list of ints: opcodes outside the set torch.save uses for tensors
    p = tmp_path / "list.pth"
    torch.save({"decoder": {"w": [1, 2, 3]}}, p)
    _expect_refusal(p, ["opcode", "REDUCE", "global", "SETITEM", "tensor", "expected"])
    # the same archive recompressed with DEFLATE
    good = tmp_path / "good.pth"
    torch.save({"decoder": {"w": torch.ones(8)}}, good)
    bad = tmp_path / "deflate.pth"
    with zipfile.ZipFile(good) as zi, zipfile.ZipFile(bad, "w", zipfile.ZIP_DEFLATED) as zo:
        for n in zi.namelist():
            zo.writestr(n, zi.read(n))
    _expect_refusal(bad, ["compressed"])
    # truncated, and not an archive at all
    t = tmp_path / "trunc.pth"
    t.write_bytes(good.read_bytes()[: len(good.read_bytes()) // 2])
    _expect_refusal(t, ["zip", "truncated", "end-of-central"])
    n = tmp_path / "text.pth"
    n.write_bytes(b"not a zip archive at all, just some text" * 4)
    _expect_refusal(n, ["zip"])
    _expect_refusal(tmp_path / "missing.pth", ["cannot open"])


def _patched_view(tmp_path, name, size_bytes, stride_bytes):
    """A torch.save archive of one [8] tensor whose pickled size and stride tuples are replaced."""
    good = tmp_path / "good8.pth"
    torch.save({"decoder": {"w": torch.ones(8)}}, good)
    out = tmp_path / name
    with zipfile.ZipFile(good) as zi, zipfile.ZipFile(out, "w", zipfile.ZIP_STORED) as zo:
        for n in zi.namelist():
            data = zi.read(n)
            if n.endswith("/data.pkl"):
                # size (8,) and stride (1,): BININT1 + TUPLE1, each followed by a BINPUT of its memo slot
                i = data.index(b"K\x08\x85q")
                j = data.index(b"K\x01\x85q", i)
                assert j == i + 5
                data = data[:i] + size_bytes + data[i + 2:j] + stride_bytes + data[j + 2:]
            zo.writestr(n, data)
    return out


def test_refuses_views_past_their_storage(tmp_path):
    """A crafted size / stride must not reach past the 32-byte storage, including extents that wrap
    int64 (the reader computes them overflow-checked, as the reference bounds every element)."""
    def long1(v):
        return b"\x8a\x08" + int(v).to_bytes(8, "little", signed=True)

    # size 2^62 with stride 2^62: (size - 1) * stride wraps int64
    _expect_refusal(_patched_view(tmp_path, "wrap.pth", long1(1 << 62), long1(1 << 62)), ["overflow"])
    # size 2^40, stride 0 (an expanded view): in bounds, but beyond any tensor of the model
    _expect_refusal(_patched_view(tmp_path, "huge.pth", long1(1 << 40), b"K\x00"), ["2^28"])
    # negative size or stride (refused by the unpickler as non-indices already)
    _expect_refusal(_patched_view(tmp_path, "negsize.pth", long1(-8), b"K\x01"), ["negative", "non-index"])
    _expect_refusal(_patched_view(tmp_path, "negstride.pth", b"K\x08", long1(-1)), ["negative", "non-index"])
    # a plain overrun: 9 elements of an 8-element storage
    _expect_refusal(_patched_view(tmp_path, "over.pth", b"K\x09", b"K\x01"), ["past storage"])
    # the unpatched archive reads back
    assert np.array_equal(_read(_patched_view(tmp_path, "same.pth", b"K\x08", b"K\x01"))["decoder.w"], np.ones(8))


def test_weight_norm():
    """The library's weight_norm equals the oracle's restatement of src/ops.rs:9-23 bit for bit, and
    torch._weight_norm within f32 rounding; a row (3, 4) has norm 5 exactly."""
    from kokoro_hip import api
    rng = np.random.default_rng(11)
    for shape in [(4, 3, 5), (256, 1, 3), (512, 256, 20), (7, 1, 1)]:
        v = rng.standard_normal(shape).astype(np.float32)
        gv = rng.uniform(0.1, 2.0, (shape[0], 1, 1)).astype(np.float32)
        w = api.weight_norm(v, gv)
        assert np.array_equal(w, O.weight_norm(v, gv))
        ref = torch._weight_norm(torch.from_numpy(v), torch.from_numpy(gv), 0).numpy()
        assert np.allclose(w, ref, rtol=3e-6, atol=1e-7)
    w = api.weight_norm(np.array([[3.0, 4.0]], np.float32), np.array([2.0], np.float32))
    assert np.array_equal(w, np.array([[1.2, 1.6]], np.float32))


def test_voice_packs(tmp_path):
    """load_voice_pack, the mean of several packs (summed in order in f32) and ref_s = row n - 1."""
    from kokoro_hip import api
    g = torch.Generator().manual_seed(3)
    packs = [torch.randn(510, 1, 256, generator=g) for _ in range(3)]
    paths = []
    for i, p in enumerate(packs):
        paths.append(tmp_path / f"v{i}.pt")
        torch.save(p, paths[-1])
    one = api.voice_load([paths[0]])
    assert one.shape == (510, 256) and np.array_equal(one, packs[0].numpy().reshape(510, 256))
    mean = api.voice_load(paths)
    a = [p.numpy().reshape(510, 256) for p in packs]
    want = ((a[0] + a[1]) + a[2]) / np.float32(3)
    assert np.array_equal(mean, want)
    assert np.array_equal(api.voice_ref_s(one, 1), one[0])
    assert np.array_equal(api.voice_ref_s(one, 510), one[509])
    for n in (0, 511):
        with pytest.raises(api.KKError):
            api.voice_ref_s(one, n)
    bad = tmp_path / "bad.pt"
    torch.save(torch.zeros(510, 2, 256), bad)
    with pytest.raises(api.KKError) as e:
        api.voice_load([bad])
    assert "voice pack" in str(e.value)
    with pytest.raises(api.KKError):
        api.voice_load([paths[0], bad])


def kokoro_like_checkpoint(weights, path, seed=5):
    """A random-init model written the way the released model file holds it: per-submodule state
    dicts ("bert", "bert_encoder", "predictor", "text_encoder", "decoder") whose keys carry a
    "module." prefix; every conv weight except the noise convs and the F0 / N projections as a
    weight_g / weight_v pair (v a rescaled copy of the weight, g within 25% of its row norms: the
    resolved weight is weight_norm(v, g), not the original); the AdaIN InstanceNorm affine
    parameters left out.  Returns the table the checkpoint resolves to, built with the oracle's
    weight_norm and the defaults 1 / 0."""
    rng = np.random.default_rng(seed)
    subs = collections.OrderedDict()
    resolved = {}
    for name, arr in weights.items():
        sub, key = name.split(".", 1)
        dec = subs.setdefault(sub, collections.OrderedDict())
        if name.endswith(".norm.weight") or name.endswith(".norm.bias"):
            if ".adain" in name or ".norm1." in name or ".norm2." in name:
                resolved[name] = np.ones_like(arr) if name.endswith("weight") else np.zeros_like(arr)
                continue
        if (name.endswith(".weight") and arr.ndim == 3 and "noise_convs" not in name and "_proj" not in name):
            v = (arr * rng.uniform(0.5, 2.0, (arr.shape[0],) + (1,) * (arr.ndim - 1))).astype(np.float32)
            # g near the original row norms, so that activations keep their scale
            norms = np.sqrt((arr.astype(np.float64) ** 2).reshape(arr.shape[0], -1).sum(1)).reshape(-1, 1, 1)
            gv = (norms * rng.uniform(0.8, 1.25, norms.shape)).astype(np.float32)
            dec["module." + key[: -len("weight")] + "weight_g"] = torch.from_numpy(gv)
            dec["module." + key[: -len("weight")] + "weight_v"] = torch.from_numpy(v)
            resolved[name] = O.weight_norm(v, gv)
            continue
        dec["module." + key] = torch.from_numpy(np.ascontiguousarray(arr, np.float32))
        resolved[name] = arr
    subs.setdefault("bert", collections.OrderedDict(dummy=torch.zeros(4)))
    torch.save(dict(subs), path)
    return resolved


@pytest.mark.gpu
def test_upload_checkpoint_matches_resolved_table(weights, tmp_path):
    """kk_upload_checkpoint (weight_norm resolved and the affine defaults applied in the library)
    gives the same audio, bit for bit, as kk_upload_model of the table resolved on the CPU."""
    from kokoro_hip import api, workloads
    path = tmp_path / "kokoro-like.pth"
    resolved = kokoro_like_checkpoint(weights, path)
    items = workloads.small_items(83, [9, 4, 15])
    a = api.Context(0)
    b = api.Context(0)
    try:
        ck = api.Checkpoint(path)
        a.upload_checkpoint(ck)
        ck.free()
        b.upload_model(resolved)
        out_a, out_b = a.forward_decoder_batch(items), b.forward_decoder_batch(items)
    finally:
        a.close()
        b.close()
    for x, y in zip(out_a, out_b):
        assert np.isfinite(x).all() and np.array_equal(x, y)


@pytest.mark.gpu
def test_upload_checkpoint_whole_model(tmp_path):
    """The whole model from a checkpoint (ALBERT, the text encoder and the predictor included, their
    weight-normed convs resolved in the library) gives the same durations and audio, bit for bit,
    through kk_forward_batch as kk_upload_model of the table resolved on the CPU."""
    from kokoro_hip import api, model_spec, workloads
    w = model_spec.random_model_weights(seed=0)
    path = tmp_path / "kokoro-like-full.pth"
    resolved = kokoro_like_checkpoint(w, path, seed=6)
    items = workloads.small_ids_items(84, [21, 9, 40])
    a = api.Context(0)
    b = api.Context(0)
    try:
        ck = api.Checkpoint(path)
        a.upload_checkpoint(ck)
        ck.free()
        b.upload_model(resolved)
        out_a, out_b = a.forward_batch(items), b.forward_batch(items)
    finally:
        a.close()
        b.close()
    for (x, dx), (y, dy) in zip(out_a, out_b):
        assert np.array_equal(dx, dy) and np.isfinite(x).all() and np.array_equal(x, y)
