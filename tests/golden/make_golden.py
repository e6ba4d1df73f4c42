"""Write tests/golden/golden_v1.npz: small input/output vectors from the float64 torch restatement
(oracle/torch_ref.py, library routines only) that pin the CPU oracle independently of the torch
version installed later.  Weights are model_spec.random_weights(seed=0); their sha256 is stored.

Run: python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "kokoro-rust_amd"))
from oracle import torch_ref as R  # noqa: E402
from kokoro_hip import model_spec, workloads  # noqa: E402


def weights_sha(w, names):
    h = hashlib.sha256()
    for n in sorted(names):
        h.update(n.encode())
        h.update(np.ascontiguousarray(w[n], np.float32).tobytes())
    return h.hexdigest()


def main():
    torch.set_num_threads(4)
    w = model_spec.random_weights(seed=0)
    rng = np.random.default_rng(2024)
    out = {}
    # conv1d, dilated (k 11, d 5) and strided (k 12, s 6)
    x = rng.standard_normal((6, 90)).astype(np.float32)
    cw = rng.standard_normal((5, 6, 11)).astype(np.float32)
    cb = rng.standard_normal(5).astype(np.float32)
    out.update(conv_x=x, conv_w=cw, conv_b=cb,
               conv_y=torch.nn.functional.conv1d(R.T(x)[None], R.T(cw), R.T(cb), padding=25, dilation=5)[0].numpy())
    # ConvTranspose1d k 20 s 10 p 5
    tx = rng.standard_normal((4, 13)).astype(np.float32)
    tw = rng.standard_normal((4, 3, 20)).astype(np.float32)
    tb = rng.standard_normal(3).astype(np.float32)
    out.update(convt_x=tx, convt_w=tw, convt_b=tb,
               convt_y=torch.nn.functional.conv_transpose1d(R.T(tx)[None], R.T(tw), R.T(tb), stride=10,
                                                            padding=5)[0].numpy())
    # STFT / iSTFT
    sx = np.tanh(rng.standard_normal(600)).astype(np.float32)
    mag, ph = R.stft(sx)
    out.update(stft_x=sx, stft_mag=mag.numpy(), stft_phase=ph.numpy())
    post = (rng.standard_normal((22, 61)) * 0.5).astype(np.float32)
    out.update(istft_post=post, istft_y=R.istft(post).numpy())
    # harmonic source with fixed noise
    f0 = workloads.smooth_curve(rng, 10, 100, 300)
    f0[4:6] = 0.0
    ri = rng.uniform(0, 1, 9).astype(np.float32)
    nz = rng.standard_normal(300 * 10 * 9).astype(np.float32)
    out.update(src_f0=f0, src_rand_ini=ri, src_noise=nz, src_har=R.sine_source(w, f0, ri, nz).numpy())
    # one Snake block (256 ch, k 3) and one decoder block
    bx = rng.standard_normal((256, 40)).astype(np.float32)
    bs = rng.standard_normal(256).astype(np.float32)
    out.update(snake_x=bx, snake_style=bs,
               snake_y=R.snake_block(w, "decoder.generator.resblocks.0", R.T(bx), bs).numpy())
    ex = rng.standard_normal((514, 6)).astype(np.float32)
    out.update(encode_x=ex, encode_y=R.resblk(w, "decoder.encode", R.T(ex), bs).numpy())
    # generator glue from a given spectrum, N = 2
    gx = rng.standard_normal((512, 4)).astype(np.float32)
    gspec = np.concatenate([np.abs(rng.standard_normal((11, 241))), rng.uniform(-3, 3, (11, 241))]).astype(np.float32)
    gf0 = workloads.smooth_curve(rng, 4, 100, 300)
    taps = {}
    gy = R.generator(w, gx, gf0, bs, ri, np.zeros(600 * 2 * 9, np.float32), taps, spec=gspec).numpy()
    out.update(gen_x=gx, gen_spec=gspec, gen_f0=gf0, gen_style=bs, gen_post=taps["post"].numpy(), gen_audio=gy)
    names = [n for n in w if n.startswith("decoder.")]
    meta = np.array([f"torch {torch.__version__}; weights model_spec.random_weights(seed=0) sha256 "
                     f"{weights_sha(w, names)}"])
    np.savez_compressed(os.path.join(HERE, "golden_v1.npz"), meta=meta, **out)
    print("wrote", os.path.join(HERE, "golden_v1.npz"), meta[0])


if __name__ == "__main__":
    main()
