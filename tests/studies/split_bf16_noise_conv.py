"""Accuracy of noise_convs.0's split-bf16 products (a CPU measurement, not a test:
`python tests/studies/split_bf16_noise_conv.py` from the repository root, a few seconds).

The kernel splits every input value and weight into its bf16 rounding (to nearest even) and the
bf16 rounding of the remainder, and accumulates each product as wh*xh + wh*xl + wl*xh.  This script
applies the same splits to spectrum-like inputs (11 magnitudes spread over seven octaves and 11
phases in [-pi, pi], stride-6 windows of 12 rows, 256 output channels with N(0, 0.1) weights) and
prints the error against float64 sums: relative to sum |w x| (the scale a dot product's rounding
is measured on) and rms relative; beside it an f32 matrix product's error and the rms of the fp16
rounding the kernel applies when it stores its output, and the share of stored fp16 values that
the split moves."""
import numpy as np


def bf16(x):
    """Round float32 values to bf16 (nearest, ties to even), returned as float32."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def main():
    rng = np.random.default_rng(0)
    n = 4000
    mag = np.abs(rng.standard_normal((n, 11))) * np.exp(rng.uniform(-6, 1, (n, 11)))
    ph = rng.uniform(-np.pi, np.pi, (n, 11))
    x = np.concatenate([mag, ph], 1).astype(np.float32)  # [rows][22]
    w = (rng.standard_normal((256, 22, 12)) * 0.1).astype(np.float32)
    cols = (n - 12) // 6
    X = np.stack([x[6 * j:6 * j + 12].T.reshape(-1) for j in range(cols)], 1)  # [22 * 12][cols]
    W = w.reshape(256, -1)
    exact = W.astype(np.float64) @ X.astype(np.float64)
    xh = bf16(X)
    xl = bf16(X - xh)
    wh = bf16(W)
    wl = bf16(W - wh)
    f64 = lambda a: a.astype(np.float64)
    split = f64(wh) @ f64(xh) + f64(wh) @ f64(xl) + f64(wl) @ f64(xh)
    f32 = f64(W @ X)
    scale = np.abs(f64(W)) @ np.abs(f64(X))
    rms = lambda e: float(np.sqrt((e ** 2).mean() / (exact ** 2).mean()))
    print("split bf16: max |err| / sum|w x| %.2e, rms relative %.2e"
          % ((np.abs(split - exact) / scale).max(), rms(split - exact)))
    print("f32 product: max |err| / sum|w x| %.2e" % (np.abs(f32 - exact) / scale).max())
    print("fp16 store: rms relative %.2e" % rms(f64(exact.astype(np.float16)) - exact))
    print("stored fp16 values moved by the split: %.4f"
          % (exact.astype(np.float16) != split.astype(np.float16)).mean())


if __name__ == "__main__":
    main()
