"""Independent torch-CPU restatement of the decoder + iSTFTNet generator, built from library routines
(F.conv1d, F.conv_transpose1d, F.instance_norm, F.interpolate, torch.stft / torch.istft), in float64.

Test infrastructure: it pins the C oracle (oracle/kk_oracle.c) from a second, structurally different
implementation that follows the upstream model definition the reference restates (StyleTTS2
AdainResBlk1d / iSTFTNet AdaINResBlock1, SineGen, TorchSTFT; docs/truth-pack/OQ_INDEX.md OQ-8,
OQ-9), so a wrong padding, dilation, weight orientation or op order in the oracle shows up here.
In float32 (set_dtype) it is also the torch-CPU functional baseline that bench.py times beside the
GPU: the op sequence upstream kokoro runs on a CPU, one item at a time.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

DT = torch.float64


def set_dtype(dt):
    """Arithmetic type of every op below (float64 to pin the oracle, float32 for the CPU baseline)."""
    global DT
    DT = dt


def T(a):
    return torch.as_tensor(np.asarray(a), dtype=DT)


def conv(w, prefix, x, stride=1, pad=0, dil=1, bias=True):
    b = T(w[prefix + ".bias"]) if bias else None
    return F.conv1d(x[None], T(w[prefix + ".weight"]), b, stride=stride, padding=pad, dilation=dil)[0]


def adain(w, prefix, x, s):
    """AdaIN1d: (1 + gamma) * InstanceNorm1d(affine)(x) + beta, gamma/beta = fc(s)."""
    c = x.shape[0]
    h = F.linear(T(s[:128]), T(w[prefix + ".fc.weight"]), T(w[prefix + ".fc.bias"]))
    n = F.instance_norm(x[None], weight=T(w[prefix + ".norm.weight"]), bias=T(w[prefix + ".norm.bias"]), eps=1e-5)[0]
    return (1 + h[:c, None]) * n + h[c:, None]


def resblk(w, p, x, s, upsample=False):
    """StyleTTS2 AdainResBlk1d: (residual + shortcut) / sqrt(2)."""
    din = x.shape[0]
    r = F.leaky_relu(adain(w, p + ".norm1", x, s), 0.2)
    if upsample:
        r = F.conv_transpose1d(r[None], T(w[p + ".pool.weight"]), T(w[p + ".pool.bias"]), stride=2, padding=1,
                               output_padding=1, groups=din)[0]
    r = conv(w, p + ".conv1", r, pad=1)
    r = F.leaky_relu(adain(w, p + ".norm2", r, s), 0.2)
    r = conv(w, p + ".conv2", r, pad=1)
    sc = x
    if upsample:
        sc = F.interpolate(sc[None], scale_factor=2, mode="nearest")[0]
    if p + ".conv1x1.weight" in w:
        sc = conv(w, p + ".conv1x1", sc, bias=False)
    return (r + sc) / math.sqrt(2)


def snake_block(w, p, x, s):
    """iSTFTNet AdaINResBlock1 with Snake activations, dilations 1, 3, 5."""
    k = w[p + ".convs1.0.weight"].shape[2]
    for i, d in enumerate((1, 3, 5)):
        a1 = T(w[f"{p}.alpha1.{i}"]).reshape(-1, 1)
        a2 = T(w[f"{p}.alpha2.{i}"]).reshape(-1, 1)
        xt = adain(w, f"{p}.adain1.{i}", x, s)
        xt = xt + (1 / a1) * torch.sin(a1 * xt) ** 2
        xt = conv(w, f"{p}.convs1.{i}", xt, pad=(k * d - d) // 2, dil=d)
        xt = adain(w, f"{p}.adain2.{i}", xt, s)
        xt = xt + (1 / a2) * torch.sin(a2 * xt) ** 2
        xt = conv(w, f"{p}.convs2.{i}", xt, pad=(k - 1) // 2)
        x = xt + x
    return x


def decoder(w, asr, f0, en, s):
    asr, f0, en = T(asr), T(f0), T(en)
    f0n = conv(w, "decoder.F0_conv", f0[None], stride=2, pad=1)
    nn_ = conv(w, "decoder.N_conv", en[None], stride=2, pad=1)
    x = resblk(w, "decoder.encode", torch.cat([asr, f0n, nn_]), s)
    ar = conv(w, "decoder.asr_res.0", asr)
    for i in range(4):
        x = resblk(w, f"decoder.decode.{i}", torch.cat([x, ar, f0n, nn_]), s, upsample=i == 3)
    return x


def sine_source(w, f0c, rand_ini, noise):
    """SineGen._f02sine + SourceModuleHnNSF with the reference's fixed noise (9 harmonics, sr 24 kHz,
    upsample 300, sine_amp 0.1, noise_std 0.003, voiced threshold 10)."""
    f0c = T(f0c)
    l = f0c.shape[0]
    s = 300 * l
    f0_up = F.interpolate(f0c[None, None], scale_factor=300, mode="nearest")[0, 0]  # [S]
    harm = torch.arange(1, 10, dtype=DT)
    rad = torch.remainder(f0_up[:, None] * harm[None, :] / 24000.0, 1.0)  # [S, 9]
    ri = T(rand_ini).clone()
    ri[0] = 0
    rad[0, :] = rad[0, :] + ri
    rad_d = F.interpolate(rad.T[None], scale_factor=1 / 300, mode="linear", align_corners=False)[0].T  # [L, 9]
    phase = torch.cumsum(rad_d, dim=0) * 2 * math.pi
    phase = F.interpolate(phase.T[None] * 300, scale_factor=300, mode="linear", align_corners=False)[0].T  # [S, 9]
    sines = torch.sin(phase) * 0.1
    uv = (f0_up > 10).to(DT)[:, None]
    noise_amp = uv * 0.003 + (1 - uv) * 0.1 / 3
    sw = sines * uv + noise_amp * T(noise).reshape(s, 9)
    lw = T(w["decoder.generator.m_source.l_linear.weight"]).reshape(9)
    lb = T(w["decoder.generator.m_source.l_linear.bias"]).reshape(())
    return torch.tanh(sw @ lw + lb)


def stft(x):
    """TorchSTFT.transform: n_fft 20, hop 5, periodic Hann, center, reflect -> (magnitude, phase)."""
    win = torch.hann_window(20, periodic=True, dtype=DT)
    X = torch.stft(T(x), n_fft=20, hop_length=5, win_length=20, window=win, center=True, pad_mode="reflect",
                   return_complex=True)
    return X.abs(), torch.angle(X)


def istft(post):
    """exp(magnitude), sin(phase), then torch.istft (TorchSTFT.inverse)."""
    post = T(post)
    mag = torch.exp(post[:11])
    ph = torch.sin(post[11:])
    win = torch.hann_window(20, periodic=True, dtype=DT)
    return torch.istft(mag * torch.exp(1j * ph), n_fft=20, hop_length=5, win_length=20, window=win, center=True)


def generator(w, x, f0, s, rand_ini, noise, taps=None, spec=None):
    """Generator forward; `spec` overrides the source + STFT output (to pin the glue separately
    from the ill-conditioned phases of near-zero STFT bins)."""
    g = "decoder.generator"
    x = T(x)
    if spec is None:
        har = sine_source(w, f0, rand_ini, noise)
        mag, ph = stft(har)
        spec = torch.cat([mag, ph])  # [22, 120N + 1]
    else:
        spec = T(spec)
    if taps is not None:
        taps["spec"] = spec
    for i in range(2):
        x = F.leaky_relu(x, 0.1)
        if i == 0:
            xs = conv(w, f"{g}.noise_convs.0", spec, stride=6, pad=3)
        else:
            xs = conv(w, f"{g}.noise_convs.1", spec)
        xs = snake_block(w, f"{g}.noise_res.{i}", xs, s)
        stride, pad = (10, 5) if i == 0 else (6, 3)
        x = F.conv_transpose1d(x[None], T(w[f"{g}.ups.{i}.weight"]), T(w[f"{g}.ups.{i}.bias"]), stride=stride,
                               padding=pad)[0]
        if i == 1:
            x = F.pad(x[None], (1, 0), mode="reflect")[0]
        x = x + xs
        acc = None
        for j in range(3):
            r = snake_block(w, f"{g}.resblocks.{3 * i + j}", x, s)
            acc = r if acc is None else acc + r
        x = acc / 3
        if taps is not None:
            taps[f"gen{i}"] = x
    x = F.leaky_relu(x, 0.01)
    post = conv(w, f"{g}.conv_post", x, pad=3)
    if taps is not None:
        taps["post"] = post
    return istft(post)
