"""Which operand roundings of the stages before the decoder move ids-level audio off float64 (a CPU
measurement, not a test: `python tests/studies/prosody_precision.py` from the repository root,
about 6 minutes).

For three items of the ids-level test batch, the torch oracle (oracle/torch_ref.py) runs the stages
before the decoder in float64 with the predicted durations held fixed, once as is and once per
variant: bf16 operand rounding at every layer the GPU rounds, at all but one group of layers, at
one group only, fp16 instead of bf16, and float32 arithmetic without any rounding.  Each variant's
t_en, F0 and N go through the same fp32 C oracle decoder + generator (oracle/kk_oracle.c), so only
the upstream differs.  Printed per item: F0's SNR (its variation around the projection bias) and
the audio's SNR against the float64 run.  Groups: ALBERT, bert_encoder, the duration encoder's
BiLSTMs, the duration LSTM + projection (durations fixed: no effect), the shared LSTM's input
projection, the F0 / N stacks' convolutions, the text encoder."""
import os
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "kokoro-rust_amd"))
sys.path.insert(0, ROOT)
from kokoro_hip import model_spec, workloads  # noqa: E402
from oracle import oracle as O  # noqa: E402
from oracle import torch_ref as R  # noqa: E402

w = model_spec.random_model_weights(seed=0)
om = O.Model(w)
items = workloads.small_ids_items(41, [30, 75, 12])
b_f0 = float(w["predictor.F0_proj.bias"][0])

def snr(ref, x):
    ref = np.asarray(ref, np.float64); x = np.asarray(x, np.float64)
    return 10 * np.log10((ref ** 2).sum() / max(((x - ref) ** 2).sum(), 1e-300))

G = {
    "albert": ("bert.",),
    "bert_encoder": ("bert_encoder",),
    "dur_encoder": ("predictor.text_encoder.",),
    "dur_lstm_proj": ("predictor.lstm", "predictor.duration_proj"),
    "shared_lstm": ("predictor.shared",),
    "f0n_convs": ("predictor.F0.", "predictor.N."),
    "text_encoder": ("text_encoder.",),
}

def run(it, dur, ctx=None, dtype=torch.float64):
    R.set_dtype(dtype)
    try:
        if ctx is None:
            _, t_en, f0, n = R.upstream(w, it.ids, it.ref_s, dur=dur)
        else:
            with ctx:
                _, t_en, f0, n = R.upstream(w, it.ids, it.ref_s, dur=dur)
    finally:
        R.set_dtype(torch.float64)
    dec = workloads.DecoderItem(dur=dur, t_en=t_en.numpy().astype(np.float32), f0=f0.numpy().astype(np.float32),
                                energy=n.numpy().astype(np.float32), ref_s=it.ref_s, seed=it.seed)
    return f0.numpy().astype(np.float64), O.synth_item(om, dec)

rows = {}
t0 = time.time()
for b, it in enumerate(items):
    dur, _, _, _ = R.upstream(w, it.ids, it.ref_s)
    f_ref, a_ref = run(it, dur)
    variants = {"bf16 everywhere (the GPU's points)": R.bf16_operands(), "float32, no rounding": None}
    for g, pre in G.items():
        variants[f"all but {g}"] = R.bf16_operands(skip=pre)
    for g, pre in G.items():
        variants[f"only {g}"] = R.bf16_operands(only=pre)
    variants["fp16 in f0n_convs, bf16 elsewhere"] = R.bf16_operands(fp16=G["f0n_convs"])
    variants["fp16 in shared_lstm + f0n_convs"] = R.bf16_operands(fp16=G["f0n_convs"] + G["shared_lstm"])
    variants["fp16 everywhere"] = R.bf16_operands(fp16=("",))
    for name, ctx in variants.items():
        if name.startswith("float32"):
            f, a = run(it, dur, None, torch.float32)
        else:
            f, a = run(it, dur, ctx)
        rows.setdefault(name, []).append((snr(f_ref - b_f0, f - b_f0), snr(a_ref, a)))
    print(f"item {b} done ({len(it.ids)} ids, {int(dur.sum())} frames) {time.time() - t0:.0f} s", flush=True)
print(f"{'variant':42s} " + "  ".join(f"item{b}: F0 dB / audio dB" for b in range(len(items))))
for name, r in rows.items():
    print(f"{name:42s} " + "  ".join(f"{f:6.1f} / {a:5.1f}            " for f, a in r))
