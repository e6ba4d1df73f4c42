"""Benchmark: batched ragged Kokoro-82M decoder + iSTFTNet generator on one MI355X.

Workload (the metric's config): 32 ragged items, N ~ U[100, 800] decoder
frames each, seeded synthetic inputs and random-init weights of the real architecture.

- `value` (the benchmark protocol: the whole call, host to host): one step = one C-ABI call of
  kk_forward_decoder_batch, from host inputs to host audio (layout, upload, duration expansion ->
  decoder -> harmonic source + STFT -> generator -> iSTFT -> audio copied back).  W warm calls, then
  K timed calls, each timed on its own; `value` = audio seconds / the median call.
- `kernel_only`: the same batch as a plan whose inputs are resident in HBM, K runs of kk_plan_run
  timed together (device time per step, no host transfers).
- `roofline`: the dominant kernel, the Snake-block MFMA convolutions.  A profiling pass of the same
  K steps runs every kernel alone on the library's stream with a HIP event pair around each launch;
  achieved = algorithmic FLOP per launch / average launch time, against the bf16 dense MFMA peak.
  `traffic` is the HBM bytes per launch from the FETCH_SIZE / WRITE_SIZE counters
  (profiles/conv_mfma_snake_config3_traffic.json, made with --calibrate-copy-mib and
  kokoro_hip/profsum.py).
- `hbm`: every bandwidth kernel of the same pass: algorithmic bytes (valid rows read and written
  once) per launch / its time, against 8 TB/s.
- `parity`: item 0 of the timed calls' audio against the fp32 CPU oracle.
- `cpu_baseline`: the oracle (a C restatement of the same path, OpenMP) on a bounded sample of the
  same batch, and on config 1; beside it the torch-CPU functional restatement (oracle/torch_ref.py,
  float32) on the same sample.  A reported baseline, not the target.
- `e2e`: BASELINE.json configs[3], the whole forward from phoneme ids (kk_forward_batch) on its own
  batch (64 ragged items, 20-510 ids), with its device-resident time, a serial per-class kernel
  breakdown and its own torch-CPU baseline (see e2e_leg).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-e2e | --only-e2e] [--config 3|5]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kokoro-rust_amd"))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
PEAK_F32_MFMA_TFLOPS = 157.3  # dense f32 matrix-core peak (the attention runs on v_mfma_f32_32x32x2f32)
BANDWIDTH_KERNELS = ["stats_tiles", "finalize", "style_fc", "expand", "f0n_conv", "copy_cols", "adain_pool",
                     "noise_conv0", "noise_conv1", "phase_pre", "source_stft", "istft"]


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(weights, items, budget_s=12.0, torch_budget_s=8.0):
    """The oracle (fp32 C restatement of the path) on the first items of the batch until `budget_s` of
    wall time, with OpenMP threads = the box's CPU share (OMP_NUM_THREADS, else nproc); config 1 with
    the same threads; and the torch-CPU float32 functional restatement on the first items until
    `torch_budget_s`."""
    import numpy as np
    from kokoro_hip import workloads
    from oracle import oracle as O
    nproc = len(os.sched_getaffinity(0))
    threads = int(os.environ.get("OMP_NUM_THREADS") or nproc)
    O.set_threads(threads)
    m = O.Model(weights)
    done_s, done_audio, n_items = 0.0, 0.0, 0
    for it in items:
        t0 = time.perf_counter()
        O.synth_item(m, it)
        done_s += time.perf_counter() - t0
        done_audio += it.n_samples / 24000.0
        n_items += 1
        if done_s >= budget_s:
            break
    res = {"value": round(done_audio / done_s, 4), "unit": "audio-s/s", "cores": threads, "kind": "port",
           "sample": f"oracle (oracle/kk_oracle.c, fp32, OpenMP {threads} threads) on the first {n_items} items "
                     f"of the same batch: {done_audio:.1f} audio-s in {done_s:.1f} s",
           "nproc": nproc, "cpu_model": _cpu_model()}
    # config 1: generator only, one item of 100 decoder frames (2.5 s of audio), median of 3
    x, f0, style, seed = workloads.config1_generator_input()
    c1_ri, c1_nz = O.rand_ini(seed), O.gen_noise(seed, 600 * (x.shape[1] // 2) * 9)
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        m.generator(x, f0, style, c1_ri, c1_nz)
        ts.append(time.perf_counter() - t0)
    c1_audio = 600 * (x.shape[1] // 2) / 24000.0
    res["config1"] = {"value": round(c1_audio / statistics.median(ts), 4), "unit": "audio-s/s",
                      "sample": f"oracle, config 1 generator ({c1_audio:.1f} audio-s), median of 3"}
    # torch-CPU functional leg (float32, torch.set_num_threads = the same threads)
    import torch
    from oracle import torch_ref as R
    R.set_dtype(torch.float32)
    torch.set_num_threads(threads)
    done_s, done_audio, n_items = 0.0, 0.0, 0
    with torch.no_grad():
        for it in items:
            t0 = time.perf_counter()
            asr = O.expand_tokens(it.t_en, it.dur)
            xd = R.decoder(weights, asr, it.f0, it.energy, it.ref_s)
            ri, nz = O.item_noise(it)
            R.generator(weights, xd, it.f0, it.ref_s, ri, nz)
            done_s += time.perf_counter() - t0
            done_audio += it.n_samples / 24000.0
            n_items += 1
            if done_s >= torch_budget_s:
                break
    res["torch_cpu"] = {"value": round(done_audio / done_s, 4), "unit": "audio-s/s", "threads": threads,
                        "sample": f"oracle/torch_ref.py in float32 on the first {n_items} items: "
                                  f"{done_audio:.1f} audio-s in {done_s:.1f} s"}
    # and config 1 (the same generator input as the oracle's), median of 3
    ts = []
    with torch.no_grad():
        for _ in range(3):
            t0 = time.perf_counter()
            R.generator(weights, x, f0, style, c1_ri, c1_nz)
            ts.append(time.perf_counter() - t0)
    res["torch_cpu"]["config1"] = {"value": round(c1_audio / statistics.median(ts), 4), "unit": "audio-s/s",
                                   "sample": f"oracle/torch_ref.py, config 1 generator ({c1_audio:.1f} audio-s), "
                                             "median of 3"}
    R.set_dtype(torch.float64)
    return res, m


def parity(model, items, audios, specs, hars):
    """Every item's audio from the timed calls against the fp32 oracle, as the GPU tests compare it:
    end to end for all items (max-abs and SNR), and -- for an item with a spectral bin whose phase
    is set by rounding (atan2's branch cut: a real bin whose imaginary part is +-0 reads +pi on one
    side and -pi on the other; a real DC / Nyquist bin whose sum cancels reads 0 or pi by its sign;
    the generator sees the jump as an input change) -- also against the oracle's STFT and generator
    run from the device's own harmonic-source samples (only the source substituted)."""
    import numpy as np
    from oracle import oracle as O

    def snr(ref, x):
        e = ((x.astype(np.float64) - ref) ** 2).sum()
        return round(float(10 * np.log10((ref.astype(np.float64) ** 2).sum() / max(e, 1e-300))), 2)

    rows = []
    for it, a, g, har in zip(items, audios, specs, hars):
        x = model.decoder(O.expand_tokens(it.t_en, it.dur), it.f0, it.energy, it.ref_s)
        ri, nz = O.item_noise(it)
        ref, spec, _ = model.generator(x, it.f0, it.ref_s, ri, nz, taps=True)
        flips = int((np.abs(g[11:].astype(np.float64) - spec[11:]) > 1e-2).sum())
        row = [it.n_frames, flips, float(np.abs(a - ref).max()), snr(ref, a)]
        sub = 0
        if flips:
            # the oracle's STFT of the device's source samples, or the device's spectrum where that STFT
            # too reads a rounding-decided phase otherwise
            spec_s = O.stft20(har)
            sub = 1 if int((np.abs(g[11:].astype(np.float64) - spec_s[11:]) > 1e-2).sum()) == 0 else 2
            ref, _ = model.generator_from_spec(x, spec_s if sub == 1 else g, it.ref_s)
        rows.append(row + [float(np.abs(a - ref).max()), snr(ref, a), sub])
    r = np.asarray(rows, np.float64)
    return {"items": len(rows), "vs": "oracle/kk_oracle.c fp32",
            "end_to_end": {"maxabs_max": float(r[:, 2].max()), "snr_db_min": float(r[:, 3].min()),
                           "items_within_bar": int(((r[:, 2] <= 2e-3) & (r[:, 3] >= 40.0)).sum())},
            "items_with_phase_unstable_bins": int((r[:, 1] > 0).sum()),
            "substituted": {"source": int((r[:, 6] == 1).sum()), "spectrum": int((r[:, 6] == 2).sum())},
            "maxabs_max": float(r[:, 4].max()), "snr_db_min": float(r[:, 5].min()),
            "items_within_bar": int(((r[:, 4] <= 2e-3) & (r[:, 5] >= 40.0)).sum()),
            "per_item": [[int(x[0]), int(x[1]), float("%.3g" % x[2]), x[3], float("%.3g" % x[4]), x[5]] for x in rows],
            "per_item_fields": ["frames", "phase_unstable_bins", "e2e_maxabs", "e2e_snr_db", "maxabs", "snr_db"],
            "note": "maxabs / snr_db: end to end, or where a phase is set by rounding from the device's source "
                    "samples (the oracle's STFT of them), or its spectrum where that STFT reads such a phase otherwise"}


def config5_leg(ctx, weights, steps, warmup):
    """BASELINE config 5 (128 ragged items, generator frames log-uniform in [80, 4000], ~28 min of
    audio) through the headline's call: host inputs in, host audio out, one kk_forward_decoder_batch
    per step, median of `steps` after `warmup` calls."""
    import numpy as np
    from kokoro_hip import workloads
    items = workloads.config5_items()
    audio_s = sum(it.n_samples for it in items) / 24000.0
    pb = ctx.prepare(items)
    times = []
    for k in range(warmup + steps):
        t0 = time.perf_counter()
        ctx.forward_prepared(pb)
        if k >= warmup:
            times.append(time.perf_counter() - t0)
        if k + 1 < warmup + steps:
            pb.release()
    finite = all(np.isfinite(pb.audio(b)).all() for b in range(len(items)))
    pb.release()
    assert finite, "non-finite audio (config 5)"
    ms = statistics.median(times) * 1e3
    return {"value": round(audio_s / (ms / 1e3), 2), "unit": "audio-s/s", "ms_per_step": round(ms, 3),
            "steps": steps, "items": len(items), "frames": sum(it.n_frames for it in items),
            "audio_s": round(audio_s, 2), "step": "kk_forward_decoder_batch, host inputs -> host audio (median)"}


def e2e_cpu_baseline(w, items, budget_s=15.0):
    """The torch-CPU float32 restatement of every stage (oracle/torch_ref.py) on the shortest items
    of the batch until `budget_s` of wall time, torch threads = the box's CPU share."""
    import torch
    from oracle import oracle as O
    from oracle import torch_ref as R
    threads = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    torch.set_num_threads(threads)
    R.set_dtype(torch.float32)
    order = sorted(range(len(items)), key=lambda b: len(items[b].ids))
    done_s, t0, n_items = 0.0, time.perf_counter(), 0
    try:
        for b in order:
            it = items[b]
            with torch.no_grad():
                pred, t_en, f0, n = R.upstream(w, it.ids, it.ref_s)
                x = R.decoder(w, O.expand_tokens(t_en.numpy(), pred), f0, n, it.ref_s)
                R.generator(w, x, f0, it.ref_s, O.rand_ini(it.seed), O.gen_noise(it.seed, 600 * int(pred.sum()) * 9))
            done_s += 600 * int(pred.sum()) / 24000.0
            n_items += 1
            if time.perf_counter() - t0 > budget_s:
                break
    finally:
        R.set_dtype(torch.float64)
    el = time.perf_counter() - t0
    return {"value": round(done_s / el, 3), "unit": "audio-s/s", "cores": threads, "kind": "port",
            "sample": f"the {n_items} shortest items of the batch ({done_s:.1f} s of audio), torch-CPU float32 "
                      "restatement of every stage (oracle/torch_ref.py)", "cpu_model": _cpu_model()}


def e2e_leg(steps, warmup, with_cpu):
    """BASELINE config 4, the whole forward from phoneme ids (kk_forward_batch): 64 ragged items,
    20-510 ids uniform over the vocabulary, random-init weights of every stage.  One step = one
    C-ABI call from host ids to host audio (token phase, the durations on the host from one copy of
    the logits, frame layout, prosody, decoder, generator, iSTFT, audio back).  Beside it: the same
    batch as a device-resident plan (token phase included), a per-launch profiling pass by kernel
    class, and the torch-CPU float32 restatement (oracle/torch_ref.py) on a bounded sample."""
    import numpy as np
    from kokoro_hip import api, model_spec, workloads
    w = model_spec.random_model_weights(seed=0)
    items = workloads.config4_items()
    ctx = api.Context(0)
    ctx.upload_model(w)
    # the C-ABI call alone: the results stay in the library's pinned output blocks until released
    pb = ctx.prepare_ids(items)
    for _ in range(warmup):
        ctx.forward_ids_prepared(pb)
        pb.release()
    times = []
    for k in range(steps):
        t0 = time.perf_counter()
        ctx.forward_ids_prepared(pb)
        times.append(time.perf_counter() - t0)
        if k + 1 < steps:
            pb.release()
    res = [(pb.audio(b), pb.pred_dur(b)) for b in range(len(items))]
    pb.release()
    frames = sum(int(d.sum()) for _, d in res)
    assert all(np.isfinite(a).all() for a, _ in res), "non-finite audio"
    audio_s = 600 * frames / 24000.0
    ms = statistics.median(times) * 1e3
    plan = api.Plan.full(ctx, items)
    for until, key in (("prosody", "to_prosody_ms"), ("all", "kernel_only_ms")):
        plan.run(until)
        plan.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            plan.run(until)
        plan.sync()
        if key == "kernel_only_ms":
            k_ms = (time.perf_counter() - t0) * 1e3 / steps
        else:
            p_ms = (time.perf_counter() - t0) * 1e3 / steps
    ctx.set_profiling(True)
    ctx.profile_read()
    plan.run()
    plan.sync()
    prof = ctx.profile_read()
    ctx.set_profiling(False)
    plan.free()
    ctx.close()
    # the recurrences are sequential in time: their cost is the longest item's steps
    lens = [len(it.ids) for it in items]
    frames_max = max(int(d.sum()) for _, d in res)
    lstm_steps = 5 * max(lens) + frames_max
    cls = {k: v for k, v in prof.items()}
    def rate(k, peak):
        v = cls.get(k)
        if not v or v["ms"] <= 0:
            return None
        t = v["flop"] / (v["ms"] / 1e3) / 1e12
        return {"serial_ms": round(v["ms"], 3), "launches": v["launches"], "tflops": round(t, 1),
                "peak_tflops": peak, "frac": round(t / peak, 4)}
    out = {"workload": "config4: phoneme ids -> audio, batch 64 ragged, 20-510 ids uniform over vocab 178",
           "value": round(audio_s / (ms / 1e3), 2), "unit": "audio-s/s", "ms_per_step": round(ms, 3),
           "step": "kk_forward_batch, host ids -> host audio (median of K calls)", "items": len(items),
           "ids": sum(len(it.ids) for it in items), "frames": frames, "audio_s": round(audio_s, 2),
           "frames_per_token": round(frames / sum(len(it.ids) for it in items), 3),
           "kernel_only": {"value": round(audio_s / (k_ms / 1e3), 2), "ms_per_step": round(k_ms, 3),
                           "through_prosody_ms": round(p_ms, 3),
                           "step": "kk_plan_run of an ids-level plan, token phase included (mean of K)"},
           "serial_ms_by_class": {k: round(v["ms"], 3) for k, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"])},
           "kernels": {
               "lstm": {"serial_ms": round(cls["lstm"]["ms"], 3), "critical_steps": lstm_steps,
                        "us_per_step": round(1e3 * cls["lstm"]["ms"] / lstm_steps, 2),
                        "note": "5 token-level BiLSTMs (longest item's ids) + the shared BiLSTM (longest item's "
                                "frames); each (item, direction) on two CUs (four for spans of >= 1,024 steps: the shared "
                                "BiLSTM) with all of W_hh on chip: per step ~0.9 (0.45) us of f32 FMA and the "
                                "exchange of h through L2"},
               "attention": rate("attention", PEAK_F32_MFMA_TFLOPS),
               "linear": rate("linear", PEAK_BF16_TFLOPS),
               "prosody_conv": rate("prosody_conv", PEAK_BF16_TFLOPS),
               "snake_conv": rate("snake_conv", PEAK_BF16_TFLOPS)}}
    if with_cpu:
        out["cpu_baseline"] = e2e_cpu_baseline(w, items)
    return out


def _traffic(config):
    """HBM bytes per Snake-conv launch (FETCH_SIZE + WRITE_SIZE, copy-calibrated) from the committed
    PMC summary of the config-3 workload; None for other workloads or when it is absent."""
    path = os.path.join(ROOT, "profiles", "conv_mfma_snake_config3_traffic.json")
    if config != 3 or not os.path.exists(path):
        return None
    with open(path) as f:
        return round(json.load(f)["traffic_bytes_per_launch"])


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-events", action="store_true", help="skip the per-launch profiling pass")
    ap.add_argument("--no-e2e", action="store_true", help="skip the ids-level (config 4) leg")
    ap.add_argument("--e2e-steps", type=int, default=5)
    ap.add_argument("--no-config5", action="store_true", help="skip the config-5 host-in -> host-out leg")
    ap.add_argument("--parity-items", type=int, default=-1,
                    help="items of the batch compared with the oracle (default: all of config 3, 8 of config 5)")
    ap.add_argument("--only-e2e", action="store_true", help="run only the ids-level (config 4) leg")
    ap.add_argument("--layers", default="", help="write the profiling pass's per-launch table (JSON) here")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run one plain copy kernel over this many MiB (reference for PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the path is data-parallel over independent items and this "
              f"build measures one GPU's share (requested --gpus {args.gpus}); more GPUs would each take "
              f"their own batches of items, with no traffic between them.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    from kokoro_hip import api, model_spec, workloads

    if args.only_e2e:
        print(json.dumps({"e2e": e2e_leg(args.e2e_steps, 1, not args.no_cpu)}), flush=True)
        return
    if args.calibrate_copy_mib:
        # one elementwise kernel that reads and writes exactly M MiB: the FETCH_SIZE / WRITE_SIZE
        # counters of this dispatch scale those of the conv kernels to bytes
        import torch
        a = torch.ones(args.calibrate_copy_mib << 18, device="cuda:0")
        b = torch.empty_like(a)
        torch.cuda.synchronize()
        torch.mul(a, 1.0, out=b)
        torch.cuda.synchronize()
        del a, b
        print(f"# calibration copy: {args.calibrate_copy_mib} MiB", file=sys.stderr, flush=True)

    weights = model_spec.random_weights(seed=0)
    if args.config == 5:
        items = workloads.config5_items()
        wl = "config5: decoder+generator, 128 ragged items, G log-uniform [80, 4000]"
    else:
        items = workloads.config3_items()
        wl = "config3: decoder+generator, batch 32 ragged, N ~ U[100, 800] frames"
    ctx = api.Context(0)
    ctx.upload_model(weights)
    samples = sum(it.n_samples for it in items)
    audio_s = samples / 24000.0

    # ---- the headline: host inputs in, host audio out, one C-ABI call per step
    pb = ctx.prepare(items)
    for _ in range(args.warmup):
        ctx.forward_prepared(pb)
        pb.release()
    times = []
    t_region0 = time.perf_counter()
    for k in range(args.steps):
        t0 = time.perf_counter()
        ctx.forward_prepared(pb)
        times.append(time.perf_counter() - t0)
        if k + 1 < args.steps:
            pb.release()
    t_region = time.perf_counter() - t_region0
    audios = [pb.audio(b).copy() for b in range(len(items))]
    finite = all(np.isfinite(a).all() for a in audios)
    pb.release()
    assert finite, "non-finite audio"
    ms = statistics.median(times) * 1e3
    value = audio_s / (ms / 1e3)

    # ---- device-resident steps (kernel_only) and the per-launch profiling pass
    plan = api.Plan.decoder(ctx, items)
    info = plan.info()
    print(f"# device {ctx.device_name()}  items {len(items)}  frames {info['frames']}  audio {audio_s:.1f} s  "
          f"plan {info['device_bytes'] / 2**30:.2f} GiB  one-shot median {ms:.2f} ms", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        plan.run()
    plan.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        plan.run()
    plan.sync()
    k_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    info = plan.info()
    prof = {}
    if not args.no_events:
        ctx.set_profiling(True)
        ctx.profile_read()
        for _ in range(args.steps):
            plan.run()
        plan.sync()
        if args.layers:
            per = {}
            for name, cls, lms, fl, by in ctx.profile_launches():
                e = per.setdefault(name, {"cls": cls, "launches": 0, "ms": 0.0, "flop": 0.0, "bytes": 0.0})
                e["launches"] += 1
                e["ms"] += lms
                e["flop"] += fl
                e["bytes"] += by
            with open(args.layers, "w") as f:
                json.dump({"steps": args.steps, "workload": wl, "layers": per}, f, indent=1)
        prof = ctx.profile_read()
        ctx.set_profiling(False)
    plan.free()
    # the parity leg's spectra and harmonic-source samples: one more run of a plan with the source tap
    # (its audio equals the timed calls' bit for bit)
    os.environ["KOKORO_HIP_TEST_TAP_SOURCE"] = "1"
    try:
        plan = api.Plan.decoder(ctx, items)
    finally:
        del os.environ["KOKORO_HIP_TEST_TAP_SOURCE"]
    plan.run()
    same = all(np.array_equal(a, b) for a, b in zip(plan.fetch(), audios))
    specs = [plan.tap("spec", b, (22, 120 * it.n_frames + 1)) for b, it in enumerate(items)]
    hars = [plan.tap("har", b, (600 * it.n_frames,)) for b, it in enumerate(items)]
    plan.free()

    roof, util, hbm = None, None, None
    if prof:
        sn = prof["snake_conv"]
        achieved = sn["flop"] / (sn["ms"] / 1e3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": _traffic(args.config),
                "kernel": "conv_mfma_kernel<PRO_ADAIN_SNAKE> (48 Snake-block convs per step)",
                "avg_launch_ms": round(sn["ms"] / max(sn["launches"], 1), 4),
                "flop_per_launch": sn["flop"] / max(sn["launches"], 1),
                "hbm_bytes_per_launch": sn["bytes"] / max(sn["launches"], 1)}
        gbs = sn["bytes"] / (sn["ms"] / 1e3) / 1e9
        roof.update({"hbm_achieved_gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)})
        convs = {k: v for k, v in prof.items() if k in ("snake_conv", "decoder_conv", "convt", "post_conv")}
        conv_ms = sum(v["ms"] for v in convs.values())
        conv_flop = sum(v["flop"] for v in convs.values())
        util = {k: {"launches_per_step": v["launches"] // args.steps, "ms_per_step": round(v["ms"] / args.steps, 3),
                    "tflops": round(v["flop"] / max(v["ms"], 1e-9) / 1e9, 1),
                    "gbs": round(v["bytes"] / max(v["ms"], 1e-9) / 1e6, 1)} for k, v in convs.items()}
        util["all_convs_mfma_util_pct"] = round(100 * conv_flop / (conv_ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 2)
        all_ms = sum(v["ms"] for v in prof.values())
        util["conv_share_of_kernel_time_pct"] = round(100 * conv_ms / all_ms, 1)
        hbm = {}
        for k in BANDWIDTH_KERNELS:
            if k not in prof:
                continue
            v = prof[k]
            g = v["bytes"] / max(v["ms"], 1e-9) / 1e6
            hbm[k] = {"launches_per_step": v["launches"] // args.steps, "ms_per_step": round(v["ms"] / args.steps, 4),
                      "bytes_per_launch": round(v["bytes"] / max(v["launches"], 1)), "gbs": round(g, 1),
                      "frac": round(g / PEAK_HBM_GBS, 4)}
        hbm["serial_kernel_ms_per_step"] = round(all_ms / args.steps, 3)

    res = {
        "metric": "audio-sec synthesized per wall-sec at batch 32 ragged; conv MFMA util %",
        "value": round(value, 2),
        "unit": "audio-s/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded inputs, random-init weights)",
        "config": {"workload": wl, "items": len(items), "frames": info["frames"], "samples": info["samples"],
                   "audio_s": round(audio_s, 2), "conv_tflop_per_step": round(info["conv_flop"] / 1e12, 3),
                   "launches_per_step": info["launches"],
                   "step": "kk_forward_decoder_batch, host inputs -> host audio (median of K calls)",
                   "timed_region_s": round(t_region, 3)},
        "kernel_only": {"value": round(audio_s / (k_ms / 1e3), 2), "unit": "audio-s/s", "ms_per_step": round(k_ms, 3),
                        "step": "kk_plan_run with inputs resident in HBM (mean of K)"},
        "roofline": roof,
        "conv_mfma": util,
        "hbm": hbm,
    }
    # parity of the measured batch: every item of the timed calls against the fp32 oracle
    from oracle import oracle as O
    if args.no_cpu:
        model = O.Model(weights)
    else:
        res["cpu_baseline"], model = cpu_baseline(weights, items)
    t0 = time.perf_counter()
    k = args.parity_items if args.parity_items > 0 else (len(items) if args.config != 5 else 8)
    res["parity"] = parity(model, items[:k], audios[:k], specs[:k], hars[:k])
    res["parity"]["tap_plan_equals_timed_call"] = same
    print(f"# parity leg {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    if args.config != 5 and not args.no_config5:
        res["config5"] = config5_leg(ctx, weights, max(3, args.steps // 4), args.warmup)
    ctx.close()
    if not args.no_e2e:
        res["e2e"] = e2e_leg(args.e2e_steps, 1, not args.no_cpu)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
