"""Benchmark: batched ragged Kokoro-82M decoder + iSTFTNet generator on one MI355X.

Workload (the metric's config): 32 ragged items, N ~ U[100, 800] decoder
frames each, seeded synthetic inputs and random-init weights.  One step = one pass of the hot path
over the batch (kk_plan_run: duration expansion -> decoder -> harmonic source + STFT -> generator ->
iSTFT), with every input already resident in HBM.  `value` = audio seconds synthesized per wall
second, timed without per-launch instrumentation.  The roofline block reports the dominant kernel
(the Snake-block MFMA convolutions): algorithmic FLOP / summed HIP-event time of those launches over
a second timed pass of the same K steps with an event pair around every conv launch on the
library's stream (with per-launch profiling on, the library runs the generator's three resblock
chains in that one stream instead of three), against the bf16 dense MFMA peak; its `traffic` is the HBM bytes per launch measured by the FETCH_SIZE / WRITE_SIZE
counters (profiles/conv_mfma_snake_config3_traffic.json, made with --calibrate-copy-mib and
kokoro_hip/profsum.py).  The CPU baseline is the oracle (a CPU restatement of the same path) on a bounded
sample of the same batch.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--config 3|5]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "kokoro-rust_amd"))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0


def cpu_baseline(weights, items, budget_s=12.0):
    """Oracle (fp32 C restatement of the path) on the first items of the batch, OpenMP threads =
    the host cores available to this process (at most 16), until `budget_s` of CPU wall time."""
    from oracle import oracle as O
    cores = min(16, len(os.sched_getaffinity(0)))
    O.set_threads(cores)
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
    return {"value": round(done_audio / done_s, 4), "unit": "audio-s/s", "cores": cores, "kind": "port",
            "sample": f"oracle (oracle/kk_oracle.c, fp32, OpenMP {cores} threads) on the first {n_items} items "
                      f"of the same batch: {done_audio:.1f} audio-s in {done_s:.1f} s"}


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
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-pcie", action="store_true", help="skip the host-buffer (PCIe-inclusive) rate")
    ap.add_argument("--no-events", action="store_true", help="time without the per-launch HIP events")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run one plain copy kernel over this many MiB (reference for PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the path is data-parallel over independent items and this "
              f"build measures one GPU's share (requested --gpus {args.gpus}); see DESIGN.md for sharding.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    from kokoro_hip import api, model_spec, workloads

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
    plan = api.Plan.decoder(ctx, items)
    info = plan.info()
    audio_s = info["samples"] / 24000.0
    print(f"# device {ctx.device_name()}  items {len(items)}  frames {info['frames']}  audio {audio_s:.1f} s  "
          f"plan {info['device_bytes'] / 2**30:.2f} GiB", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        plan.run()
    plan.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        plan.run()
    plan.sync()
    t1 = time.perf_counter()
    info = plan.info()
    ms = (t1 - t0) * 1e3 / args.steps
    value = audio_s / (ms / 1e3)
    # per-kernel durations: the same K steps again, launched one by one with a HIP event pair
    # around every conv launch on the library's stream (the resblock chains serial, so that each
    # kernel has the GPU to itself)
    prof = {}
    if not args.no_events:
        ctx.set_profiling(True)
        ctx.profile_read()
        for _ in range(args.steps):
            plan.run()
        plan.sync()
        prof = ctx.profile_read()
        ctx.set_profiling(False)

    # parity spot check of the measured batch's first item is done by the test suite; here only a
    # sanity check that the output is finite
    out = plan.fetch()
    assert all(np.isfinite(a).all() for a in out[:2])

    roof = None
    util = None
    if prof:
        sn = prof["snake_conv"]
        achieved = sn["flop"] / (sn["ms"] / 1e3) / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": _traffic(args.config),
                "kernel": "conv_mfma_kernel<PRO_ADAIN_SNAKE> (48 Snake-block convs per step)",
                "avg_launch_ms": round(sn["ms"] / max(sn["launches"], 1), 4),
                "flop_per_launch": sn["flop"] / max(sn["launches"], 1)}
        if args.config == 3:
            # the same launches against HBM: algorithmic bytes (activations in and out) per launch
            from kokoro_hip import profsum
            layers, _ = profsum.snake_layers()
            alg = sum(l["bytes"] for l in layers) / len(layers)
            gbs = alg / (roof["avg_launch_ms"] / 1e3) / 1e9
            roof.update({"hbm_bytes_per_launch": alg, "hbm_achieved_gbs": round(gbs, 1),
                         "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)})
        conv_ms = sum(v["ms"] for v in prof.values())
        conv_flop = sum(v["flop"] for v in prof.values())
        util = {k: {"launches": v["launches"], "ms_per_step": round(v["ms"] / args.steps, 3),
                    "tflops": round(v["flop"] / max(v["ms"], 1e-9) / 1e9, 1)} for k, v in prof.items()}
        util["all_convs_mfma_util_pct"] = round(100 * conv_flop / (conv_ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS, 2)
        util["conv_share_of_step_pct"] = round(100 * conv_ms / args.steps / ms, 1)

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
                   "launches_per_step": info["launches"]},
        "roofline": roof,
        "conv_mfma": util,
    }
    plan.free()
    if not args.no_pcie:
        # the one-shot entry with host buffers (upload, plan build, run, audio back): reported
        # beside the device-resident rate, never as `value`
        ctx.forward_decoder_batch(items)
        t0 = time.perf_counter()
        reps = 3
        for _ in range(reps):
            ctx.forward_decoder_batch(items)
        dt = (time.perf_counter() - t0) / reps
        res["pcie_inclusive"] = {"value": round(audio_s / dt, 2), "unit": "audio-s/s", "ms_per_call": round(dt * 1e3, 2),
                                 "entry": "kk_forward_decoder_batch (host inputs in, host audio out)"}
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(weights, items)
    ctx.close()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
