"""Summaries of rocprofv3 output for bench.py runs of the config-3 workload.

    python -m kokoro_hip.profsum stats <trace_dir> <steps> [<trailing>]
        per-kernel table from a `rocprofv3 --kernel-trace` CSV run of bench.py, plus the average
        Snake-block conv duration of its profiling pass (<steps> runs, followed by <trailing> other
        runs: 1 for bench.py's config-3 leg, whose parity leg runs a plan once more)
    python -m kokoro_hip.profsum serial <trace_dir> <steps> [<trailing>]
        per-kernel table of bench.py's profiling pass alone (<steps> runs before the trace's last
        <trailing>, every kernel alone on one stream), for any workload whose runs end with the iSTFT
    python -m kokoro_hip.profsum kernels <trace_dir>
        per-kernel table (calls, total, average, share) of any `rocprofv3 --kernel-trace --stats` run
    python -m kokoro_hip.profsum layers <layers.json>
        per-layer table of bench.py's profiling pass (`--layers`): every kernel alone on the stream,
        HIP events around each launch; time per launch, algorithmic TFLOP/s and GB/s, and the
        fraction of the launch's roofline floor max(FLOP / 2.5 PFLOP/s, bytes / 8 TB/s)
    python -m kokoro_hip.profsum traffic <fetch_dir> <write_dir> <M>
        HBM bytes per Snake-conv launch from a `--pmc FETCH_SIZE` and a `--pmc WRITE_SIZE` run of
        `bench.py --calibrate-copy-mib M`, each scaled by what the same counter reads for the plain
        copy kernel of known size (M MiB read, M MiB written) that the run starts with; prints JSON

Run from the kokoro-rust_amd directory (or with it on sys.path).  Only reads CSV files.
"""
import csv
import json
import os
import re
import sys

SNAKE = re.compile(r"conv_mfma_kernel<4,")
COPY = re.compile(r"elementwise_kernel<.*MulFunctor")  # torch's out = a * 1 over M MiB of float32


def snake_layers():
    """The 48 Snake-block convs of one config-3 step in launch order: per stage the noise resblock,
    then resblocks k3, k7, k11; per block dilations 1, 3, 5; per dilation conv1 then conv2."""
    from kokoro_hip import workloads
    items = workloads.config3_items()
    frames = sum(it.n_frames for it in items)
    cols0 = 20 * frames
    cols1 = sum(120 * it.n_frames + 1 for it in items)
    out = []
    for st, c, cols, nrk in [(0, 256, cols0, 7), (1, 128, cols1, 11)]:
        for blk, k in [("noise_res", nrk), ("resblock", 3), ("resblock", 7), ("resblock", 11)]:
            for d in (1, 3, 5):
                for cv in (1, 2):
                    # bytes per column and channel; every stream is fp16: conv1 reads the stream
                    # (or the stage input) and writes h (2 + 2); conv2 reads h and adds it to the
                    # stream (or the stage input) into the stream (2 + 2 + 2); the last conv of
                    # the three resblocks reads the three streams and writes their mean as the next
                    # layer's bf16 operand (2 + 3 x 2 + 2)
                    per_col = 4 if cv == 1 else (10 if (blk, k, d) == ("resblock", 11, 5) else 6)
                    by = c * cols * per_col
                    out.append({"name": f"stage{st} {blk} k{k} d{d} conv{cv}", "flop": 2.0 * c * c * k * cols,
                                "bytes": by})
    return out, frames


def _rows(path):
    with open(path) as f:
        return list(csv.DictReader(f))


def _short(name):
    m = re.search(r"conv_mfma_kernel<([^>]*)>", name)
    if m:
        return f"conv_mfma_kernel<{m.group(1)}>"
    m = re.search(r"(\w+)(<[^(]*>)?\(", name)
    return m.group(1) if m else name[:48]


def _table(rows, dur, per_step=0):
    per = {}
    for r in rows:
        per.setdefault(_short(r["Kernel_Name"]), []).append(dur(r))
    total = sum(sum(v) for v in per.values())
    head = "| kernel | calls | total ms | avg us | % |" + (" ms per step |" if per_step else "")
    lines = [head, "|---|---:|---:|---:|---:|" + ("---:|" if per_step else "")]
    for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        line = f"| `{k}` | {len(v)} | {sum(v) / 1e3:.2f} | {sum(v) / len(v):.1f} | {100 * sum(v) / total:.2f} |"
        lines.append(line + (f" {sum(v) / 1e3 / per_step:.3f} |" if per_step else ""))
    return lines, total


def _serial_window(rows, steps, trailing):
    """The dispatches of bench.py's profiling pass: the `steps` runs that come before the trace's
    last `trailing` runs (each run ends with an iSTFT): every dispatch that starts after the end of
    the run before them and ends by the end of their last iSTFT.  None when the trace is shorter."""
    ist = [r for r in rows if "istft_kernel" in r["Kernel_Name"]]
    if len(ist) <= steps + trailing:
        return None
    t0 = int(ist[-steps - trailing - 1]["End_Timestamp"])
    t1 = int(ist[-trailing - 1]["End_Timestamp"])
    return [r for r in rows if int(r["Start_Timestamp"]) > t0 and int(r["End_Timestamp"]) <= t1]


def _serial_lines(rows, steps, dur, trailing=0):
    """The per-kernel table of bench.py's profiling pass (`_serial_window`); empty when the trace
    has no such run."""
    ser = _serial_window(rows, steps, trailing)
    if not ser:
        return []
    st, tot = _table(ser, dur, steps)
    after = f" before the trace's last {trailing}" if trailing else ""
    return [f"The profiling pass alone ({len(ser)} dispatches of the {steps} runs{after}, each kernel alone on "
            f"one stream; {tot / 1e3 / steps:.3f} ms of kernels per run):", ""] + st


def serial(trace_dir, steps, trailing=0):
    """The per-kernel table of bench.py's profiling pass alone (`steps` runs, then `trailing` more)."""
    rows = _rows(os.path.join(trace_dir, "run_kernel_trace.csv"))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    return "\n".join(_serial_lines(rows, steps, dur, trailing))


def stats(trace_dir, steps, trailing=0):
    """Per-kernel table of the whole trace; the same table over bench.py's profiling pass alone
    (`steps` runs followed by `trailing` other runs, every kernel alone on one stream: no span
    includes another stream's work); and the Snake-block convs' average duration per launch in that
    pass."""
    rows = _rows(os.path.join(trace_dir, "run_kernel_trace.csv"))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    lines, _ = _table(rows, dur)
    st = _serial_lines(rows, steps, dur, trailing)
    if st:
        lines += [""] + st
    layers, frames = snake_layers()
    sn = [r for r in rows if SNAKE.search(r["Kernel_Name"])]
    win = _serial_window(rows, steps, trailing)
    last = [r for r in win if SNAKE.search(r["Kernel_Name"])] if win else sn[-steps * len(layers):]
    avg = sum(dur(r) for r in last) / len(last)
    fl = sum(l["flop"] for l in layers) / len(layers)
    lines += ["", f"Snake-block convs of the profiling pass ({steps} steps, {len(last)} dispatches, "
                  f"each alone on the stream): **{avg:.1f} us** per launch on average, "
                  f"{fl / avg / 1e6:.1f} TFLOP/s algorithmic ({100 * fl / avg / 1e6 / 2500:.1f}% of 2.5 PFLOP/s); "
                  f"all {len(sn)} Snake dispatches of the trace (the timed steps overlap three chains) "
                  f"average {sum(dur(r) for r in sn) / len(sn):.1f} us."]
    return "\n".join(lines)


PEAK_FLOPS, PEAK_BYTES = 2.5e15, 8e12


def kernels_table(trace_dir, top=40):
    """Every kernel of a `rocprofv3 --kernel-trace --stats` CSV run: calls, total, average, share."""
    rows = []
    for root, _, files in os.walk(trace_dir):
        for f in files:
            if f.endswith("kernel_stats.csv"):
                rows += _rows(os.path.join(root, f))
    tot = sum(float(r["TotalDurationNs"]) for r in rows) or 1.0
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    out = ["| kernel | calls | total ms | avg us | % |", "|---|---:|---:|---:|---:|"]
    for r in rows[:top]:
        t = float(r["TotalDurationNs"])
        out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {t / 1e6:.2f} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{100 * t / tot:.2f} |")
    out.append(f"\nAll kernels: {tot / 1e6:.2f} ms over {sum(int(r['Calls']) for r in rows)} dispatches.")
    return "\n".join(out)


def layers_table(path):
    with open(path) as f:
        d = json.load(f)
    k = d["steps"]
    lines = [f"Per-launch profile, {d['workload']} ({k} steps; each kernel alone on the stream):", "",
             "| layer | class | launches/step | us per launch | TFLOP/s | GB/s | floor us | frac of floor |",
             "|---|---|---:|---:|---:|---:|---:|---:|"]
    tot = {}
    for name, e in d["layers"].items():
        n = e["launches"]
        us = e["ms"] * 1e3 / n
        fl, by = e["flop"] / n, e["bytes"] / n
        floor = max(fl / PEAK_FLOPS, by / PEAK_BYTES) * 1e6
        t = tot.setdefault(e["cls"], [0.0, 0.0, 0.0, 0.0])
        t[0] += e["ms"] / k
        t[1] += e["flop"] / k
        t[2] += e["bytes"] / k
        t[3] += floor * n / k / 1e3
        lines.append(f"| {name} | {e['cls']} | {n // k} | {us:.1f} | {fl / max(us, 1e-9) / 1e6:.1f} | "
                     f"{by / max(us, 1e-9) / 1e3:.1f} | {floor:.1f} | {floor / max(us, 1e-9):.3f} |")
    lines += ["", "| class | ms per step | TFLOP/s | GB/s | floor ms | frac of floor |", "|---|---:|---:|---:|---:|---:|"]
    for c, (ms, fl, by, floor) in sorted(tot.items(), key=lambda kv: -kv[1][0]):
        lines.append(f"| {c} | {ms:.3f} | {fl / ms / 1e9:.1f} | {by / ms / 1e6:.1f} | {floor:.3f} | "
                     f"{floor / ms:.3f} |")
    all_ms = sum(v[0] for v in tot.values())
    lines.append(f"| **all** | {all_ms:.3f} | | | {sum(v[3] for v in tot.values()):.3f} | |")
    return "\n".join(lines)


def _per_dispatch(run_dir, counter):
    rows = [r for r in _rows(os.path.join(run_dir, "run_counter_collection.csv")) if r["Counter_Name"] == counter]
    by = {}
    for r in rows:  # one row per dispatch (the counter is summed over the device)
        by.setdefault(int(r["Dispatch_Id"]), [r["Kernel_Name"], 0.0])[1] += float(r["Counter_Value"])
    return [by[k] for k in sorted(by)]


def traffic(fetch_dir, write_dir, mib):
    """FETCH_SIZE and WRITE_SIZE are in KiB per dispatch; the copy kernel moves M MiB each way."""
    res = {}
    layers, _ = snake_layers()
    for key, d, counter in [("fetch", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE")]:
        disp = _per_dispatch(d, counter)
        copies = [v for n, v in disp if COPY.search(n)]
        scale = (mib * 1024.0) / (sum(copies) / len(copies))
        sn = [v for n, v in disp if SNAKE.search(n)]
        n = len(sn) - len(sn) % len(layers)
        res[key] = {"copy_kib_expected": mib * 1024.0, "copy_kib_read": sum(copies) / len(copies),
                    "scale": round(scale, 4), "snake_launches": n,
                    "kib_per_launch_raw": sum(sn[:n]) / n, "bytes_per_launch": sum(sn[:n]) / n * 1024.0 * scale}
    alg = sum(l["bytes"] for l in layers) / len(layers)
    res["traffic_bytes_per_launch"] = res["fetch"]["bytes_per_launch"] + res["write"]["bytes_per_launch"]
    res["algorithmic_bytes_per_launch"] = alg
    res["traffic_over_algorithmic"] = round(res["traffic_bytes_per_launch"] / alg, 3)
    return res


def counters(run_dir):
    """MFMA utilisation of the conv kernels from one `rocprofv3 --pmc` pass (SQ_VALU_MFMA_BUSY_CYCLES,
    SQ_INSTS_MFMA, GRBM_GUI_ACTIVE, ...; the counters summed over the device per dispatch).  The
    matrix cores' busy cycles (SQ_VALU_MFMA_BUSY_CYCLES: each v_mfma_f32_32x32x16_bf16 counts its
    32 pipeline cycles) against the cycles every SIMD had while the dispatch ran (GRBM_GUI_ACTIVE,
    summed over the XCDs, / XCDs x SIMDs); the sustained clock is GRBM_GUI_ACTIVE / XCDs / duration.
    Returns the markdown table and the totals."""
    gpu = [r for r in _rows(os.path.join(run_dir, "run_agent_info.csv")) if "GPU" in r["Agent_Type"]][0]
    simds, xcc = int(gpu["Simd_Count"]), int(gpu["Num_Xcc"])
    disp = {}
    for r in _rows(os.path.join(run_dir, "run_counter_collection.csv")):
        d = disp.setdefault(int(r["Dispatch_Id"]), {"name": _short(r["Kernel_Name"]),
                                                    "ns": int(r["End_Timestamp"]) - int(r["Start_Timestamp"])})
        d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    groups = {}
    for d in disp.values():
        if not d["name"].startswith("conv_mfma_kernel"):
            continue
        cls = "Snake-block convs" if SNAKE.search(d["name"]) else "other convs (decoder, ConvT, conv_post)"
        for key in (cls, "all convs"):
            g = groups.setdefault(key, {"n": 0, "ns": 0.0, "busy": 0.0, "insts": 0.0, "gui": 0.0})
            g["n"] += 1
            g["ns"] += d["ns"]
            g["busy"] += d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
            g["insts"] += d.get("SQ_INSTS_MFMA", 0.0)
            g["gui"] += d.get("GRBM_GUI_ACTIVE", 0.0)
    lines = ["| kernels | dispatches | ms | MFMA instructions | busy cycles per MFMA | sustained clock (GHz) | "
             "MFMA busy (of every SIMD's cycles) |", "|---|---:|---:|---:|---:|---:|---:|"]
    out = {}
    for key, g in groups.items():
        util = g["busy"] / max(g["gui"] / xcc * simds, 1.0)
        clock = g["gui"] / xcc / max(g["ns"], 1.0)
        out[key] = {"util": util, "clock_ghz": clock, "mfma_insts": g["insts"], "ms": g["ns"] / 1e6}
        lines.append(f"| {key} | {g['n']} | {g['ns'] / 1e6:.2f} | {g['insts']:.4g} | "
                     f"{g['busy'] / max(g['insts'], 1.0):.1f} | {clock:.2f} | {100 * util:.1f}% |")
    return "\n".join(lines), out


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    trailing = int(sys.argv[4]) if len(sys.argv) > 4 and sys.argv[1] in ("stats", "serial") else 0
    if sys.argv[1] == "stats":
        print(stats(sys.argv[2], int(sys.argv[3]), trailing))
    elif sys.argv[1] == "serial":
        print(serial(sys.argv[2], int(sys.argv[3]), trailing))
    elif sys.argv[1] == "kernels":
        print(kernels_table(sys.argv[2]))
    elif sys.argv[1] == "layers":
        print(layers_table(sys.argv[2]))
    elif sys.argv[1] == "traffic":
        print(json.dumps(traffic(sys.argv[2], sys.argv[3], float(sys.argv[4])), indent=1))
    elif sys.argv[1] == "counters":
        print(counters(sys.argv[2])[0])
    else:
        sys.exit(__doc__)
