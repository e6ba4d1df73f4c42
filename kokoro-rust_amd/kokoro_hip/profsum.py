"""Summaries of rocprofv3 output for bench.py runs of the config-3 workload.

    python -m kokoro_hip.profsum stats <trace_dir>
        per-kernel table from a `rocprofv3 --kernel-trace` CSV run, plus the per-layer breakdown of
        the 48 Snake-block convolutions of one step (algorithmic TFLOP/s and GB/s per layer)
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
                    # conv1 reads the f32 stream and writes fp16; conv2 reads fp16 and the f32
                    # residual, writes f32; the last conv of the three resblocks also reads the
                    # other two blocks' streams and writes their mean
                    per_col = 6 if cv == 1 else (18 if (blk, k, d) == ("resblock", 11, 5) else 10)
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


def stats(trace_dir):
    rows = _rows(os.path.join(trace_dir, "run_kernel_trace.csv"))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    dur = lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    per = {}
    for r in rows:
        per.setdefault(_short(r["Kernel_Name"]), []).append(dur(r))
    total = sum(sum(v) for v in per.values())
    lines = ["| kernel | calls | total ms | avg us | % |", "|---|---:|---:|---:|---:|"]
    for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{k}` | {len(v)} | {sum(v) / 1e3:.2f} | {sum(v) / len(v):.1f} | {100 * sum(v) / total:.2f} |")
    layers, frames = snake_layers()
    sn = [r for r in rows if SNAKE.search(r["Kernel_Name"])]
    n_steps = len(sn) // len(layers)
    lines += ["", f"Snake-block convs, per layer (config 3: {frames} frames; average over {n_steps} steps):", "",
              "| layer | avg us | TFLOP/s | GB/s (algorithmic) |", "|---|---:|---:|---:|"]
    acc = [[] for _ in layers]
    for i, r in enumerate(sn[: n_steps * len(layers)]):
        acc[i % len(layers)].append(dur(r))
    tot = 0.0
    for lay, v in zip(layers, acc):
        us = sum(v) / len(v)
        tot += us
        lines.append(f"| {lay['name']} | {us:.1f} | {lay['flop'] / us / 1e6:.1f} | {lay['bytes'] / us / 1e3:.1f} |")
    fl = sum(l["flop"] for l in layers)
    lines.append(f"| **all 48** | {tot:.1f} | {fl / tot / 1e6:.1f} | |")
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


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    if sys.argv[1] == "stats":
        print(stats(sys.argv[2]))
    elif sys.argv[1] == "traffic":
        print(json.dumps(traffic(sys.argv[2], sys.argv[3], float(sys.argv[4])), indent=1))
    else:
        sys.exit(__doc__)
