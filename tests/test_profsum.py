"""The measurement helper that turns rocprofv3 CSV output into the bench's traffic figure."""
import csv
import os
import sys

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "kokoro-rust_amd"))

from kokoro_hip import profsum  # noqa: E402

COPY = "void at::native::vectorized_elementwise_kernel<4, at::native::AUnaryFunctor<float, float, float, " \
       "at::native::binary_internal::MulFunctor<float> >, std::array<char*, 2ul> >(int)"
FILL = "void at::native::vectorized_elementwise_kernel<4, at::native::FillFunctor<float>, std::array<char*, 1ul> >(int)"
SNAKE = "void kk::(anonymous namespace)::conv_mfma_kernel<4, 0, 2, 2, true, false, true>(kk::ConvParams)"


def _write(d, counter, rows):
    os.makedirs(d)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for i, (name, v) in enumerate(rows):
            w.writerow([i + 1, name, counter, v])


def test_snake_layers_bytes_and_flop():
    layers, frames = profsum.snake_layers()
    assert len(layers) == 48 and frames == 13501
    # fp16 streams throughout: conv1 moves 4 C bytes per column (stream in, fp16 h out), conv2 6 C
    # (h and the stream in, the stream out), the blocks' mean 10 C (three streams and h in, the
    # next layer's bf16 operand out)
    c0 = 20 * frames
    first = layers[0]
    assert first["bytes"] == 256 * c0 * 4 and first["flop"] == 2.0 * 256 * 256 * 7 * c0
    assert layers[1]["bytes"] == 256 * c0 * 6
    by = {l["name"]: l["bytes"] / (256 * c0) for l in layers if l["name"].startswith("stage0 resblock k3")}
    assert by == {"stage0 resblock k3 d1 conv1": 4, "stage0 resblock k3 d1 conv2": 6,
                  "stage0 resblock k3 d3 conv1": 4, "stage0 resblock k3 d3 conv2": 6,
                  "stage0 resblock k3 d5 conv1": 4, "stage0 resblock k3 d5 conv2": 6}
    means = [l for l in layers if l["name"].endswith("resblock k11 d5 conv2")]
    assert len(means) == 2 and means[0]["bytes"] == 256 * c0 * 10


def test_traffic_scales_by_the_copy_kernel(tmp_path):
    # the copy kernel reads 1 MiB but FETCH_SIZE shows half: every conv dispatch scales by 2;
    # the fill kernel (no reads) must not take part in the calibration
    snake_kib = [1000.0 + i for i in range(48)]
    _write(str(tmp_path / "f"), "FETCH_SIZE", [(FILL, 3.0), (COPY, 512.0)] + [(SNAKE, v) for v in snake_kib])
    _write(str(tmp_path / "w"), "WRITE_SIZE", [(FILL, 1024.0), (COPY, 1024.0)] + [(SNAKE, 500.0)] * 48)
    r = profsum.traffic(str(tmp_path / "f"), str(tmp_path / "w"), 1)
    mean_kib = sum(snake_kib) / 48
    assert abs(r["fetch"]["scale"] - 2.0) < 1e-9 and abs(r["write"]["scale"] - 1.0) < 1e-9
    assert abs(r["fetch"]["bytes_per_launch"] - mean_kib * 1024 * 2) < 1e-6
    assert abs(r["traffic_bytes_per_launch"] - (mean_kib * 2 + 500.0) * 1024) < 1e-6


def test_counters_mfma_utilisation(tmp_path):
    """MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs), the clock
    GRBM_GUI_ACTIVE / XCDs / duration; counters split over several rows of a dispatch are summed."""
    d = tmp_path / "pmc"
    os.makedirs(d)
    with open(d / "run_agent_info.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Agent_Type", "Simd_Count", "Num_Xcc"])
        w.writerow(["CPU", "0", "0"])
        w.writerow(["GPU", "1024", "8"])
    other = "void kk::(anonymous namespace)::conv_mfma_kernel<2, 0, 1, 2, false, false, false, 16, 1>(kk::ConvParams)"
    rows = []
    # a Snake conv of 1 ms at 2 GHz (2e6 cycles per SIMD): half its SIMD cycles busy with MFMAs
    gui = 2e6 * 8
    busy = 0.5 * 2e6 * 1024
    for name, k in ((SNAKE, 1), (other, 2)):
        rows += [(k, name, "GRBM_GUI_ACTIVE", gui / 2), (k, name, "GRBM_GUI_ACTIVE", gui / 2),
                 (k, name, "SQ_VALU_MFMA_BUSY_CYCLES", busy / (1 if name == SNAKE else 4)),
                 (k, name, "SQ_INSTS_MFMA", busy / 32 / (1 if name == SNAKE else 4))]
    with open(d / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp",
                    "End_Timestamp"])
        for k, name, c, v in rows:
            w.writerow([k, name, c, v, 0, 1_000_000])
    _, tot = profsum.counters(str(d))
    sn = tot["Snake-block convs"]
    assert abs(sn["util"] - 0.5) < 1e-12 and abs(sn["clock_ghz"] - 2.0) < 1e-12
    assert abs(tot["other convs (decoder, ConvT, conv_post)"]["util"] - 0.125) < 1e-12
    assert abs(tot["all convs"]["util"] - 0.3125) < 1e-12


def test_serial_pass_is_the_last_runs(tmp_path):
    """The serial table covers only the `steps` runs before the trace's last `trailing` runs (each
    run ends with the iSTFT); earlier, overlapped runs and the trailing runs stay out of it."""
    d = tmp_path / "trace"
    os.makedirs(d)
    ist = "void kk::(anonymous namespace)::istft_kernel(float const*, float*)"
    fin = "void kk::(anonymous namespace)::finalize_kernel<16, 1>(kk::StatPart const*)"
    # three runs: [fin 100 us, istft 10 us] each; the first two overlapped (long finalize)
    seq = [(fin, 100), (ist, 10), (fin, 100), (ist, 10), (fin, 7), (ist, 10)]
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        t = 0
        for name, us in seq:
            w.writerow([name, t, t + us * 1000])
            t += us * 1000 + 1000
    out = profsum.serial(str(d), 1)
    assert "(2 dispatches of the 1 runs," in out
    assert "| `finalize_kernel` | 1 | 0.01 | 7.0 |" in out
    assert "| `istft_kernel` | 1 | 0.01 | 10.0 |" in out
    assert profsum.serial(str(d), 3) == ""
    # one trailing run after the profiling pass (bench.py's parity plan): the window is the run before it
    out = profsum.serial(str(d), 1, 1)
    assert "(2 dispatches of the 1 runs before the trace's last 1," in out
    assert "| `finalize_kernel` | 1 | 0.10 | 100.0 |" in out and "7.0 |" not in out
    assert profsum.serial(str(d), 2, 1) == ""
