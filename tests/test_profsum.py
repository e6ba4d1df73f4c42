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
    # conv1 moves 6 C bytes per column, conv2 10 C, the blocks' mean 16 C (three f32 residual
    # streams, the fp16 input, the next layer's bf16 operand out)
    c0 = 20 * frames
    first = layers[0]
    assert first["bytes"] == 256 * c0 * 6 and first["flop"] == 2.0 * 256 * 256 * 7 * c0
    means = [l for l in layers if l["name"].endswith("resblock k11 d5 conv2")]
    assert len(means) == 2 and means[0]["bytes"] == 256 * c0 * 16


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
