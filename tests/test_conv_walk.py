"""CPU check of the MFMA conv kernel's walk over units, slabs and taps (kokoro-rust_amd/csrc/kk_walk.h,
the functions conv_mfma_kernel runs): tests/conv_walk_check.hip simulates every block of 6,048
launch shapes (tile counts, M-blocks, taps, slabs, CU counts) on the host and counts out-of-range
weight-fragment loads, units run twice or never, and producer / consumer disagreements; and the
ConvT epilogue's column mapping (convt_cols) against the per-column rule on 200,000 random unit
geometries.  A planted mistake in the next-tap rule must be caught.  Any change to the kernel's prefetch or unit walk is
checked here, on the CPU, before it runs on a GPU."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_conv_walk_bounds_and_coverage(tmp_path):
    exe = tmp_path / "conv_walk_check"
    cmd = [os.environ.get("HIPCC", "/opt/rocm/bin/hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17",
           "-I", os.path.join(ROOT, "kokoro-rust_amd", "csrc"), os.path.join(ROOT, "tests", "conv_walk_check.hip"),
           "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=300).stdout
    assert "convt columns violations 0" in out.splitlines(), out[:2000]
    assert out.strip().splitlines()[-1] == "launches 6048 violations 0", out[-2000:]
    planted = subprocess.run([str(exe), "--plant"], check=True, capture_output=True, text=True, timeout=300).stdout
    assert int(planted.strip().split()[-1]) > 0
