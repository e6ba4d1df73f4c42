"""The conv epilogue's division by 3 (the generator stage means, kk_conv.hip `div3`: one multiply
and two FMAs in place of a correctly rounded division) equals x / 3.0f for every finite float, and
its leaky ReLU max(x, slope x) equals x < 0 ? slope x : x for every float at the slopes used: an
exhaustive check of the same arithmetic in C with hardware FMA, on the CPU."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_div3_equals_division_for_every_finite_float(tmp_path):
    exe = str(tmp_path / "div3_check")
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
                    os.path.join(ROOT, "tests", "numerics", "div3_check.c"), "-o", exe, "-lm"],
                   check=True, capture_output=True, text=True, timeout=120)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1))))
    assert r.returncode == 0, r.stderr
    (n, bad), (ln, lbad) = [map(int, line.split()) for line in r.stdout.split("\n")[:2]]
    assert n == 2**32 - 2**24  # every bit pattern but the infinities and NaNs
    assert bad == 0
    assert ln == 5 * 2**32 and lbad == 0
