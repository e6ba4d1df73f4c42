"""The host code under AddressSanitizer + UndefinedBehaviorSanitizer, on the CPU.

- The library's host-only sources (the torch.save reader kk_ckpt.hip, which replaces the
  reference's memory-safe Rust reader src/torchpt.rs:311-335, and kk_host.cpp: the layout tables,
  the duration rule, the ids-level item checks) built with g++ -fsanitize=address,undefined into
  tests/sanitize/host_fuzz.cpp, which mutates a seeded corpus of torch.save archives (a model file
  with views, offsets, shared storages, scalars and empty tensors; a voice pack) and checks every
  mutant is read or refused with an error, then drives the host rules with random and adversarial
  arguments.  The first sanitizer report ends the run with a non-zero status.
- The oracle (oracle/kk_oracle.c) built the same way and its own CPU tests run against that build
  (LD_PRELOAD of the sanitizer runtimes into a child Python).
"""
import collections
import os
import subprocess
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kokoro-rust_amd", "csrc")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def _corpus(d):
    g = torch.Generator().manual_seed(5)
    base = torch.randn(6, 10, generator=g)
    sd = collections.OrderedDict()
    sd["module.conv.weight_g"] = torch.rand(4, 1, 1, generator=g)
    sd["module.conv.weight_v"] = torch.randn(4, 3, 5, generator=g)
    sd["module.lin.weight"] = torch.randn(6, 4, generator=g).t()
    sd["module.slice"] = base[2:5, 1:8]
    sd["module.shared"] = base[1]
    sd["module.scalar"] = torch.tensor(3.5)
    sd["module.empty"] = torch.zeros(0, 3)
    model = os.path.join(d, "model.pth")
    torch.save({"decoder": sd, "bert": collections.OrderedDict(x=torch.arange(5, dtype=torch.float32))}, model)
    voice = os.path.join(d, "voice.pt")
    torch.save(torch.randn(7, 1, 256, generator=g), voice)
    return [model, voice]


def test_host_code_fuzzed_under_sanitizers(tmp_path):
    exe = str(tmp_path / "host_fuzz")
    cmd = ["g++", "-std=c++17", *SAN, "-I", CSRC, "-I", os.path.join(ROOT, "include"), "-x", "c++",
           os.path.join(CSRC, "kk_ckpt.hip"), os.path.join(CSRC, "kk_host.cpp"),
           os.path.join(ROOT, "tests", "sanitize", "host_fuzz.cpp"), "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=300)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:allocator_may_return_null=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([exe, "2500", *_corpus(str(tmp_path))], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
    last = r.stdout.strip().splitlines()[-1]
    print(last)
    words = last.split()
    mutants, read, refused = int(words[1]), int(words[3]), int(words[5])
    assert mutants == 2 * 2501 and read + refused == 2 * mutants
    assert read > 0 and refused > mutants // 2  # most mutants are refused, the seeds themselves read
    assert "other 0" in last and int(words[-2]) > 10000


def test_oracle_tests_under_sanitizers(tmp_path):
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if not asan or not ubsan:
        pytest.skip("gcc's sanitizer runtimes are not installed")
    lib = str(tmp_path / "libkk_oracle_san.so")
    cmd = ["gcc", "-std=gnu11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-fno-math-errno",
           "-march=x86-64-v3", *SAN, os.path.join(ROOT, "oracle", "kk_oracle.c"), "-o", lib, "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True, timeout=300)
    env = dict(os.environ, KK_ORACLE_LIB=lib, LD_PRELOAD=f"{asan}:{ubsan}",
               ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1", OMP_NUM_THREADS="4")
    r = subprocess.run([sys.executable, "-m", "pytest", "-x", "-q", "-p", "no:cacheprovider",
                        os.path.join(ROOT, "tests", "test_oracle.py"), os.path.join(ROOT, "tests", "test_golden.py")],
                       capture_output=True, text=True, timeout=900, env=env, cwd=ROOT)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr
    print(r.stdout.strip().splitlines()[-1])
