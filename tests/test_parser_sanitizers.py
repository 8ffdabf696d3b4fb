"""The two safetensors / config.json readers under AddressSanitizer and UndefinedBehaviorSanitizer.

The engine's reader (csrc/checkpoint.cpp, the contract of cpu_inference.rs:58-96) and the
oracle's (oracle/oracle.c) are built for the host with g++ / gcc and fed mutated copies of a
valid checkpoint: truncated files, garbled header bytes, bogus header lengths, broken JSON and
config values. Any out-of-bounds access, use after free, leak or undefined behaviour aborts the
harness. Host code only: no GPU, no HIP compiler.
"""
import os
import shutil
import subprocess

import pytest

import qe
from conftest import TINY

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SAN = ["-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer"]
ITERS = "1000"


def _build(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        if "sanitize" in r.stderr or "asan" in r.stderr or "ubsan" in r.stderr:
            pytest.skip(f"sanitizer runtime unavailable: {r.stderr[-300:]}")
        raise AssertionError(r.stderr[-2000:])


def _run(cmd):
    env = dict(os.environ, ASAN_OPTIONS="abort_on_error=0:halt_on_error=1", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run(cmd, capture_output=True, text=True, env=env, timeout=300)
    report = r.stdout + r.stderr
    assert r.returncode == 0 and "runtime error" not in report and "Sanitizer" not in report, report[-4000:]
    return report


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_engine_reader_under_sanitizers(tmp_path):
    exe = str(tmp_path / "checkpoint_fuzz")
    _build(["g++", "-std=c++17", *SAN, os.path.join(HERE, "fuzz", "checkpoint_fuzz.cpp"),
            os.path.join(ROOT, "mac-gpu-compiler_amd", "csrc", "checkpoint.cpp"), "-o", exe])
    (tmp_path / "ck").mkdir()
    out = _run([exe, str(tmp_path / "ck"), ITERS])
    assert "accepted" in out


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_oracle_reader_under_sanitizers(tmp_path):
    exe = str(tmp_path / "oracle_fuzz")
    _build(["gcc", "-std=c11", *SAN, os.path.join(HERE, "fuzz", "oracle_fuzz.c"),
            os.path.join(ROOT, "oracle", "oracle.c"), "-o", exe, "-lm", "-lpthread"])
    (tmp_path / "ck").mkdir()
    d = str(tmp_path / "ck")
    qe.write_random_checkpoint(d, 1234, TINY)
    out = _run([exe, d, ITERS])
    assert "accepted" in out
