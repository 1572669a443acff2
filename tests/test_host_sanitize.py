"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU).

tests/host_sanitize.cpp is built with g++ together with the host sources it exercises (the GGUF catalogue
parser, satori_amd/csrc/gguf.cpp, and the payload validation / quantizer / bitplane entry points,
satori_amd/csrc/host_cpu.cpp) and run over the reference's golden GGUF files and containers built the way
test_gguf.py builds them (every scalar and array type at alignments 8 and 64; Q4_K and Q6_K tensors with
their quantization version): the seeds, every truncation and single-byte and 64-bit mutations of their
first 1,024 bytes. Any sanitizer report, or a parse that publishes a window outside the file, fails the run.
"""
from __future__ import annotations

import os
import shutil
import struct
import subprocess

import pytest

from helpers import GOLDEN
from test_gguf import _value, container, gguf_string

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _seeds(directory) -> list[str]:
    paths = [os.path.join(GOLDEN, n) for n in sorted(os.listdir(GOLDEN)) if n.endswith(".gguf")]
    meta = b"".join(gguf_string(f"custom.value_{t}") + struct.pack("<I", t) + _value(t) for t in range(13))
    meta += gguf_string("custom.empty") + struct.pack("<IIQ", 9, 8, 0)
    meta += gguf_string("custom.strings") + struct.pack("<IIQ", 9, 8, 2) + gguf_string("è\0漢") + gguf_string("")
    built = {}
    for alignment in (8, 64):
        prefix = container(alignment, meta, 15)
        built[f"mixed-{alignment}.gguf"] = prefix + bytes(alignment * 2 + 3)
    version = gguf_string("general.quantization_version") + struct.pack("<II", 4, 2)
    prefix = container(32, version, 1, [("q4k", [256, 2], 12, 0), ("q6k", [256, 1], 14, 288)])
    built["k-types.gguf"] = prefix + bytes(512)
    for name, data in built.items():
        path = os.path.join(directory, name)
        with open(path, "wb") as f:
            f.write(data)
        paths.append(path)
    return paths


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ builds the sanitizer harness")
def test_host_code_under_address_and_undefined_behaviour_sanitizers(tmp_path):
    exe = str(tmp_path / "host_sanitize")
    sources = [os.path.join(ROOT, "tests", "host_sanitize.cpp"),
               os.path.join(ROOT, "satori_amd", "csrc", "gguf.cpp"),
               os.path.join(ROOT, "satori_amd", "csrc", "host_cpu.cpp")]
    build = subprocess.run(
        ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=all", "-static-libasan", "-static-libubsan", *sources, "-o", exe],
        capture_output=True, text=True, timeout=600)
    assert build.returncode == 0, build.stderr[-4000:]
    work = tmp_path / "work"
    work.mkdir()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    run = subprocess.run([exe, str(work), *_seeds(str(tmp_path))], capture_output=True, text=True, timeout=900,
                         env=env)
    assert run.returncode == 0, run.stdout[-2000:] + run.stderr[-6000:]
    assert run.stdout.rstrip().endswith("ok"), run.stdout[-2000:]
    assert "runtime error" not in run.stderr and "AddressSanitizer" not in run.stderr, run.stderr[-6000:]
