"""The CPU-side C code under AddressSanitizer and UBSan (host builds only, tests/sanitize/Makefile): the oracle on every
entry point and weight type, and the GGUF reader on well-formed and 300 corrupted files (truncations and byte flips,
as tests/test_gguf.py makes them).  A sanitizer report aborts the driver, which fails the test."""
import os
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tests.gguf_writer import write_gguf
from tests.test_gguf import KV, _expert_tensors, _layer, _model

SAN = Path(__file__).resolve().parent / "sanitize"


@pytest.fixture(scope="module")
def built():
    if not shutil.which("gcc") or not shutil.which("g++") or not shutil.which("make"):
        pytest.skip("gcc, g++ or make missing")
    r = subprocess.run(["make", "-s", "-C", str(SAN)], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr
    return SAN


def _run(exe, args, tmp_path):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1", OMP_NUM_THREADS="2")
    r = subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True, timeout=600, env=env, cwd=tmp_path)
    assert r.returncode == 0 and "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stdout + r.stderr[-4000:]
    return r.stdout


def test_oracle_under_asan_ubsan(built, tmp_path):
    assert "oracle_san: done" in _run(built / "oracle_san", [], tmp_path)


def test_gguf_reader_under_asan_ubsan(built, tmp_path):
    L = _layer()
    good, _, _ = _model(tmp_path, L)
    split = []
    for i in range(2):   # a two-shard split model
        p = tmp_path / f"s-{i + 1:05d}-of-00002.gguf"
        kv = KV + [("split.count", 4, 2)] if i == 0 else [("general.architecture", 8, "qwen3moe")]
        write_gguf(p, kv, _expert_tensors(L) if i == 1 else [], alignment=64)
        split.append(p)
    raw = bytearray(good.read_bytes())
    rng = np.random.default_rng(12)
    files = [good, split[0]]
    for i in range(300):
        b = bytearray(raw)
        if i % 3 == 0:
            b = b[: int(rng.integers(1, len(b)))]
        else:
            for _ in range(int(rng.integers(1, 4))):
                pos = int(rng.integers(0, min(len(b), 2048)))
                b[pos] = int(rng.integers(0, 256))
        p = tmp_path / f"bad{i}.gguf"
        p.write_bytes(bytes(b))
        files.append(p)
    out = _run(built / "gguf_san", files, tmp_path)
    assert out.startswith("gguf_san: ") and int(out.split()[1]) >= 2
