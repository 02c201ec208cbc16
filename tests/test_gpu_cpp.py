"""Runs the reference-style C++ operator test (tests/cpp/test_asr_ops.cc) through the C++
drop-in header, with the reference's fixture files written from tests/golden."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "test_asr_ops"


def test_cpp_dropin_asr_ops(golden, tmp_path):
    assert BIN.exists(), "build() compiles tests/cpp/test_asr_ops"
    for name, arr in golden.items():
        ext = ".i32" if arr.dtype == np.int32 else ".f32"
        np.ascontiguousarray(arr).astype("<i4" if ext == ".i32" else "<f4").tofile(tmp_path / (name + ext))
    print("[gpu-case] C++ drop-in test", flush=True)
    proc = subprocess.run([str(BIN), str(tmp_path)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "PASSED" in proc.stdout


def test_cpp_dropin_asr_decoder():
    """tests/cpp/test_asr_decoder.cc: the reference decoder test's incremental-prefill and
    truncate checks plus graph-replayed vs eager greedy decoding, through the C++ class."""
    exe = BIN.parent / "test_asr_decoder"
    assert exe.exists(), "build() compiles tests/cpp/test_asr_decoder"
    print("[gpu-case] C++ drop-in decoder test", flush=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "PASSED" in proc.stdout
