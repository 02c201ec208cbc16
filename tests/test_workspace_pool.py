"""CPU test of the library's workspace bookkeeping (orator_amd/csrc/workspace_pool.hpp), built
with AddressSanitizer: blocks grow geometrically (1000 creeping requests retire a handful); a
grown block is freed once the work queued before its retirement completes, never earlier, and
never while a captured graph may replay over it; each host thread has its own block per stream
(as the reference's thread_local scratch, src/model/asr_gemm.cu:23-43) and gives it back when
it exits; releasing a stream frees exactly its blocks."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "cpp" / "test_workspace_pool.cc"


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_workspace_pool_host_logic(tmp_path):
    exe = tmp_path / "test_workspace_pool"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-pthread",
                    "-fsanitize=address,undefined", str(SRC), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    assert "workspace pool OK" in out.stdout
