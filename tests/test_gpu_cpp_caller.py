"""The drop-in C++ headers (include/fns/ggml_kernels.h, include/fns/kernels.h) called exactly as the reference engine
calls them - Engine::ffn_block at 1 and 2 columns (reference src/engine.cu:655-696) and Engine::prefill_chunk's FFN
(src/engine.cu:330-357) - from a hipcc-compiled C++ program (tests/cpp/engine_caller.cpp, built by build()), every
stage checked against the CPU oracle inside that program. Also covers the Q8_0 output head (150144 rows)."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "engine_caller"


def test_engine_caller_cpp():
    assert BIN.exists(), "tests/cpp/engine_caller is not built: run __graft_entry__.build() first"
    env = dict(os.environ, OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "8"))
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=110, env=env)
    print(r.stdout[-4000:])
    assert r.returncode == 0 and "ENGINE_CALLER_OK" in r.stdout, r.stdout[-4000:] + r.stderr[-2000:]
