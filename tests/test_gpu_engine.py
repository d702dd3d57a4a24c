"""The C++ host side (embla-metal_amd/host: Engine.encodeAttention and Prefill.encode mirrored over
the C ABI): a three-layer decode stack checked stage by stage against the C oracle, and prefill
against token-by-token decode, with the full layers' caches in int8 and then in bf16 (the
reference's EMBLA_KV8=0), by tests/cpp's test binary."""
import subprocess
from pathlib import Path

import pytest

from conftest import gpu_available
from gpu_util import say

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "test_attention_engine"


def test_attention_engine_stack():
    if not gpu_available():
        pytest.skip("no GPU")
    assert BIN.exists(), f"{BIN} is not built: run __graft_entry__.build()"
    say("C++ attention engine: sliding, full (scores + selection), sparse layers, positions 0 .. 1400")
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=110)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert " 0 failed" in r.stdout
