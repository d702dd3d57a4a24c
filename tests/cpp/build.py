"""Builds the C++ engine test (test_attention_engine.cpp) beside this file: the oracle's C source
compiled as the checker, linked with libembla_host.so and libembla_attn.so (found at run time from
the binary's location). Called by __graft_entry__.build(); the GPU test only runs the binary."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
PKG = ROOT / "embla-metal_amd" / "embla_attn"
BIN = HERE / "test_attention_engine"


def build() -> Path:
    obj = HERE / "_build"
    obj.mkdir(exist_ok=True)
    orc_o = obj / "oracle.o"
    r = subprocess.run(["gcc", "-O2", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-c",
                        str(ROOT / "oracle" / "oracle.c"), "-o", str(orc_o)], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle compile failed:\n{r.stderr}")
    test_o = obj / "test_attention_engine.o"
    hipcc = "/opt/rocm/bin/hipcc"
    cmd = [hipcc, "--offload-arch=gfx950", "-O2", "-std=c++17", "-Wno-unused-result",
           f"-I{ROOT / 'include'}", f"-I{ROOT / 'embla-metal_amd' / 'host'}", f"-I{ROOT / 'embla-metal_amd' / 'csrc'}",
           "-c", str(HERE / "test_attention_engine.cpp"), "-o", str(test_o)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"engine test compile failed:\n{r.stderr}")
    tmp = BIN.with_suffix(".tmp")
    cmd = [hipcc, "--offload-arch=gfx950", str(test_o), str(orc_o), f"-L{PKG}", "-lembla_host", "-lembla_attn",
           "-Wl,-rpath,$ORIGIN/../../embla-metal_amd/embla_attn", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"engine test link failed:\n{r.stderr}")
    tmp.replace(BIN)
    return BIN


if __name__ == "__main__":
    print(build())
