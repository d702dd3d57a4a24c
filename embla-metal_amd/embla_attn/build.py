"""Builds libembla_attn.so (gfx950) in-tree with hipcc: one object a source file, then a link.

Run as ``python -m embla_attn.build`` from ``embla-metal_amd/`` or call :func:`build`.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parent.parent / "include"
LIB = PKG / "libembla_attn.so"
HOST = PKG.parent / "host"
HOST_LIB = PKG / "libembla_host.so"
PROBE = PKG.parent / "probe"
PROBE_LIB = PKG / "libembla_probe.so"
OBJ = PKG.parent / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 instructions stay off (they have given silent wrong results on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs: the AGPR form costs a v_accvgpr_read per result the VALU then
    # uses (C2 step 9.05 -> 8.78 us; neutral on the other configs)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-result", f"-I{INCLUDE}", f"-I{CSRC}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = OBJ / (src.name + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    build_host()
    build_probe()
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources, {HOST_LIB.name} and {PROBE_LIB.name}")
    return LIB


def build_host() -> Path:
    """The C++ host side over the C ABI (host/*.cpp: the attention engine) as libembla_host.so,
    linked to libembla_attn.so beside it."""
    tmp = HOST_LIB.with_suffix(".so.tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-I{INCLUDE}", f"-I{HOST}",
           *map(str, sorted(HOST.glob("*.cpp"))), f"-L{PKG}", "-lembla_attn", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host library build failed:\n{r.stderr}")
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build_probe() -> Path:
    """The bench-only bandwidth probe (probe/*.hip) as its own libembla_probe.so: bench.py's read
    floor uses it; the attention library does not contain it."""
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-shared", "-x", "hip", *map(str, sorted(PROBE.glob("*.hip"))), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"probe library build failed:\n{r.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
