"""The bench-only bandwidth probe behind bench.py's read floor (libembla_probe.so) reads every byte once: the
xor of its per-workgroup words equals the xor of every 32-bit word of the buffer, for any grid."""
import numpy as np
import pytest

from conftest import gpu_available
from gpu_util import dev, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,grid", [(16, 1), (4096, 7), (1 << 20, 64), (34078720, 1024), (1000016, 2048)])
@pytest.mark.parametrize("depth", [4, 16, 32])
@pytest.mark.parametrize("mode", [0, 2])
def test_stream_read_covers_every_word(nbytes, grid, depth, mode):
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    from embla_attn import ops
    say(f"stream read bytes={nbytes} grid={grid} depth={depth} mode={mode}")
    host = np.random.default_rng(nbytes).integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    sink = torch.zeros(grid, dtype=torch.int32, device="cuda")
    ops.stream_read(dev(host.view(np.uint8)), sink, grid, depth=depth, mode=mode)
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)
