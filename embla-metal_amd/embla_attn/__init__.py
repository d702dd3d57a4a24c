"""embla_attn — MI355X (gfx950) attention hot path of embla-metal behind a C ABI.

`_lib` binds libembla_attn.so; `ops` wraps it for torch device tensors; `layout` packs host rows
into the device cache layouts; `synth` draws the configurations' seeded inputs.
"""
from ._lib import BF16, F16, F32, RELU2_SINK, SOFTMAX, EmblaError, lib  # noqa: F401

__all__ = ["lib", "EmblaError", "F16", "BF16", "F32", "SOFTMAX", "RELU2_SINK"]
