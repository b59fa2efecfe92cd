"""REXL3's token-sampling hot path on MI355X (gfx950): the keyed sampler of crates/sampling, the accept steps of
crates/spec, and the extended pipeline, as hand-written HIP kernels behind the C ABI of include/gbs_sample.h."""
from . import _lib  # noqa: F401

__all__ = ["sampling"]
