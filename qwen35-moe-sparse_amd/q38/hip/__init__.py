"""HIP (gfx950) kernels of the Q38 MoE prefill path, reached through libq38moe.so's C ABI."""
from . import ops  # noqa: F401
from ._lib import LIB_PATH, lib  # noqa: F401
