"""ftmoe -- FreeToken-Intel's fused quantized MoE expert layer, rebuilt for
AMD Instinct MI355X (gfx950): hand-written HIP kernels behind a C ABI
(include/ftmoe.h), with the reference's Python host API on top."""
from . import _native  # noqa: F401
from .banks import Proj, proj_from_bank, single_proj  # noqa: F401
from .layer import MoeLayer  # noqa: F401

__version__ = "0.1.0"
