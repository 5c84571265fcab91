"""axs -- MI355X (gfx950) implementation of the AXS-6 NF5 hot path.

The package mirrors the reference's ``axs.unified`` API (see
``axs.unified``) on top of libaxs6.so, a C-ABI library of hand-written HIP
kernels built by ``python axs-6_amd/build.py``.
"""
from axs.core import (  # noqa: F401
    AXS6_EXPONENT_BIAS,
    AXS6_MAX_MAGNITUDE,
    DEFAULT_BLOCK_SIZE,
    VALID_BLOCK_SIZES,
    AXSTensor,
)

__version__ = "0.1.0"
