"""r4dx_amd -- MI355X (gfx950) build of r4dx's quantized-weight matrix-product path.

The product is the C-ABI library libr4d_mi355x.so (declared in include/r4d_mi355x.h).  This package
loads it and exposes thin Python mirrors of its entry points (r4dx_amd.api) that take torch device
tensors.  There is no fallback: if the library is missing, every call raises."""
from .loader import lib, LIB_PATH  # noqa: F401
