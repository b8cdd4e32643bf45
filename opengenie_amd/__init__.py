"""opengenie_amd: MI355X-native (gfx950) fused LTX-2.3 DiT block ops.

`opengenie_amd.ltx_ops` is the drop-in for plugyawn/opengenie's
`ltx_serve/triton_ltx_ops.py` fused-op API; the kernels live in
libopengenie_amd.so (C ABI: include/opengenie_amd.h), built by
`python -m opengenie_amd.build`.
"""

from . import ltx_ops  # noqa: F401
from ._lib import LIB_PATH, LibraryMissing, available  # noqa: F401

__version__ = "0.1.0"
