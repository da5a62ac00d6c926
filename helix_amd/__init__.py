"""helix_amd: MI355X-native HELIX chunked SSD (Mamba-2) prefill scan.

The product is the C-ABI library helix_amd/csrc/libhelix.so (include/helix/helix.h)
with its embedded gfx950 code object. This package is the Python host mirror of
that ABI: ctypes bindings (helix_amd.abi) and a torch-facing operator
(helix_amd.scan). Importing the package loads nothing; the library is opened on
first use and a missing library raises instead of falling back.
"""
from .desc import (HELIX_ABI_VERSION, HelixScanDesc, HelixTensor, desc_init,  # noqa: F401
                   algorithmic_bytes, algorithmic_flops)
