"""agens-engine_amd: the mixed-bit (W2/W3/W4) group-quantized GEMV path of Agens Engine on MI355X (gfx950).

The product is the C-ABI library libagens_kernels.so (declarations in include/agens_kernels.h), built in-tree by
build.py; this module only locates and loads it.  There is no fallback: a missing library is an error.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libagens_kernels.so")


def load():
    """ctypes handle of libagens_kernels.so; raises if it has not been built."""
    if not os.path.exists(LIBRARY):
        raise RuntimeError(f"{LIBRARY} is missing: build it with `python agens-engine_amd/build.py`")
    return ctypes.CDLL(LIBRARY)
