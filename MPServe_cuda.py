"""Drop-in ``import MPServe_cuda`` for the MI355X build: the reference's module
name (reference kernel/wrapper.cpp:132, setup.py:18) over mpserve_amd's HIP ops."""
from mpserve_amd.mpserve_cuda import *  # noqa: F401,F403
from mpserve_amd.mpserve_cuda import (  # noqa: F401
    SIDECAR_KEYS, cuda_clock_rate_khz, huffman_build_fp8_decode_tables, huffman_decode_fp8,
)
from mpserve_amd import mpserve_cuda as _impl

for _n in dir(_impl):
    if not _n.startswith("_") and _n not in globals():
        globals()[_n] = getattr(_impl, _n)
