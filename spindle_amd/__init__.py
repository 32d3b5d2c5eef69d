"""spindle_amd: MI355X-native decode/verify hot path of WiseHax/spindle.

The compute runs in hand-written gfx950 HIP kernels behind the C ABI in include/spx.h
(libspx.so, built by spindle_amd/build.py). This package is the host-side mirror of the
reference's operator interface over that ABI; there is no CPU fallback: if the library is
missing or no GPU is visible, the entry points raise.
"""
from ._lib import LIB_PATH, SpxError, lib, load  # noqa: F401
