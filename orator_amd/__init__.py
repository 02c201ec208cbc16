"""MI355X (gfx950) attention hot path of Orator: HIP kernels behind a C ABI
(include/orator_attn.h) with the reference's operator names on the host side."""
from ._lib import GpuError, LIB_PATH  # noqa: F401
