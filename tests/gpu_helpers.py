"""Small helpers for the GPU parity tests (upload / download through the C ABI)."""
from __future__ import annotations

import sys

import numpy as np

from orator_amd.runtime import DeviceBuffer, synchronize


def up(arr) -> DeviceBuffer:
    return DeviceBuffer.from_array(np.ascontiguousarray(arr))


def empty(shape, dtype) -> DeviceBuffer:
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    return DeviceBuffer(n)


def down(buf: DeviceBuffer, shape, dtype=np.float32) -> np.ndarray:
    synchronize()
    return buf.download(dtype, shape)


def say(*msg) -> None:
    """Names the case before a GPU step, flushed, so a fault can be attributed."""
    print("[gpu-case]", *msg, flush=True)
    sys.stdout.flush()
