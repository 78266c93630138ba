"""Writers of the reference's NIT0 / NIT1 tensor files (serialize.hpp:1-23):
"NIT0" | int32 ndim | int32 shape | fp32 payload, and "NIT1" | int32 dtype
(0 fp32, 1 bf16) | int32 ndim | int32 shape | payload, little-endian."""
import numpy as np


def write_nit0(path, a):
    a = np.ascontiguousarray(a, np.float32)
    with open(path, "wb") as f:
        f.write(b"NIT0")
        f.write(np.int32(a.ndim).tobytes())
        f.write(np.asarray(a.shape, np.int32).tobytes())
        f.write(a.tobytes())


def write_nit1(path, a, dtype):
    """dtype 0: fp32 payload; 1: bf16 payload = the top 16 bits of each fp32
    (pass values that are exact in bf16 for a lossless round trip)."""
    a = np.ascontiguousarray(a, np.float32)
    with open(path, "wb") as f:
        f.write(b"NIT1")
        f.write(np.int32(dtype).tobytes())
        f.write(np.int32(a.ndim).tobytes())
        f.write(np.asarray(a.shape, np.int32).tobytes())
        if dtype == 1:
            f.write((a.view(np.uint32) >> 16).astype(np.uint16).tobytes())
        else:
            f.write(a.tobytes())


def bf16_exact(a):
    """Values of a truncated to bf16 (exactly representable in a bf16 payload)."""
    a = np.ascontiguousarray(a, np.float32)
    return (a.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
