"""nanoinfer_amd — the MI355X (gfx950) quantized-weight matrix path.

libnq_hip.so holds the hand-written HIP kernels behind the C ABI declared in
include/nq.h; ``nanoinfer_amd.quant`` mirrors the reference's quant op interface
(cpp/src/quant.hpp) over it. Importing ``nanoinfer_amd.quant`` fails when the
library has not been built (``python -m nanoinfer_amd.build``).
"""
__all__ = ["build", "quant"]
