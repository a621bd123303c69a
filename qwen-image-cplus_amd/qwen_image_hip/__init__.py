"""qwen_image_hip: MI355X (gfx950) QIPACK INT4 linear backend.

A drop-in for the reference engine's INT4 linear path
(netdur/qwen-image-cplus, qwen_image_cuda/cuda/gemm.cu and its caller
qwen_image_cuda/src/transformer.cplus:669-713).  The compute lives in
libqwen_image_hip.so (hand-written HIP for gfx950); this package is the
host-side mirror of the reference's linear-op interface.
"""
from ._lib import ABI_VERSION, LIB_PATH, QiHipError, load  # noqa: F401
from . import ops  # noqa: F401
from .linear import (SCHEME_W4A16, SCHEME_W4A4_H256, W4A4_FP6, W4A4_INT8, PackedLinear, Work,  # noqa: F401
                     linear)
from . import qipack  # noqa: F401
from .stream import BlockStream  # noqa: F401
