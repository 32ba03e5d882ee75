"""titania_amd: a gfx950 (MI355X) `hip` device for Titania's Qwen3 forward pass.

The compute path is libtitania_hip.so (hand-written HIP kernels behind the C ABI
of include/titania_hip.h); this package binds it for tests and benchmarks.
"""

from ._lib import (TH_KV_BF16, TH_KV_F32, TH_PATH_FUSED, TH_PATH_OPS, TH_PATH_TRAIT, HipError, InvalidArgument)
from .config import QWEN3_0_6B, QWEN3_4B, QWEN3_TINY, Config
from .device import Buffer, Hip, Tensor, Weight
from .sampler import Sampler

__all__ = [
    "Hip", "Tensor", "Weight", "Buffer", "Sampler", "Config", "QWEN3_0_6B", "QWEN3_4B", "QWEN3_TINY",
    "HipError", "InvalidArgument", "TH_KV_F32", "TH_KV_BF16", "TH_PATH_OPS", "TH_PATH_FUSED", "TH_PATH_TRAIT",
]
