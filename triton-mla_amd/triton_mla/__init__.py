"""triton_mla: weight-absorbed MLA decode for MI355X (gfx950), HIP kernels.

Drop-in for the reference package's public API (src/triton_mla/__init__.py:1-14).
"""

from .fp8 import dequantize_kv_fp8, quantize_kv_fp8
from .kernel import get_num_splits, mla_decode
from .model import MLA, MLAConfig
from .reference import mla_decode_ref, mla_decode_torch

__version__ = "0.1.1"

__all__ = [
    "MLA",
    "MLAConfig",
    "dequantize_kv_fp8",
    "get_num_splits",
    "mla_decode",
    "mla_decode_ref",
    "mla_decode_torch",
    "quantize_kv_fp8",
]
