"""stratum_amd: MI355X (gfx950) implementation of Stratum's NF4 frozen-weight path.

Public surface mirrors the reference's exports for this path
(``stratum/__init__.py:51-54`` and the module-level names of ``stratum/upload.py``
and ``stratum/nf4_linear.py``); the NF4 arithmetic runs in the HIP library
``libstratum_nf4.so`` (C ABI: ``include/stratum_nf4.h``).
"""

from .functional import (QuantState, dequantize_4bit, dequantize_4bit_many, get_4bit_type, nf4_gemm_bwd_dx,
                         nf4_gemm_fwd, nf4_grouped_gemm, quantize_4bit, quantize_4bit_many, stack_nf4)
from .nf4_linear import NF4Linear, NF4LoRALinear, nf4_linear
from .upload import (FP16_ATTR, NF4_ATTR, FP16StagedPayload, NF4Payload, NF4Prefetch, NF4Stats,
                     ensure_prefetched_weights, ensure_weights, estimate_module_upload_gib, free_weights,
                     prefetch_weights, prepare_fp16_staged, prepare_nf4, prepare_nf4_from_cache,
                     quantize_and_attach, restore_module_buffers, snapshot_module_buffers, upload_stream)

__all__ = [
    "QuantState", "dequantize_4bit", "dequantize_4bit_many", "get_4bit_type", "quantize_4bit",
    "quantize_4bit_many", "stack_nf4", "nf4_gemm_fwd", "nf4_gemm_bwd_dx", "nf4_grouped_gemm", "NF4Linear", "NF4LoRALinear", "nf4_linear", "FP16_ATTR", "NF4_ATTR",
    "FP16StagedPayload", "NF4Payload", "NF4Prefetch", "NF4Stats", "ensure_prefetched_weights", "ensure_weights",
    "estimate_module_upload_gib", "free_weights", "prefetch_weights", "prepare_fp16_staged", "prepare_nf4",
    "prepare_nf4_from_cache", "quantize_and_attach", "restore_module_buffers", "snapshot_module_buffers",
    "upload_stream",
]
