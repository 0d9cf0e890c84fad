"""MI355X-native GQA streaming-attention engine with the LARA KV260 driver API.

``lara_amd.attn_driver`` is the drop-in for the board driver ``sw/attn_driver.py``;
``libgqa.so`` (built by ``lara_amd.build``) holds the HIP kernels behind the C ABI
declared in ``include/gqa.h``.
"""
from .attn_driver import AttentionAccelerator, RunProfile, TensorByteCounts, bf16_u16_to_fp32, fp32_to_bf16_u16

__all__ = ["AttentionAccelerator", "RunProfile", "TensorByteCounts", "bf16_u16_to_fp32", "fp32_to_bf16_u16"]
