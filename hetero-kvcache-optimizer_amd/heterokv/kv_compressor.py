"""KVCompressor: group-wise asymmetric INT4 quantizer on the GPU.

Drop-in for src/quantization/kv_compressor.py:24-171 of the reference: the same
constructor, the same compress / decompress / mse_error / relative_error /
compression_ratio methods, the same outputs (codes uint8 in the input's shape,
1-D float32 scales, 1-D uint8 zero points), bit for bit.  The arithmetic runs in
the HIP kernels hkv_quantize_groups / hkv_dequantize_groups; tensors must live
on a ROCm GPU (there is no CPU path).
"""
from typing import Tuple

import torch

from . import ops


class KVCompressor:
    """4-bit group-wise asymmetric quantizer (kv_compressor.py:24-44).

    scale = max((max - min) / 15, 1e-8); zp = clamp(round(-min / scale), 0, 15);
    q = clamp(round(x / scale + zp), 0, 15); x' = (q - zp) * scale.
    """

    def __init__(self, group_size: int = 128, bits: int = 4):
        assert bits == 4, "Current implementation only supports 4-bit quantization"
        self.group_size = group_size
        self.bits = bits
        self.qmax = (1 << bits) - 1
        self.qmin = 0

    def compress(self, tensor: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """kv_compressor.py:50-98: (codes uint8 same shape, scales f32 [G], zps u8 [G])."""
        return ops.quantize_groups(tensor, self.group_size)

    def decompress(self, quantized: torch.Tensor, scales: torch.Tensor, zero_points: torch.Tensor,
                   target_dtype: torch.dtype = torch.float16) -> torch.Tensor:
        """kv_compressor.py:100-132."""
        return ops.dequantize_groups(quantized, scales, zero_points, self.group_size, target_dtype)

    def mse_error(self, original, quantized, scales, zero_points) -> float:
        """kv_compressor.py:138-144."""
        restored = self.decompress(quantized, scales, zero_points, target_dtype=original.dtype)
        return torch.nn.functional.mse_loss(restored.float(), original.float()).item()

    def relative_error(self, original, quantized, scales, zero_points) -> float:
        """kv_compressor.py:146-154: mean|x' - x| / (mean|x| + 1e-8) * 100."""
        restored = self.decompress(quantized, scales, zero_points, target_dtype=original.dtype)
        orig_f = original.float()
        rel = (restored.float() - orig_f).abs().mean() / (orig_f.abs().mean() + 1e-8)
        return rel.item() * 100.0

    def compression_ratio(self, tensor: torch.Tensor) -> float:
        """kv_compressor.py:160-171 (INT4 packed + fp32 scale + u8 zp per group vs fp16)."""
        n = tensor.numel()
        num_groups = (n + self.group_size - 1) // self.group_size
        return 1.0 - (n * 4 + num_groups * (32 + 8)) / (n * 16)
