"""Symmetric absmax INT8 with fp16 scales: the quantizer API of the INT8 caches, as torch ops.

Same contract as the reference's engine/quant.py:19-48: the scale is absmax / 127 rounded to fp16, the values are
quantized with that rounded scale (so dequantization uses exactly the stored scale), codes lie in [-127, 127],
an all-zero group gets scale 0 and codes 0. The fused HIP kernels (engine/hip_quant.py) produce the same bits;
the INT8 cache uses these torch ops only where the reference does too: CPU-resident caches and
fused_writes = False.
"""

import torch

QMAX = 127


def _scale(absmax: torch.Tensor) -> torch.Tensor:
    """fp16 scale of an absmax."""
    return (absmax.float() / QMAX).to(torch.float16)


def _quantize(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """round-half-even(x / scale) clamped to [-127, 127]; zero scales give zeros."""
    s = scale.float()
    nonzero = s > 0
    q = torch.where(nonzero, torch.round(x.float() / torch.where(nonzero, s, torch.ones_like(s))),
                    torch.zeros((), dtype=torch.float32, device=x.device))
    return q.clamp(-QMAX, QMAX).to(torch.int8)


def quantize_per_token(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """x [..., D] -> (int8 [..., D], fp16 [...]): one scale per vector over its last dimension."""
    scale = _scale(x.abs().amax(dim=-1))
    return _quantize(x, scale[..., None]), scale


def quantize_per_channel(x: torch.Tensor, dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """One scale per position of every dimension except `dim` (the tokens of a block)."""
    scale = _scale(x.abs().amax(dim=dim, keepdim=True))
    return _quantize(x, scale), scale.squeeze(dim)


def dequantize(q: torch.Tensor, scale: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """q * scale in `dtype`; scale must broadcast against q."""
    return (q.float() * scale.float()).to(dtype)
