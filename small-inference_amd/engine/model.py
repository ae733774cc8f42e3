"""A Qwen2-shaped decoder with random weights: the caller of the paged cache in the decode-step measurement.

It drives the cache exactly as the reference's model does (engine/model.py:124-175): per forward, cache.begin(T,
meta) once; per layer, cache.write(layer, k, v) and then cache.attend(layer, q, positions, scale), so a decode step
through it runs the HIP store and decode kernels the way the reference's ContinuousEngine would. The GEMMs are
torch (hipBLASLt on ROCm). Layer math (RMSNorm in fp32, rotary embedding with rotate-half, fused QKV with bias,
SwiGLU MLP, tied embeddings) follows the Qwen2 architecture the reference serves; weights are drawn from a seeded
normal distribution since no checkpoint is used.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .config import ModelConfig


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """x * rsqrt(mean(x^2) + eps) * weight, computed in fp32, returned in x's dtype."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * weight


class Rotary:
    """Rotary position embedding tables (theta = cfg.rope_theta) for the rotate-half convention."""

    def __init__(self, cfg: ModelConfig, device: torch.device, max_positions: int):
        d = cfg.head_dim
        inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float64, device=device) / d))
        ang = torch.arange(max_positions, dtype=torch.float64, device=device)[:, None] * inv[None, :]
        self.cos = torch.cat([ang.cos(), ang.cos()], -1).float()
        self.sin = torch.cat([-ang.sin(), ang.sin()], -1).float()  # sign of rotate-half folded in

    def rows(self, positions: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        """cos, signed sin [T, 1, d] for these positions."""
        return self.cos[positions][:, None].to(dtype), self.sin[positions][:, None].to(dtype)


def rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + swap_halves(x) * signed sin, for x [T, H, d]."""
    h = x.shape[-1] // 2
    return x * cos + torch.cat([x[..., h:], x[..., :h]], -1) * sin


@dataclass
class Layer:
    input_norm: torch.Tensor
    qkv_w: torch.Tensor
    qkv_b: torch.Tensor
    o_w: torch.Tensor
    post_norm: torch.Tensor
    gate_up_w: torch.Tensor
    down_w: torch.Tensor


class Qwen2Model:
    """Random-init decoder of cfg's shape in `dtype` on `device`."""

    def __init__(self, cfg: ModelConfig, device: str | torch.device = "cuda", dtype: torch.dtype = torch.bfloat16,
                 seed: int = 0, max_positions: int = 32768, std: float = 0.02):
        self.cfg, self.device, self.dtype = cfg, torch.device(device), dtype
        g = torch.Generator(device=self.device).manual_seed(seed)

        def rand(*shape):
            return (torch.randn(*shape, generator=g, device=self.device, dtype=torch.float32) * std).to(dtype)

        def ones(n):
            return torch.ones(n, device=self.device, dtype=dtype)

        H, qkv = cfg.hidden_size, cfg.q_size + 2 * cfg.kv_size
        self.embed = rand(cfg.vocab_size, H)
        self.layers = [Layer(ones(H), rand(qkv, H), rand(qkv), rand(H, cfg.q_size), ones(H),
                             rand(2 * cfg.intermediate_size, H), rand(H, cfg.intermediate_size))
                       for _ in range(cfg.num_layers)]
        self.final_norm = ones(H)
        self.lm_head = self.embed  # tied embeddings
        self.rotary = Rotary(cfg, self.device, max_positions)
        self.scale = cfg.head_dim ** -0.5

    def layer_forward(self, i: int, x: torch.Tensor, positions: torch.Tensor, cache, rot) -> torch.Tensor:
        """Decoder layer i on hidden states x [T, hidden]; K/V go through the cache."""
        cfg, w = self.cfg, self.layers[i]
        T, Hq, Hkv, d = x.shape[0], cfg.num_q_heads, cfg.num_kv_heads, cfg.head_dim
        qkv = F.linear(rms_norm(x, w.input_norm, cfg.rms_norm_eps), w.qkv_w, w.qkv_b)
        qk = rotate(qkv[:, :cfg.q_size + cfg.kv_size].view(T, Hq + Hkv, d), *rot)
        q, k = qk[:, :Hq], qk[:, Hq:]
        v = qkv[:, cfg.q_size + cfg.kv_size:].view(T, Hkv, d)
        cache.write(i, k, v)
        x = x + F.linear(cache.attend(i, q, positions, self.scale), w.o_w)
        gate, up = F.linear(rms_norm(x, w.post_norm, cfg.rms_norm_eps), w.gate_up_w).chunk(2, dim=-1)
        return x + F.linear(F.silu(gate) * up, w.down_w)

    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, cache, meta, last_only: bool = True):
        """Logits [num_seqs, vocab] (last token of each sequence; every token if not last_only) for a packed batch
        described by meta (positions must be meta.positions)."""
        cache.begin(input_ids.shape[0], meta)
        x = self.embed[input_ids]
        rot = self.rotary.rows(positions, x.dtype)
        for i in range(self.cfg.num_layers):
            x = self.layer_forward(i, x, positions, cache, rot)
        if last_only:
            x = x[meta.last_token_indices]
        return F.linear(rms_norm(x, self.final_norm, self.cfg.rms_norm_eps), self.lm_head)
