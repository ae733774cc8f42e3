"""Causal GQA attention over one sequence's gathered K/V: the cache's gather backend (and, on the HIP backend, the
rows of shapes the paged kernels do not cover).

Same contract as the reference's attention() (engine/attention.py:6-28): q [T, Hq, d]; k, v [Hkv, S, d];
query t sees key s iff k_pos[s] <= q_pos[t]; query head h uses KV head h // g; the g heads of a group are stacked
along M so each KV head is read once; softmax in at least fp32; returns [T, Hq * d]. Decode rows (one new token
per sequence) and prefill chunks do not come here on the HIP backend: they go to the paged decode and prefill
kernels.
"""

import torch


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_pos: torch.Tensor, k_pos: torch.Tensor,
              scale: float) -> torch.Tensor:
    """Causal GQA attention for one sequence; see the module docstring."""
    T, Hq, d = q.shape
    Hkv = k.shape[0]
    g = Hq // Hkv
    qg = q.reshape(T, Hkv, g, d).permute(1, 2, 0, 3).reshape(Hkv, g * T, d)
    scores = torch.bmm(qg, k.transpose(1, 2).contiguous()) * scale  # [Hkv, g*T, S]
    if T > 1:  # one query is always the newest token and sees every key
        hidden = k_pos[None, :] > q_pos[:, None]  # [T, S]
        scores = scores.view(Hkv, g, T, -1).masked_fill(hidden, float("-inf")).view(Hkv, g * T, -1)
    probs = torch.softmax(scores, dim=-1, dtype=torch.promote_types(q.dtype, torch.float32)).to(q.dtype)
    out = torch.bmm(probs, v.contiguous())  # [Hkv, g*T, d]
    return out.view(Hkv, g, T, d).permute(2, 0, 1, 3).reshape(T, Hq * d)
