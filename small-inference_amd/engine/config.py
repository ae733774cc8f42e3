"""Model hyperparameters the paged cache needs (the caller's ModelConfig, reference engine/config.py:8-39).

The cache reads num_layers, num_kv_heads, head_dim and kv_bytes_per_token(); the other fields exist so that the
reference's callers (and this repo's decode-step driver) can pass the same object.
"""

from dataclasses import dataclass


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 32768
    tie_word_embeddings: bool = True

    @property
    def group_size(self) -> int:
        """Query heads per KV head."""
        return self.num_q_heads // self.num_kv_heads

    @property
    def q_size(self) -> int:
        """Width of the query projection output."""
        return self.num_q_heads * self.head_dim

    @property
    def kv_size(self) -> int:
        """Width of each of the K and V projection outputs."""
        return self.num_kv_heads * self.head_dim

    def kv_bytes_per_token(self, bytes_per_elem: int = 2) -> int:
        """K and V of one token across all layers (12,288 B for Qwen2.5-0.5B in bf16)."""
        return 2 * self.num_layers * self.kv_size * bytes_per_elem


# The two attention shapes the benchmarks use (reference README.md:22).
QWEN2_5_0_5B = ModelConfig(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_layers=24,
                           num_q_heads=14, num_kv_heads=2, head_dim=64)
QWEN2_5_1_5B = ModelConfig(vocab_size=151936, hidden_size=1536, intermediate_size=8960, num_layers=28,
                           num_q_heads=12, num_kv_heads=2, head_dim=128)
