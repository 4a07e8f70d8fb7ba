"""Qwen3-4B projection geometry and the byte/FLOP accounting of the path.

Constants follow leanstack's model registry (src/leanstack/model_registry.py:16-23)
and the fused shapes its packer writes (src/leanstack/pack.py:269-286):
q/k/v are concatenated along rows into qkv_proj [4096+1024+1024, 2560] and
gate/up into gate_up_proj [2*9728, 2560]; every weight is [N, K] with
y = x . W^T.
"""

from __future__ import annotations

from dataclasses import dataclass

BF16_BYTES = 2


@dataclass(frozen=True)
class QwenGeometry:
    num_hidden_layers: int = 36
    hidden_size: int = 2560
    intermediate_size: int = 9728
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    vocab_size: int = 151936
    max_position_embeddings: int = 32768
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0

    @property
    def q_dim(self) -> int:
        return self.num_attention_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_key_value_heads * self.head_dim

    @property
    def qkv_dim(self) -> int:
        return self.q_dim + 2 * self.kv_dim

    def projections(self) -> dict[str, tuple[int, int]]:
        """(N, K) of each per-layer projection weight, in call order."""
        return {
            "qkv_proj": (self.qkv_dim, self.hidden_size),
            "o_proj": (self.hidden_size, self.q_dim),
            "gate_up_proj": (2 * self.intermediate_size, self.hidden_size),
            "down_proj": (self.hidden_size, self.intermediate_size),
        }

    def output_dim(self, name: str) -> int:
        """Columns each projection writes (gate_up writes SiLU(gate)*up)."""
        n, _ = self.projections()[name]
        return n // 2 if name == "gate_up_proj" else n

    def layer_weight_bytes(self) -> int:
        return sum(n * k * BF16_BYTES for n, k in self.projections().values())

    def layer_params(self) -> int:
        return sum(n * k for n, k in self.projections().values())

    def lm_head_bytes(self) -> int:
        return self.vocab_size * self.hidden_size * BF16_BYTES

    def projection_bytes(self, name: str, m: int) -> int:
        """Algorithmic HBM bytes of one projection call at M rows: weights +
        activations read + outputs written (bf16)."""
        n, k = self.projections()[name]
        return (n * k + m * k + m * self.output_dim(name)) * BF16_BYTES

    def layer_bytes(self, m: int) -> int:
        return sum(self.projection_bytes(name, m) for name in self.projections())

    def stack_bytes(self, m: int) -> int:
        return self.num_hidden_layers * self.layer_bytes(m)

    def lm_head_call_bytes(self, m: int, logits: bool = True) -> int:
        """Weights + hidden rows (bf16), + fp32 logits when the call writes
        them (the cuTile head's score precision).  The greedy head of the
        reference (cutile_logits.py:17-31) writes only its tile maxima, so
        its bytes are the weights and hidden rows (logits=False)."""
        return (self.lm_head_bytes() + m * self.hidden_size * BF16_BYTES
                + (m * self.vocab_size * 4 if logits else 0))

    def projection_flops(self, name: str, m: int) -> int:
        n, k = self.projections()[name]
        return 2 * m * n * k

    def layer_flops(self, m: int) -> int:
        return sum(self.projection_flops(name, m) for name in self.projections())


QWEN3_4B = QwenGeometry()
