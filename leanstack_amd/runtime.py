"""Runtime holders of the resident projection weights.

Same roles and field names as the reference's semantic runtime dataclasses
(src/leanstack/runtime/qwen_explicit.py:79-104, :123-144), with the
projection weights held as PackedWeight views into the resident arena.  The
fused tensors stay fused; the q/k/v weights are zero-copy views of the fused
QKV tensor, because the packed layout keeps every 16-row block contiguous
(the reference builds the same split views at src/leanstack/leanserve.py:
429-438).  The gate/up halves are interleaved in the packed layout, so they
are only reachable through the fused tensor.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import torch

from .layout import PackedWeight


@dataclass(frozen=True)
class QwenServeConfig:
    """Geometry + hyper-parameters (src/leanstack/leanserve.py:36-48)."""

    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    max_position_embeddings: int
    head_dim: int
    rms_norm_eps: float
    rope_parameters: dict


@dataclass
class QwenSemanticAttentionRuntime:
    layer_idx: int
    q_proj_weight: PackedWeight
    k_proj_weight: PackedWeight
    v_proj_weight: PackedWeight
    qkv_proj_weight: PackedWeight
    q_proj_out_dim: int
    k_proj_out_dim: int
    num_attention_heads: int
    num_key_value_heads: int
    num_key_value_groups: int
    head_dim: int
    attention_scale: float
    o_proj_weight: PackedWeight
    q_norm_weight: torch.Tensor
    k_norm_weight: torch.Tensor


@dataclass
class QwenSemanticMlpRuntime:
    gate_up_proj_weight: PackedWeight
    gate_proj_out_dim: int
    down_proj_weight: PackedWeight


@dataclass
class QwenSemanticLayerRuntime:
    layer_idx: int
    input_layernorm_weight: torch.Tensor
    attention: QwenSemanticAttentionRuntime
    post_attention_layernorm_weight: torch.Tensor
    mlp: QwenSemanticMlpRuntime


@dataclass
class QwenSemanticStackRuntime:
    model_path: Path
    config: QwenServeConfig
    layer_indices: tuple[int, ...]
    embed_tokens_weight: torch.Tensor
    layers: tuple[QwenSemanticLayerRuntime, ...]
    rope_inv_freq: torch.Tensor
    attention_scaling: float
    final_norm_weight: torch.Tensor | None
    lm_head_weight: PackedWeight | None
    device: torch.device
    dtype: torch.dtype


def split_rows(fused: PackedWeight, sizes: tuple[int, ...]) -> tuple[PackedWeight, ...]:
    """Zero-copy row splits of a packed weight at 16-row block boundaries."""
    if sum(sizes) != fused.n or any(s % 16 for s in sizes):
        raise ValueError(f"row split {sizes} does not tile {fused.n} rows in 16-row blocks")
    out, start = [], 0
    for s in sizes:
        out.append(PackedWeight(fused.data[start * fused.k : (start + s) * fused.k], s, fused.k, fused.layout))
        start += s
    return tuple(out)
