"""CPU torch restatement of the reference's projection arithmetic (oracle).

Each function follows the eager reference function cited in its docstring,
with the same torch ops in the same dtype (bf16 tensors on the CPU), so its
outputs are what the reference's own torch path produces on these inputs.
Test infrastructure only -- see oracle/__init__.py.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def mv(weight: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """torch.mv(W[N,K], x[K]) -> bf16 [N]: the M=1 projection
    (qwen_explicit.py:787, :913, :942, :948, :959)."""
    return torch.mv(weight, x)


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """F.linear(x[..., K], W[N, K]) -> bf16 [..., N]: the M>1 projection
    (qwen_explicit.py:748, :819, :828, :830, :1202, :1208)."""
    return F.linear(x, weight)


def silu_mul(gate_up: torch.Tensor, gate_dim: int) -> torch.Tensor:
    """Split [gate | up] at gate_dim and return F.silu(gate) * up in bf16
    (qwen_explicit.py:829-830, :943-948, :1203-1208)."""
    gate, up = torch.split(gate_up, (gate_dim, gate_up.shape[-1] - gate_dim), dim=-1)
    return F.silu(gate) * up


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """F.rms_norm over the last dim (qwen_explicit.py:621-628)."""
    return F.rms_norm(x, normalized_shape=(x.shape[-1],), weight=weight, eps=eps)


def mlp_epilogue_vector(hidden: torch.Tensor, post_ln_w: torch.Tensor, gate_up_w: torch.Tensor, gate_dim: int,
                        down_w: torch.Tensor, eps: float) -> torch.Tensor:
    """_semantic_mlp_epilogue_vector_eager (qwen_explicit.py:932-949)."""
    residual = hidden
    h = rmsnorm(hidden.view(1, -1), post_ln_w, eps).view(-1)
    gate_up = torch.mv(gate_up_w, h)
    return residual + torch.mv(down_w, silu_mul(gate_up, gate_dim))


def post_attention_mlp(attn: torch.Tensor, residual: torch.Tensor, o_w: torch.Tensor, post_ln_w: torch.Tensor,
                       gate_up_w: torch.Tensor, gate_dim: int, down_w: torch.Tensor, eps: float) -> torch.Tensor:
    """_semantic_post_attention_mlp_eager (qwen_explicit.py:809-831)."""
    h = residual + F.linear(attn, o_w)
    residual = h
    h = rmsnorm(h, post_ln_w, eps)
    gate_up = F.linear(h, gate_up_w)
    return residual + F.linear(silu_mul(gate_up, gate_dim), down_w)


def mlp_forward(hidden: torch.Tensor, gate_up_w: torch.Tensor, gate_dim: int, down_w: torch.Tensor) -> torch.Tensor:
    """semantic_qwen_mlp_forward (qwen_explicit.py:1201-1208)."""
    return F.linear(silu_mul(F.linear(hidden, gate_up_w), gate_dim), down_w)


def greedy_head_vector(hidden: torch.Tensor, final_norm_w: torch.Tensor, lm_w: torch.Tensor,
                       eps: float) -> torch.Tensor:
    """_semantic_greedy_head_vector_eager (qwen_explicit.py:952-960): bf16
    logits from torch.mv, first maximum -> int64 [1, 1]."""
    h = rmsnorm(hidden.view(1, -1), final_norm_w, eps).view(-1)
    logits = torch.mv(lm_w, h)
    return logits.argmax(dim=0, keepdim=True).view(1, 1)


def logits_scores_fp32(hidden: torch.Tensor, lm_w: torch.Tensor) -> torch.Tensor:
    """The cuTile head's scores: sum_k f32(W[v, k]) * f32(h[k]) with fp32
    accumulation (cutile_logits.py:20-27).  hidden [K] or [M, K] -> fp32 [V] or [M, V]."""
    return hidden.float() @ lm_w.float().t()


def logits_argmax(hidden: torch.Tensor, lm_w: torch.Tensor) -> torch.Tensor:
    """cutile_logits_argmax semantics (cutile_logits.py:37-69): fp32 scores,
    first maximum -> int64 [1, 1] (or [M, 1] for M rows)."""
    scores = logits_scores_fp32(hidden, lm_w)
    if scores.ndim == 1:
        return scores.argmax(dim=0).view(1, 1)
    return scores.argmax(dim=-1, keepdim=True)


def bf16_logits_argmax(hidden: torch.Tensor, lm_w: torch.Tensor) -> torch.Tensor:
    """Greedy token of bf16 logits per row (torch.mv / F.linear head,
    qwen_explicit.py:928-929, :959-960) -> int64 [M]."""
    h = hidden.view(-1, hidden.shape[-1])
    logits = torch.stack([torch.mv(lm_w, h[i]) for i in range(h.shape[0])])
    return logits.argmax(dim=-1)
