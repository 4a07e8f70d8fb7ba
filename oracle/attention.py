"""CPU restatement of one decode token's attention step and of a whole decode
layer (oracle) -- test infrastructure only, see oracle/__init__.py.

Each function follows the reference's eager code cited in its docstring with
the same torch ops in bf16 on the CPU, so the per-op bf16 roundings are the
reference's.  The attention itself is computed in fp32 from the bf16 q, K, V
(F.scaled_dot_product_attention's math: fp32 scores, softmax and weighted
sum, bf16 output).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .projections import rmsnorm


def rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """qwen_apply_rotary_pos_emb (qwen_explicit.py:690-716), unsqueeze_dim=1:
    q, k [B, heads, T, d]; cos, sin [B, T, d/2] (half width)."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)

    def rotate(t):
        first, second = t.chunk(2, dim=-1)
        return torch.cat(((first * cos) - (second * sin), (second * cos) + (first * sin)), dim=-1)

    return rotate(q), rotate(k)


def qk_heads_vector(qkv: torch.Tensor, n_q: int, n_kv: int, d: int, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                    eps: float, cos: torch.Tensor, sin: torch.Tensor):
    """The tail of _semantic_attention_qkv_vector_eager (qwen_explicit.py:788-806):
    split [q|k|v], per-head RMSNorm of q and k, RoPE -> q [1,n_q,1,d],
    k / v [1,n_kv,1,d]."""
    q, k, v = torch.split(qkv, (n_q * d, n_kv * d, n_kv * d), dim=0)
    q = rmsnorm(q.view(1, n_q, d), q_norm_w, eps).view(1, n_q, 1, d)
    k = rmsnorm(k.view(1, n_kv, d), k_norm_w, eps).view(1, n_kv, 1, d)
    v = v.view(1, n_kv, 1, d)
    q, k = rope(q, k, cos.view(1, 1, -1), sin.view(1, 1, -1))
    return q, k, v


def sdpa_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, groups: int) -> torch.Tensor:
    """F.scaled_dot_product_attention(q, k, v, is_causal=False, scale=scale,
    enable_gqa=True) (qwen_explicit.py:894-912) in fp32: q [B,n_q,T,d],
    k / v [B,n_kv,S,d]; q head h reads kv head h // groups.  bf16 out."""
    kf = k.float().repeat_interleave(groups, dim=1)
    vf = v.float().repeat_interleave(groups, dim=1)
    scores = torch.matmul(q.float(), kf.transpose(-2, -1).contiguous()) * scale
    return torch.matmul(torch.softmax(scores, dim=-1), vf).to(q.dtype)


def decode_attention(qkv: torch.Tensor, n_q: int, n_kv: int, d: int, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                     eps: float, cos: torch.Tensor, sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     pos: int, scale: float):
    """One decode token: the q/k heads (:788-806), the static cache append at
    row `pos` (kv_cache.py:222-245, batch 1) and attention over rows 0..pos
    (:894-912).  k_cache / v_cache [n_kv, S, d] are not modified; returns
    (out [n_q*d], new k_cache, new v_cache)."""
    q, k, v = qk_heads_vector(qkv, n_q, n_kv, d, q_norm_w, k_norm_w, eps, cos, sin)
    k_cache = k_cache.clone()
    v_cache = v_cache.clone()
    k_cache[:, pos] = k.view(n_kv, d)
    v_cache[:, pos] = v.view(n_kv, d)
    out = sdpa_gqa(q, k_cache[None, :, : pos + 1], v_cache[None, :, : pos + 1], scale, n_q // n_kv)
    return out.reshape(-1), k_cache, v_cache


def decode_layer(hidden: torch.Tensor, input_ln_w: torch.Tensor, qkv_w: torch.Tensor, n_q: int, n_kv: int, d: int,
                 q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 k_cache: torch.Tensor, v_cache: torch.Tensor, pos: int, scale: float, o_w: torch.Tensor,
                 post_ln_w: torch.Tensor, gate_up_w: torch.Tensor, gate_dim: int, down_w: torch.Tensor,
                 eps: float):
    """semantic_qwen_decode_layer_forward (qwen_explicit.py:1247-1272) with
    _semantic_qwen_attention_decode_forward (:1147-1176) and
    _semantic_mlp_epilogue_vector_eager (:932-949): hidden [H] -> ([H], new
    k_cache, new v_cache)."""
    residual = hidden
    h = rmsnorm(residual.view(1, -1), input_ln_w, eps).view(-1)
    qkv = torch.mv(qkv_w, h)
    attn, k_cache, v_cache = decode_attention(qkv, n_q, n_kv, d, q_norm_w, k_norm_w, eps, cos, sin, k_cache, v_cache,
                                              pos, scale)
    hidden = residual + torch.mv(o_w, attn)
    residual = hidden
    h = rmsnorm(hidden.view(1, -1), post_ln_w, eps).view(-1)
    gate_up = torch.mv(gate_up_w, h)
    gate, up = torch.split(gate_up, (gate_dim, gate_up.shape[0] - gate_dim), dim=0)
    out = residual + torch.mv(down_w, F.silu(gate) * up)
    return out, k_cache, v_cache
