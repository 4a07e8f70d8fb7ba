"""Drop-in dispatch entry points with the reference's names and signatures.

leanstack's semantic runtime calls these module-level names once per layer
per step (src/leanstack/runtime/qwen_explicit.py:963-971, call sites :1117,
:1155, :1170, :1235, :1264, :1293).  Here every projection inside them runs
on the gfx950 kernels through the C ABI; the work around the projections
that is not part of this path (RMSNorm, q/k norm, RoPE, attention) stays
torch code with the reference's semantics (attention is computed explicitly
in fp32 with contiguous operands, see _sdpa).  The weight arguments are PackedWeight objects
from the resident arena (leanstack_amd.leanserve) instead of row-major
tensors; a row-major tensor is rejected with ValueError.

Differences from the reference, on purpose:
  - no torch.compile wrapper (the reference's _compile_reduce_overhead,
    :578-604, routes through Inductor/Triton, which this path does not use);
  - no silent fallback: the reference's "auto" logits backend falls back to
    torch when its kernel raises (:1820-1832); here a missing library or a
    rejected argument always raises.
  - residual adds that follow a projection (:820, :831, :949) are fused into
    that projection's epilogue, with the same bf16 rounding;
  - for decode and verify rows (M <= 16) the RMSNorm in front of gate_up
    (:821-827, :941) runs inside the gate_up kernel (kernels.rmsnorm_linear,
    one bf16 rounding as F.rms_norm); _semantic_input_norm_attention_qkv_vector
    offers the same for input_layernorm + QKV (:1255 then :787).
"""

from __future__ import annotations

import os

import torch
import torch.nn.functional as F

from . import _lib, kernels
from .layout import PackedWeight

# ---------------------------------------------------------------- torch glue
# (out of this path's scope; restated with the reference's semantics)


def qwen_rmsnorm(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """F.rms_norm over the last dim (qwen_explicit.py:621-628)."""
    return F.rms_norm(hidden_states, normalized_shape=(hidden_states.shape[-1],), weight=weight, eps=eps)


def qwen_rmsnorm_vector(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return qwen_rmsnorm(hidden_states.view(1, -1), weight, eps).view(-1)


def qwen_apply_rotary_pos_emb(query_states, key_states, cos, sin, unsqueeze_dim: int = 1):
    """Rotate-half RoPE on q and k (qwen_explicit.py:690-716)."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)

    def rotate(t):
        first, second = t.chunk(2, dim=-1)
        return torch.cat((first * cos - second * sin, second * cos + first * sin), dim=-1)

    return rotate(query_states), rotate(key_states)


def _sdpa(query_states, key_states, value_states, attention_scale, num_key_value_groups):
    """Non-causal GQA attention with the semantics of the reference's
    F.scaled_dot_product_attention call (qwen_explicit.py:894-912), computed
    in fp32 with contiguous operands: softmax(q k^T * scale) v, kv heads
    repeated per group, result in the query dtype."""
    k = key_states.float()
    v = value_states.float()
    if num_key_value_groups > 1:
        k = k.repeat_interleave(num_key_value_groups, dim=1)
        v = v.repeat_interleave(num_key_value_groups, dim=1)
    scores = torch.matmul(query_states.float(), k.transpose(-2, -1).contiguous()) * attention_scale
    probs = torch.softmax(scores, dim=-1)
    return torch.matmul(probs, v.contiguous()).to(query_states.dtype)


def _require_packed(weight, what: str, layout: int = _lib.LAYOUT_MFMA16X32) -> PackedWeight:
    if not isinstance(weight, PackedWeight):
        raise ValueError(f"{what} must be a PackedWeight from the resident arena, got {type(weight).__name__}")
    if weight.layout != layout:
        raise ValueError(f"{what} must use packed layout {layout}, got {weight.layout}")
    return weight


def _check_gate_dim(gate_up_proj_weight: PackedWeight, gate_proj_out_dim: int) -> None:
    if gate_proj_out_dim * 2 != gate_up_proj_weight.n:
        raise ValueError(
            f"gate_proj_out_dim={gate_proj_out_dim} must be half of the fused gate_up rows ({gate_up_proj_weight.n})"
        )


# ------------------------------------------------------------ projections


def _norm_gate_up(hidden_states, norm_weight, eps, gu_w: PackedWeight):
    """SiLU(gate)*up of rms_norm(hidden_states): fused into the gate_up kernel
    for decode / verify rows, F.rms_norm then the GEMM for prefill rows."""
    if hidden_states.numel() // gu_w.k <= _lib.DECODE_MAX_M:
        return kernels.rmsnorm_linear(hidden_states, norm_weight, eps, gu_w, epilogue=_lib.EPI_SILU_MUL)
    return kernels.linear(qwen_rmsnorm(hidden_states, norm_weight, eps), gu_w, epilogue=_lib.EPI_SILU_MUL)


def _semantic_attention_qkv(hidden_states, qkv_proj_weight, q_proj_out_dim, k_proj_out_dim, num_attention_heads,
                            num_key_value_heads, head_dim, q_norm_weight, k_norm_weight, cos, sin, rms_norm_eps):
    """M>1 fused QKV (qwen_explicit.py:733-770): [B,T,H] -> q [B,nq,T,d], k/v [B,nkv,T,d]."""
    w = _require_packed(qkv_proj_weight, "qkv_proj_weight")
    batch_size, query_len, _ = hidden_states.shape
    qkv_states = kernels.linear(hidden_states, w)
    query_states, key_states, value_states = torch.split(
        qkv_states, (q_proj_out_dim, k_proj_out_dim, k_proj_out_dim), dim=-1)
    query_states = query_states.view(batch_size, query_len, num_attention_heads, head_dim)
    key_states = key_states.view(batch_size, query_len, num_key_value_heads, head_dim)
    value_states = value_states.view(batch_size, query_len, num_key_value_heads, head_dim)
    query_states = F.rms_norm(query_states, normalized_shape=(head_dim,), weight=q_norm_weight,
                              eps=rms_norm_eps).transpose(1, 2)
    key_states = F.rms_norm(key_states, normalized_shape=(head_dim,), weight=k_norm_weight,
                            eps=rms_norm_eps).transpose(1, 2)
    value_states = value_states.transpose(1, 2)
    return qwen_apply_rotary_pos_emb(query_states, key_states, cos, sin) + (value_states,)


def _semantic_attention_qkv_vector(hidden_states, qkv_proj_weight, q_proj_out_dim, k_proj_out_dim,
                                   num_attention_heads, num_key_value_heads, head_dim, q_norm_weight, k_norm_weight,
                                   cos, sin, rms_norm_eps):
    """M=1 fused QKV GEMV (qwen_explicit.py:773-806): hidden [H] -> q [1,nq,1,d], k/v [1,nkv,1,d]."""
    w = _require_packed(qkv_proj_weight, "qkv_proj_weight")
    qkv_states = kernels.linear(hidden_states.view(1, -1), w).view(-1)
    return _qkv_heads_vector(qkv_states, q_proj_out_dim, k_proj_out_dim, num_attention_heads, num_key_value_heads,
                             head_dim, q_norm_weight, k_norm_weight, cos, sin, rms_norm_eps)


def _qkv_heads_vector(qkv_states, q_proj_out_dim, k_proj_out_dim, num_attention_heads, num_key_value_heads,
                      head_dim, q_norm_weight, k_norm_weight, cos, sin, rms_norm_eps):
    """Split a [qkv] row into heads, q/k norm and RoPE (qwen_explicit.py:788-806)."""
    query_states, key_states, value_states = torch.split(
        qkv_states, (q_proj_out_dim, k_proj_out_dim, k_proj_out_dim), dim=0)
    query_states = F.rms_norm(query_states.view(1, num_attention_heads, head_dim), normalized_shape=(head_dim,),
                              weight=q_norm_weight, eps=rms_norm_eps).view(1, num_attention_heads, 1, head_dim)
    key_states = F.rms_norm(key_states.view(1, num_key_value_heads, head_dim), normalized_shape=(head_dim,),
                            weight=k_norm_weight, eps=rms_norm_eps).view(1, num_key_value_heads, 1, head_dim)
    value_states = value_states.view(1, num_key_value_heads, 1, head_dim)
    return qwen_apply_rotary_pos_emb(query_states, key_states, cos, sin) + (value_states,)


def _semantic_input_norm_attention_qkv_vector(residual, input_layernorm_weight, qkv_proj_weight, q_proj_out_dim,
                                              k_proj_out_dim, num_attention_heads, num_key_value_heads, head_dim,
                                              q_norm_weight, k_norm_weight, cos, sin, rms_norm_eps):
    """qwen_rmsnorm_vector(residual, input_layernorm_weight) followed by
    _semantic_attention_qkv_vector (qwen_explicit.py:1255, then :773-806), with
    the RMSNorm computed inside the QKV kernel: no normalised copy of the
    hidden state is written.  Returns q [1,nq,1,d], k/v [1,nkv,1,d]."""
    w = _require_packed(qkv_proj_weight, "qkv_proj_weight")
    qkv_states = kernels.rmsnorm_linear(residual.reshape(1, -1), input_layernorm_weight, rms_norm_eps, w).view(-1)
    return _qkv_heads_vector(qkv_states, q_proj_out_dim, k_proj_out_dim, num_attention_heads, num_key_value_heads,
                             head_dim, q_norm_weight, k_norm_weight, cos, sin, rms_norm_eps)


def _semantic_post_attention_mlp(attention_output, residual, o_proj_weight, post_attention_layernorm_weight,
                                 gate_up_proj_weight, gate_proj_out_dim, down_proj_weight, rms_norm_eps):
    """M>1 o_proj + residual, RMSNorm, gate_up + SiLU*up, down + residual
    (qwen_explicit.py:809-831)."""
    o_w = _require_packed(o_proj_weight, "o_proj_weight")
    gu_w = _require_packed(gate_up_proj_weight, "gate_up_proj_weight", _lib.LAYOUT_MFMA16X32_GATEUP)
    d_w = _require_packed(down_proj_weight, "down_proj_weight")
    _check_gate_dim(gu_w, gate_proj_out_dim)
    hidden_states = kernels.linear(attention_output, o_w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=residual)
    act = _norm_gate_up(hidden_states, post_attention_layernorm_weight, rms_norm_eps, gu_w)
    return kernels.linear(act, d_w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=hidden_states)


def _semantic_mlp_epilogue(hidden_states, post_attention_layernorm_weight, gate_up_proj_weight, gate_proj_out_dim,
                           down_proj_weight, rms_norm_eps):
    """M>1 MLP block with residual (qwen_explicit.py:834-852)."""
    gu_w = _require_packed(gate_up_proj_weight, "gate_up_proj_weight", _lib.LAYOUT_MFMA16X32_GATEUP)
    d_w = _require_packed(down_proj_weight, "down_proj_weight")
    _check_gate_dim(gu_w, gate_proj_out_dim)
    act = _norm_gate_up(hidden_states, post_attention_layernorm_weight, rms_norm_eps, gu_w)
    return kernels.linear(act, d_w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=hidden_states)


def _semantic_mlp_epilogue_vector(hidden_states, post_attention_layernorm_weight, gate_up_proj_weight,
                                  gate_proj_out_dim, down_proj_weight, rms_norm_eps):
    """M=1 RMSNorm, gate_up GEMV + SiLU*up, down GEMV + residual (qwen_explicit.py:932-949)."""
    gu_w = _require_packed(gate_up_proj_weight, "gate_up_proj_weight", _lib.LAYOUT_MFMA16X32_GATEUP)
    d_w = _require_packed(down_proj_weight, "down_proj_weight")
    _check_gate_dim(gu_w, gate_proj_out_dim)
    residual = hidden_states.reshape(1, -1)
    act = kernels.rmsnorm_linear(residual, post_attention_layernorm_weight, rms_norm_eps, gu_w,
                                 epilogue=_lib.EPI_SILU_MUL)
    return kernels.linear(act, d_w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=residual).view(-1)


def _semantic_decode_attention_output(query_states, key_states, value_states, o_proj_weight, attention_scale,
                                      num_key_value_groups):
    """SDPA then o_proj over [B,T,nq*d] (qwen_explicit.py:855-883)."""
    o_w = _require_packed(o_proj_weight, "o_proj_weight")
    attn = _sdpa(query_states, key_states, value_states, attention_scale, num_key_value_groups)
    attn = attn.transpose(1, 2).reshape(query_states.shape[0], query_states.shape[2], -1)
    return kernels.linear(attn, o_w)


def _semantic_decode_attention_output_vector(query_states, key_states, value_states, o_proj_weight, attention_scale,
                                             num_key_value_groups):
    """SDPA then the M=1 o_proj GEMV (qwen_explicit.py:886-913) -> [H]."""
    o_w = _require_packed(o_proj_weight, "o_proj_weight")
    attn = _sdpa(query_states, key_states, value_states, attention_scale, num_key_value_groups)
    return kernels.linear(attn.reshape(1, -1), o_w).view(-1)


# ------------------------------------------------------------ decode layer


def _static_cache_layer(kv_cache, layer_idx: int):
    """The layer's [n_kv, max_seq_len, d] key / value caches and its cached
    row count, from a static cache with the reference's interface
    (src/leanstack/runtime/kv_cache.py:207-266: key_cache / value_cache
    [L, B, n_kv, S, d], layer_seq_lens), batch 1."""
    if hasattr(kv_cache, "layer_tensors"):
        k, v = kv_cache.layer_tensors(layer_idx)
    else:
        if kv_cache.key_cache.shape[1] != 1:
            raise ValueError("the decode attention kernel serves batch 1")
        k, v = kv_cache.key_cache[layer_idx, 0], kv_cache.value_cache[layer_idx, 0]
    return k, v, int(kv_cache.layer_seq_lens[layer_idx])


def _advance_cache(kv_cache, layer_idx: int) -> None:
    """Count the row the kernel wrote, as StaticKVBlockManager.append does
    after its copy (kv_cache.py:243-245)."""
    if hasattr(kv_cache, "advance"):
        kv_cache.advance(layer_idx, 1)
    else:
        kv_cache.layer_seq_lens[layer_idx] += 1
        kv_cache.max_layer_seq_len = max(kv_cache.max_layer_seq_len, kv_cache.layer_seq_lens[layer_idx])


def _attend_vector(attention, qkv_states, kv_cache, position_embeddings, rms_norm_eps):
    """q/k norms, RoPE, the cache append and GQA attention of one decode token
    in one kernel (the work of qwen_explicit.py:796-806, kv_cache.py:222-245
    and :894-912) -> [n_q * d]."""
    cos, sin = position_embeddings
    k_layer, v_layer, pos = _static_cache_layer(kv_cache, attention.layer_idx)
    out = kernels.decode_attention(
        qkv_states, attention.q_norm_weight, attention.k_norm_weight, rms_norm_eps, cos, sin, k_layer, v_layer, pos,
        attention.attention_scale, num_attention_heads=attention.num_attention_heads,
        num_key_value_heads=attention.num_key_value_heads)
    _advance_cache(kv_cache, attention.layer_idx)
    return out


def _semantic_qwen_attention_decode_forward(attention, hidden_states, kv_cache, position_embeddings, rms_norm_eps):
    """QKV GEMV, the attention kernel, o_proj GEMV (qwen_explicit.py:1147-1176) -> [H].
    `hidden_states` is the normalised hidden state, as the reference passes it."""
    qkv_w = _require_packed(attention.qkv_proj_weight, "qkv_proj_weight")
    o_w = _require_packed(attention.o_proj_weight, "o_proj_weight")
    qkv = kernels.linear(hidden_states.reshape(1, -1), qkv_w)
    attn = _attend_vector(attention, qkv, kv_cache, position_embeddings, rms_norm_eps)
    return kernels.linear(attn.view(1, -1), o_w).view(-1)


def semantic_qwen_decode_layer_forward(layer, hidden_states, kv_cache, position_embeddings, rms_norm_eps):
    """One decode layer (qwen_explicit.py:1247-1272) in five kernels:
    input_layernorm + QKV, the attention kernel, o_proj + residual,
    post_attention_layernorm + gate_up + SiLU*up, down + residual.
    Returns [1, 1, H]."""
    a = layer.attention
    qkv_w = _require_packed(a.qkv_proj_weight, "qkv_proj_weight")
    o_w = _require_packed(a.o_proj_weight, "o_proj_weight")
    gu_w = _require_packed(layer.mlp.gate_up_proj_weight, "gate_up_proj_weight", _lib.LAYOUT_MFMA16X32_GATEUP)
    d_w = _require_packed(layer.mlp.down_proj_weight, "down_proj_weight")
    _check_gate_dim(gu_w, layer.mlp.gate_proj_out_dim)
    residual = hidden_states.reshape(1, -1)
    qkv = kernels.rmsnorm_linear(residual, layer.input_layernorm_weight, rms_norm_eps, qkv_w)
    attn = _attend_vector(a, qkv, kv_cache, position_embeddings, rms_norm_eps)
    hidden = kernels.linear(attn.view(1, -1), o_w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=residual)
    act = kernels.rmsnorm_linear(hidden, layer.post_attention_layernorm_weight, rms_norm_eps, gu_w,
                                 epilogue=_lib.EPI_SILU_MUL)
    return kernels.linear(act, d_w, epilogue=_lib.EPI_RESIDUAL_ADD, residual=hidden).view(1, 1, -1)


def semantic_qwen_mlp_forward(mlp, hidden_states):
    """gate_up + SiLU*up, down (qwen_explicit.py:1201-1208); `mlp` has
    gate_up_proj_weight, gate_proj_out_dim and down_proj_weight."""
    gu_w = _require_packed(mlp.gate_up_proj_weight, "gate_up_proj_weight", _lib.LAYOUT_MFMA16X32_GATEUP)
    _check_gate_dim(gu_w, mlp.gate_proj_out_dim)
    act = kernels.linear(hidden_states, gu_w, epilogue=_lib.EPI_SILU_MUL)
    return kernels.linear(act, _require_packed(mlp.down_proj_weight, "down_proj_weight"))


# ----------------------------------------------------------------- lm_head


def _greedy_rows(hidden: torch.Tensor, lm_head_weight: PackedWeight, logits_mode: int) -> torch.Tensor:
    w = _require_packed(lm_head_weight, "lm_head_weight")
    return kernels.lm_head_argmax(hidden.reshape(-1, w.k), w, logits_mode=logits_mode)


def _greedy_rows_normed(rows: torch.Tensor, final_norm_weight, lm_head_weight, rms_norm_eps,
                        logits_mode: int) -> torch.Tensor:
    """Final RMSNorm + head + argmax of [M, H] rows: in the lm_head kernel
    (lsk_rmsnorm_lm_head_argmax_bf16) for the Qwen3-4B hidden size and up to
    8 rows, else a separate norm in front of the head."""
    w = _require_packed(lm_head_weight, "lm_head_weight")
    rows = rows.reshape(-1, w.k)
    if w.k == 2560 and rows.shape[0] <= 8 and final_norm_weight.dtype == torch.bfloat16 and \
            final_norm_weight.device.type == "cuda":
        return kernels.lm_head_argmax(rows, w, logits_mode=logits_mode, norm_weight=final_norm_weight,
                                      eps=rms_norm_eps)
    normed = torch.nn.functional.rms_norm(rows, (w.k,), final_norm_weight, rms_norm_eps)
    return _greedy_rows(normed, w, logits_mode)


def _semantic_greedy_head_vector(hidden_states, final_norm_weight, lm_head_weight, rms_norm_eps):
    """RMSNorm, bf16 logits, first maximum -> int64 [1, 1] (qwen_explicit.py:952-960),
    the norm inside the lm_head kernel."""
    return _greedy_rows_normed(hidden_states, final_norm_weight, lm_head_weight, rms_norm_eps,
                               _lib.LOGITS_BF16).view(1, 1)


def _semantic_greedy_head(hidden_states, final_norm_weight, lm_head_weight, rms_norm_eps):
    """RMSNorm, bf16 logits of the last position, argmax -> [B, 1] (qwen_explicit.py:916-929)."""
    return _greedy_rows_normed(hidden_states[:, -1, :], final_norm_weight, lm_head_weight, rms_norm_eps,
                               _lib.LOGITS_BF16).view(-1, 1)


def hip_logits_argmax(hidden_states: torch.Tensor, lm_head_weight: PackedWeight, *, vocab_tile: int = 128,
                      hidden_tile: int = 64) -> torch.LongTensor:
    """The cutile_logits_argmax contract (src/leanstack/runtime/cutile_logits.py:37-69):
    1-D hidden, fp32 scores, first maximum -> int64 [1, 1]; same ValueErrors."""
    if hidden_states.ndim != 1:
        raise ValueError(f"expected a 1D hidden-state vector, got shape={tuple(hidden_states.shape)}")
    w = _require_packed(lm_head_weight, "lm_head_weight")
    if hidden_states.device.type != "cuda" or w.device.type != "cuda":
        raise ValueError("HIP logits argmax requires GPU tensors")
    vocab_size, hidden_size = w.shape
    if vocab_size % vocab_tile != 0:
        raise ValueError(f"vocab_size={vocab_size} must be divisible by vocab_tile={vocab_tile}")
    if hidden_size % hidden_tile != 0:
        raise ValueError(f"hidden_size={hidden_size} must be divisible by hidden_tile={hidden_tile}")
    return _greedy_rows(hidden_states, w, _lib.LOGITS_FP32).view(1, 1)


def hip_logits_argmax_rows(hidden_states: torch.Tensor, lm_head_weight: PackedWeight) -> torch.LongTensor:
    """M-row greedy head for a verify block ([M, H] or [1, M, H], M <= 16): one
    launch instead of the per-position head loop with a host sync per row
    (experiments/models/qwen_explicit_runtime_loop.py:805-812) -> int64 [M, 1]."""
    return _greedy_rows(hidden_states, lm_head_weight, _lib.LOGITS_FP32).view(-1, 1)


def resolve_semantic_logits_backend() -> str:
    """LEANSTACK_SEMANTIC_LOGITS_BACKEND (qwen_explicit.py:150-151)."""
    return os.environ.get("LEANSTACK_SEMANTIC_LOGITS_BACKEND", "auto").strip().lower()


def last_hidden_vector(hidden_states: torch.Tensor) -> torch.Tensor:
    return hidden_states[:, -1, :].reshape(-1)


def select_semantic_greedy_token(runtime, hidden_states: torch.Tensor) -> torch.LongTensor:
    """Greedy token of the last position (qwen_explicit.py:1814-1832).

    Backends "auto", "cutile" and "hip" use the fp32-score head (the cuTile
    semantics); any other value uses the bf16-logit head of
    _semantic_greedy_head_vector.  Both run on the HIP kernels; errors raise."""
    if runtime.final_norm_weight is None or runtime.lm_head_weight is None:
        raise ValueError("runtime does not include model.norm and lm_head")
    last = last_hidden_vector(hidden_states)
    backend = resolve_semantic_logits_backend()
    if backend in {"auto", "cutile", "hip"}:
        return _greedy_rows_normed(last, runtime.final_norm_weight, runtime.lm_head_weight,
                                   runtime.config.rms_norm_eps, _lib.LOGITS_FP32).view(1, 1)
    return _semantic_greedy_head_vector(last, runtime.final_norm_weight, runtime.lm_head_weight,
                                        runtime.config.rms_norm_eps)


def select_semantic_greedy_tokens(runtime, hidden_states: torch.Tensor) -> torch.LongTensor:
    """Greedy token of every position of a verify block [1, M, H] in one call
    (M <= 16) -> int64 [M, 1]; replaces the per-position select loop of
    qwen_explicit_runtime_loop.py:805-812."""
    normed = qwen_rmsnorm(hidden_states.reshape(-1, hidden_states.shape[-1]), runtime.final_norm_weight,
                          runtime.config.rms_norm_eps)
    return hip_logits_argmax_rows(normed, runtime.lm_head_weight)


def project_semantic_hidden_to_logits(runtime, hidden_states: torch.Tensor) -> torch.Tensor:
    """bf16 logits of the last position -> [1, 1, V] (qwen_explicit.py:1775-1783)."""
    w = _require_packed(runtime.lm_head_weight, "lm_head_weight")
    normed = qwen_rmsnorm_vector(last_hidden_vector(hidden_states), runtime.final_norm_weight,
                                 runtime.config.rms_norm_eps)
    logits = torch.empty((1, w.n), device=normed.device, dtype=torch.float32)
    kernels.lm_head_argmax(normed.view(1, -1), w, logits_mode=_lib.LOGITS_BF16, logits_out=logits)
    return logits.to(torch.bfloat16).view(1, 1, -1)


# The reference binds these names lazily through torch.compile
# (qwen_explicit.py:963-971); here they are the HIP-backed functions above.
_semantic_attention_qkv_eager = _semantic_attention_qkv
_semantic_attention_qkv_vector_eager = _semantic_attention_qkv_vector
_semantic_post_attention_mlp_eager = _semantic_post_attention_mlp
_semantic_mlp_epilogue_eager = _semantic_mlp_epilogue
_semantic_mlp_epilogue_vector_eager = _semantic_mlp_epilogue_vector
_semantic_decode_attention_output_eager = _semantic_decode_attention_output
_semantic_decode_attention_output_vector_eager = _semantic_decode_attention_output_vector
_semantic_greedy_head_vector_eager = _semantic_greedy_head_vector
_semantic_greedy_head_eager = _semantic_greedy_head
