"""GPU tests of the drop-in dispatch entry points (leanstack_amd.dispatch)
against the CPU oracle on the same seeded inputs, and of the HIP kernels
against the committed golden vectors."""

from __future__ import annotations

import os
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from leanstack_amd import _lib, dispatch, kernels
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.layout import PackedWeight
from oracle import brute
from oracle import projections as ref
from tests.helpers import activations, assert_parity, from_bits, seeded_normal, weight

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = Path(__file__).resolve().parent / "golden"


def _pw(w, layout=_lib.LAYOUT_MFMA16X32):
    return PackedWeight.from_rowmajor(w.to(DEV), layout)


def _rope_cpu(q, k, cos, sin):
    """Rotate-half RoPE as qwen_explicit.py:690-716 defines it."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)

    def rot(t):
        a, b = t.chunk(2, dim=-1)
        return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)

    return rot(q), rot(k)


def _cos_sin(positions: int):
    """Half-width position cache, as build_qwen_position_cache makes it
    (qwen_explicit.py:664-676): [1, S, head_dim/2]."""
    inv = 1.0 / (G.rope_theta ** (torch.arange(0, G.head_dim, 2, dtype=torch.float32) / G.head_dim))
    freqs = torch.outer(torch.arange(positions, dtype=torch.float32), inv)
    return freqs.cos().to(torch.bfloat16)[None], freqs.sin().to(torch.bfloat16)[None]


def test_attention_qkv_vector(gpu):
    w = weight(G.qkv_dim, G.hidden_size, seed=1)
    h = activations(1, G.hidden_size, seed=2).view(-1)
    qn = seeded_normal((G.head_dim,), 0.1, 3) + 1
    kn = seeded_normal((G.head_dim,), 0.1, 4) + 1
    cos, sin = _cos_sin(8)
    cos, sin = cos[:, 5:6], sin[:, 5:6]
    q, k, v = dispatch._semantic_attention_qkv_vector(
        h.to(DEV), _pw(w), G.q_dim, G.kv_dim, G.num_attention_heads, G.num_key_value_heads, G.head_dim,
        qn.to(DEV), kn.to(DEV), cos.to(DEV), sin.to(DEV), G.rms_norm_eps)
    qkv = ref.mv(w, h)
    qs, ks, vs = torch.split(qkv, (G.q_dim, G.kv_dim, G.kv_dim))
    qs = F.rms_norm(qs.view(1, 32, 128), (128,), qn, G.rms_norm_eps).view(1, 32, 1, 128)
    ks = F.rms_norm(ks.view(1, 8, 128), (128,), kn, G.rms_norm_eps).view(1, 8, 1, 128)
    eq, ek = _rope_cpu(qs, ks, cos, sin)
    assert q.shape == (1, 32, 1, 128) and k.shape == (1, 8, 1, 128) and v.shape == (1, 8, 1, 128)
    assert_parity(q.cpu(), eq, "q")
    assert_parity(k.cpu(), ek, "k")
    assert_parity(v.cpu(), vs.view(1, 8, 1, 128), "v")


def test_input_norm_attention_qkv_vector(gpu):
    """input_layernorm + QKV in one kernel equals qwen_rmsnorm_vector (:1255)
    followed by the QKV path (:773-806) on the oracle."""
    w = weight(G.qkv_dim, G.hidden_size, seed=11)
    resid = (activations(1, G.hidden_size, seed=12).float() * 6.0).to(torch.bfloat16).view(-1)
    ln = seeded_normal((G.hidden_size,), 0.2, 13) + 1
    qn = seeded_normal((G.head_dim,), 0.1, 14) + 1
    kn = seeded_normal((G.head_dim,), 0.1, 15) + 1
    cos, sin = _cos_sin(8)
    cos, sin = cos[:, 3:4], sin[:, 3:4]
    q, k, v = dispatch._semantic_input_norm_attention_qkv_vector(
        resid.to(DEV), ln.to(DEV), _pw(w), G.q_dim, G.kv_dim, G.num_attention_heads, G.num_key_value_heads,
        G.head_dim, qn.to(DEV), kn.to(DEV), cos.to(DEV), sin.to(DEV), G.rms_norm_eps)
    h = ref.rmsnorm(resid.view(1, -1), ln, G.rms_norm_eps).view(-1)
    qkv = ref.mv(w, h)
    qs, ks, vs = torch.split(qkv, (G.q_dim, G.kv_dim, G.kv_dim))
    qs = F.rms_norm(qs.view(1, 32, 128), (128,), qn, G.rms_norm_eps).view(1, 32, 1, 128)
    ks = F.rms_norm(ks.view(1, 8, 128), (128,), kn, G.rms_norm_eps).view(1, 8, 1, 128)
    eq, ek = _rope_cpu(qs, ks, cos, sin)
    assert_parity(q.cpu(), eq, "q")
    assert_parity(k.cpu(), ek, "k")
    assert_parity(v.cpu(), vs.view(1, 8, 1, 128), "v")


def test_attention_qkv_batched(gpu):
    t = 5
    w = weight(G.qkv_dim, G.hidden_size, seed=11)
    h = activations(t, G.hidden_size, seed=12).view(1, t, -1)
    qn = torch.ones(G.head_dim, dtype=torch.bfloat16)
    cos, sin = _cos_sin(t)
    q, k, v = dispatch._semantic_attention_qkv(
        h.to(DEV), _pw(w), G.q_dim, G.kv_dim, 32, 8, 128, qn.to(DEV), qn.to(DEV), cos.to(DEV), sin.to(DEV), 1e-6)
    qkv = ref.linear(h, w)
    qs, ks, vs = torch.split(qkv, (G.q_dim, G.kv_dim, G.kv_dim), dim=-1)
    qs = F.rms_norm(qs.view(1, t, 32, 128), (128,), qn, 1e-6).transpose(1, 2)
    ks = F.rms_norm(ks.view(1, t, 8, 128), (128,), qn, 1e-6).transpose(1, 2)
    eq, ek = _rope_cpu(qs, ks, cos, sin)
    assert_parity(q.cpu(), eq, "q batched")
    assert_parity(k.cpu(), ek, "k batched")
    assert_parity(v.cpu(), vs.view(1, t, 8, 128).transpose(1, 2), "v batched")


def test_decode_attention_output_vector(gpu):
    s = 7
    w = weight(G.hidden_size, G.q_dim, seed=21)
    q = activations(32, 128, seed=22).view(1, 32, 1, 128)
    k = activations(8 * s, 128, seed=23).view(1, 8, s, 128)
    v = activations(8 * s, 128, seed=24).view(1, 8, s, 128)
    scale = 128 ** -0.5
    y = dispatch._semantic_decode_attention_output_vector(q.to(DEV), k.to(DEV), v.to(DEV), _pw(w), scale, 4)
    attn = F.scaled_dot_product_attention(q.float(), k.float().repeat_interleave(4, 1),
                                          v.float().repeat_interleave(4, 1), scale=scale)
    expect = ref.mv(w, attn.reshape(-1).to(torch.bfloat16))
    assert y.shape == (G.hidden_size,)
    assert_parity(y.cpu(), expect, "attention output + o_proj")


def _mlp_weights(seed):
    return (seeded_normal((G.hidden_size,), 0.1, seed) + 1, weight(2 * G.intermediate_size, G.hidden_size, seed + 1),
            weight(G.hidden_size, G.intermediate_size, seed + 2))


def test_mlp_epilogue_vector(gpu):
    ln, gu, dn = _mlp_weights(31)
    h = activations(1, G.hidden_size, seed=34).view(-1)
    y = dispatch._semantic_mlp_epilogue_vector(h.to(DEV), ln.to(DEV), _pw(gu, _lib.LAYOUT_MFMA16X32_GATEUP),
                                               G.intermediate_size, _pw(dn), G.rms_norm_eps)
    expect = ref.mlp_epilogue_vector(h, ln, gu, G.intermediate_size, dn, G.rms_norm_eps)
    assert y.shape == (G.hidden_size,)
    assert_parity(y.cpu(), expect, "mlp epilogue vector")


@pytest.mark.parametrize("t", [4, 64])
def test_post_attention_mlp(gpu, t):
    ln, gu, dn = _mlp_weights(41)
    o = weight(G.hidden_size, G.q_dim, seed=44)
    attn = activations(t, G.q_dim, seed=45).view(1, t, -1)
    res = activations(t, G.hidden_size, seed=46).view(1, t, -1)
    y = dispatch._semantic_post_attention_mlp(attn.to(DEV), res.to(DEV), _pw(o), ln.to(DEV),
                                              _pw(gu, _lib.LAYOUT_MFMA16X32_GATEUP), G.intermediate_size, _pw(dn),
                                              G.rms_norm_eps)
    expect = ref.post_attention_mlp(attn, res, o, ln, gu, G.intermediate_size, dn, G.rms_norm_eps)
    assert_parity(y.cpu(), expect, f"post-attention mlp T={t}")


def test_mlp_forward(gpu):
    _, gu, dn = _mlp_weights(51)
    h = activations(3, G.hidden_size, seed=54)
    mlp = SimpleNamespace(gate_up_proj_weight=_pw(gu, _lib.LAYOUT_MFMA16X32_GATEUP),
                          gate_proj_out_dim=G.intermediate_size, down_proj_weight=_pw(dn))
    y = dispatch.semantic_qwen_mlp_forward(mlp, h.to(DEV))
    assert_parity(y.cpu(), ref.mlp_forward(h, gu, G.intermediate_size, dn), "mlp forward")


@pytest.fixture(scope="module")
def head():
    e = weight(G.vocab_size, G.hidden_size, seed=61)
    norm = seeded_normal((G.hidden_size,), 0.1, 62) + 1
    return e, norm, _pw(e)


def test_greedy_head_vector_and_logits(gpu, head):
    e, norm, pe = head
    h = activations(1, G.hidden_size, seed=63).view(-1)
    idx = dispatch._semantic_greedy_head_vector(h.to(DEV), norm.to(DEV), pe, G.rms_norm_eps)
    assert idx.shape == (1, 1) and idx.dtype == torch.long
    assert idx.item() == ref.greedy_head_vector(h, norm, e, G.rms_norm_eps).item()
    runtime = SimpleNamespace(final_norm_weight=norm.to(DEV), lm_head_weight=pe,
                              config=SimpleNamespace(rms_norm_eps=G.rms_norm_eps))
    logits = dispatch.project_semantic_hidden_to_logits(runtime, h.view(1, 1, -1).to(DEV))
    normed = ref.rmsnorm(h.view(1, -1), norm, G.rms_norm_eps).view(-1)
    assert_parity(logits.view(-1).cpu(), ref.mv(e, normed), "bf16 logits")


def test_hip_logits_argmax_contract(gpu, head):
    e, _, pe = head
    h = activations(1, G.hidden_size, seed=64).view(-1)
    got = dispatch.hip_logits_argmax(h.to(DEV), pe)
    assert got.shape == (1, 1) and got.item() == ref.logits_argmax(h, e).item()
    with pytest.raises(ValueError):
        dispatch.hip_logits_argmax(h.view(1, -1).to(DEV), pe)        # not 1-D
    with pytest.raises(ValueError):
        dispatch.hip_logits_argmax(h.to(DEV), pe, vocab_tile=100)     # V % tile
    with pytest.raises(ValueError):
        dispatch.hip_logits_argmax(h.to(DEV), e.to(DEV))             # row-major weight


@pytest.mark.parametrize("backend", ["auto", "hip", "torch"])
def test_select_greedy_token_backends(gpu, head, backend, monkeypatch):
    e, norm, pe = head
    monkeypatch.setenv("LEANSTACK_SEMANTIC_LOGITS_BACKEND", backend)
    h = activations(3, G.hidden_size, seed=65).view(1, 3, -1)
    runtime = SimpleNamespace(final_norm_weight=norm.to(DEV), lm_head_weight=pe,
                              config=SimpleNamespace(rms_norm_eps=G.rms_norm_eps))
    tok = dispatch.select_semantic_greedy_token(runtime, h.to(DEV))
    normed = ref.rmsnorm(h[0, -1].view(1, -1), norm, G.rms_norm_eps).view(-1)
    if backend in ("auto", "hip"):
        assert tok.item() == ref.logits_argmax(normed, e).item()
    else:
        assert tok.item() == ref.greedy_head_vector(h[0, -1], norm, e, G.rms_norm_eps).item()


def test_select_greedy_tokens_verify_block(gpu, head):
    e, norm, pe = head
    m = 5
    h = activations(m, G.hidden_size, seed=66).view(1, m, -1)
    runtime = SimpleNamespace(final_norm_weight=norm.to(DEV), lm_head_weight=pe,
                              config=SimpleNamespace(rms_norm_eps=G.rms_norm_eps))
    toks = dispatch.select_semantic_greedy_tokens(runtime, h.to(DEV)).cpu()
    normed = ref.rmsnorm(h[0], norm, G.rms_norm_eps)
    assert toks.shape == (m, 1)
    assert torch.equal(toks.view(-1), ref.logits_scores_fp32(normed, e).argmax(dim=-1))


def test_rejects_row_major_weights(gpu):
    w = weight(G.hidden_size, G.q_dim, seed=71).to(DEV)
    q = activations(32, 128, seed=72).view(1, 32, 1, 128).to(DEV)
    with pytest.raises(ValueError):
        dispatch._semantic_decode_attention_output_vector(q, q[:, :8], q[:, :8], w, 0.1, 4)


# ----------------------------------------------------------- golden vectors


def _golden(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


@pytest.mark.parametrize("name", ["linear_m1", "linear_m5"])
def test_hip_linear_golden(gpu, name):
    g = _golden(name)
    y = kernels.linear(from_bits(g["x"]).to(DEV), _pw(from_bits(g["w"]))).double().cpu().numpy()
    slack = 0.5 * np.maximum(brute.bf16_ulp(g["y64"]), brute.bf16_ulp(y)) + g["bound"] + 1e-30
    assert np.all(np.abs(y - g["y64"]) <= slack)


def test_hip_silu_golden(gpu):
    g = _golden("silu_mul")
    y = kernels.linear(from_bits(g["x"]).to(DEV), _pw(from_bits(g["w"]), _lib.LAYOUT_MFMA16X32_GATEUP),
                       epilogue=_lib.EPI_SILU_MUL).double().cpu().numpy()
    slack = brute.bf16_ulp(g["out64"]) * 2 + 4 * g["bound"].max()
    assert np.all(np.abs(y - g["out64"]) <= slack)
    assert np.mean(y == g["out64"]) > 0.98


def test_hip_residual_golden(gpu):
    g = _golden("residual")
    y = kernels.linear(from_bits(g["x"]).to(DEV), _pw(from_bits(g["w"])), epilogue=_lib.EPI_RESIDUAL_ADD,
                       residual=from_bits(g["r"]).to(DEV)).double().cpu().numpy()
    assert np.all(np.abs(y - g["out64"]) <= brute.bf16_ulp(g["out64"]) + 2 * g["bound"])


def test_hip_lm_head_golden(gpu):
    g = _golden("lm_head")
    idx = kernels.lm_head_argmax(from_bits(g["x"]).to(DEV), _pw(from_bits(g["w"]))).cpu().numpy()
    assert np.array_equal(idx, g["expect"])
    idx_bf16 = kernels.lm_head_argmax(from_bits(g["x"]).to(DEV), _pw(from_bits(g["w"])),
                                      logits_mode=_lib.LOGITS_BF16).cpu().numpy()
    assert idx_bf16[-1] == g["tie_low"]
