"""GPU parity of the decode attention kernel (lsk_decode_attention_bf16) and of
the fused decode layer against the CPU oracle (oracle/attention.py).

Bar: attention outputs and layer outputs within cosine >= 0.9999 and
normwise max relative error <= 1e-2; the cache row the kernel writes: v bit
for bit, k (normalised and rotated) equal on >= 98 % of the values and
within one bf16 step elsewhere (the kernel's per-head sum of squares is
added in another order than torch's); every other cache row unchanged bit
for bit.  Rows past `pos` hold NaN, so a kernel that read them would return
NaN.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from leanstack_amd import _lib, dispatch, kernels
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.kv_cache import ArenaKVCache
from leanstack_amd.layout import PackedWeight
from oracle import attention as ref_attn
from tests.helpers import assert_greedy_rows, assert_parity, bits, seeded_normal, weight

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
D = 128
EPS = 1e-6


def _inputs(n_q, n_kv, s_max, pos, seed):
    gen = torch.Generator().manual_seed(seed)
    qkv = (torch.randn((n_q + 2 * n_kv) * D, generator=gen) * 2).to(torch.bfloat16)
    qn = (1 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16)
    kn = (1 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16)
    ang = torch.rand(D // 2, generator=gen) * 50
    cos, sin = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
    kc = torch.randn((n_kv, s_max, D), generator=gen).to(torch.bfloat16)
    vc = torch.randn((n_kv, s_max, D), generator=gen).to(torch.bfloat16)
    kc[:, pos + 1:] = float("nan")
    vc[:, pos + 1:] = float("nan")
    return qkv, qn, kn, cos, sin, kc, vc


def _check_case(n_q, n_kv, s_max, pos, seed):
    qkv, qn, kn, cos, sin, kc, vc = _inputs(n_q, n_kv, s_max, pos, seed)
    kd, vd = kc.to(DEV), vc.to(DEV)
    out = kernels.decode_attention(qkv.to(DEV), qn.to(DEV), kn.to(DEV), EPS, cos.to(DEV), sin.to(DEV), kd, vd, pos,
                                   D ** -0.5, num_attention_heads=n_q, num_key_value_heads=n_kv)
    torch.cuda.synchronize()
    out, kd, vd = out.cpu(), kd.cpu(), vd.cpu()
    expect, k2, v2 = ref_attn.decode_attention(qkv, n_q, n_kv, D, qn, kn, EPS, cos, sin, kc, vc, pos, D ** -0.5)
    what = f"n_q={n_q} n_kv={n_kv} pos={pos}"
    assert not torch.isnan(out).any(), what
    assert_parity(out, expect, what)
    rows = [t for t in range(s_max) if t != pos]
    assert (bits(kd[:, rows]) == bits(kc[:, rows])).all(), f"{what}: k rows other than pos changed"
    assert (bits(vd[:, rows]) == bits(vc[:, rows])).all(), f"{what}: v rows other than pos changed"
    assert torch.equal(vd[:, pos], v2[:, pos]), f"{what}: v row"
    kdiff = (kd[:, pos].float() - k2[:, pos].float()).abs()
    assert (kdiff == 0).float().mean() >= 0.98, f"{what}: k row"
    assert (kdiff <= k2[:, pos].float().abs() * 2.0 ** -7 + 1e-30).all(), f"{what}: k row beyond one bf16 step"


@pytest.mark.parametrize("pos", [0, 1, 2, 15, 16, 17, 63, 64, 127, 128, 191, 192, 319, 511, 512, 513, 1000, 1023,
                                 1024, 1500, 2047, 3071, 3072, 4095])
def test_decode_attention_qwen3_4b(gpu, pos):
    """32 q heads, 8 kv heads, head_dim 128, a 4096-row cache: one 128-row
    chunk up to pos 127, 3..8 chunks of 64 rows up to pos 511 (the last one
    holding 1 or 64 rows), then 5..32 chunks of 128 rows combined through the
    workspace (8, 16, 24 and 32 chunk slots per combine round at the edges;
    pos 1500: 12 chunks, so 4 slots of the round lie past the last chunk)."""
    _check_case(G.num_attention_heads, G.num_key_value_heads, 4096, pos, seed=9000 + pos)


@pytest.mark.parametrize("pos", [4096, 8191, 8192, 12287, 12288, 16383])
def test_decode_attention_long_cache(gpu, pos):
    """A 16384-row cache: chunks of 256, 384 and 512 rows once more than
    4096, 8192 and 12288 rows are attended."""
    _check_case(G.num_attention_heads, G.num_key_value_heads, 16384, pos, seed=9300 + pos)


def _same_bits(a, b):
    """bf16 tensors equal bit for bit (NaN payloads included)."""
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def _device_pos_case(s_max, positions, seed):
    """The device-position entry point against the host-position one, launch
    by launch on the same inputs: outputs and caches bit for bit."""
    n_q, n_kv = G.num_attention_heads, G.num_key_value_heads
    gen = torch.Generator().manual_seed(seed)
    qkv = (torch.randn((n_q + 2 * n_kv) * D, generator=gen) * 2).to(torch.bfloat16).to(DEV)
    qn = (1 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16).to(DEV)
    kn = (1 + 0.2 * torch.randn(D, generator=gen)).to(torch.bfloat16).to(DEV)
    ang = torch.rand((s_max, D // 2), generator=gen) * 50
    cos_t, sin_t = ang.cos().to(torch.bfloat16).to(DEV), ang.sin().to(torch.bfloat16).to(DEV)
    kc = torch.randn((n_kv, s_max, D), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((n_kv, s_max, D), generator=gen).to(torch.bfloat16).to(DEV)
    pos_dev = torch.zeros((1,), dtype=torch.int32, device=DEV)
    ws_a = torch.zeros(_lib.load().lsk_attention_workspace_bytes(n_q, n_kv, D, s_max), dtype=torch.uint8, device=DEV)
    ws_b = torch.zeros_like(ws_a)
    k1, v1, k2, v2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    for pos in positions:
        a = kernels.decode_attention(qkv, qn, kn, EPS, cos_t[pos], sin_t[pos], k1, v1, pos, D ** -0.5,
                                     num_attention_heads=n_q, num_key_value_heads=n_kv, workspace=ws_a)
        pos_dev.fill_(pos)
        b = kernels.decode_attention(qkv, qn, kn, EPS, cos_t, sin_t, k2, v2, pos_dev, D ** -0.5,
                                     num_attention_heads=n_q, num_key_value_heads=n_kv, workspace=ws_b)
        torch.cuda.synchronize()
        assert not torch.isnan(b).any(), pos
        assert _same_bits(a, b), f"pos={pos}: device-position output differs"
        assert _same_bits(k1, k2) and _same_bits(v1, v2), f"pos={pos}: caches differ"
    assert not ws_b[:256].any(), "the arrival counters are left zero"


def test_decode_attention_device_position(gpu):
    """Positions in device memory at every chunk-rule regime up to 4096 rows."""
    _device_pos_case(4096, [0, 1, 127, 128, 129, 200, 511, 512, 1000, 1500, 2047, 3072, 4095], 9400)


def test_decode_attention_device_position_long_cache(gpu):
    """A 16384-row cache: chunks of 256, 384 and 512 rows from the device pos."""
    _device_pos_case(16384, [4096, 8192, 12288, 16383, 3], 9401)


def test_decode_attention_device_position_out_of_range(gpu):
    """A device pos outside [0, max_seq_len) leaves the output, the caches and
    the workspace untouched."""
    n_q, n_kv, s_max = 8, 2, 256
    gen = torch.Generator().manual_seed(9402)
    qkv = torch.randn((n_q + 2 * n_kv) * D, generator=gen).to(torch.bfloat16).to(DEV)
    ones = torch.ones(D, dtype=torch.bfloat16, device=DEV)
    tab = torch.ones((s_max, D // 2), dtype=torch.bfloat16, device=DEV)
    kc = torch.randn((n_kv, s_max, D), generator=gen).to(torch.bfloat16).to(DEV)
    vc = kc.clone()
    k0, v0 = kc.clone(), vc.clone()
    ws = torch.zeros(_lib.load().lsk_attention_workspace_bytes(n_q, n_kv, D, s_max), dtype=torch.uint8, device=DEV)
    for bad in (s_max, -1, 1 << 30):
        out = torch.full((n_q * D,), 7.0, dtype=torch.bfloat16, device=DEV)
        pos_dev = torch.full((1,), bad, dtype=torch.int32, device=DEV)
        kernels.decode_attention(qkv, ones, ones, EPS, tab, tab, kc, vc, pos_dev, D ** -0.5, num_attention_heads=n_q,
                                 num_key_value_heads=n_kv, out=out, workspace=ws)
        torch.cuda.synchronize()
        assert (out == 7.0).all() and torch.equal(kc, k0) and torch.equal(vc, v0) and not ws.any(), bad


@pytest.mark.parametrize("n_q", [2, 4, 16])
@pytest.mark.parametrize("pos", [0, 100, 511])
def test_decode_attention_group_sizes(gpu, n_q, pos):
    """q heads per kv head 1, 2 and 8 (two kv heads)."""
    _check_case(n_q, 2, 512, pos, seed=9100 + n_q + pos)


def test_decode_attention_repeatable(gpu):
    """Two launches on the same inputs give the same bits."""
    qkv, qn, kn, cos, sin, kc, vc = _inputs(32, 8, 1024, 700, 9200)
    outs = []
    for _ in range(2):
        kd, vd = kc.to(DEV), vc.to(DEV)
        outs.append(kernels.decode_attention(qkv.to(DEV), qn.to(DEV), kn.to(DEV), EPS, cos.to(DEV), sin.to(DEV), kd,
                                             vd, 700, D ** -0.5, num_attention_heads=32, num_key_value_heads=8).cpu())
    assert torch.equal(outs[0], outs[1])


def _layer(seed):
    """A Qwen3-4B-shaped layer: packed weights on the GPU, row-major on the CPU."""
    h, i = G.hidden_size, G.intermediate_size
    w = {
        "qkv": weight(G.qkv_dim, h, seed=seed),
        "o": weight(h, G.q_dim, seed=seed + 1),
        "gate_up": weight(2 * i, h, seed=seed + 2),
        "down": weight(h, i, seed=seed + 3),
        "in_ln": (1 + seeded_normal((h,), 0.1, seed + 4).float()).to(torch.bfloat16),
        "post_ln": (1 + seeded_normal((h,), 0.1, seed + 5).float()).to(torch.bfloat16),
        "qn": (1 + seeded_normal((D,), 0.1, seed + 6).float()).to(torch.bfloat16),
        "kn": (1 + seeded_normal((D,), 0.1, seed + 7).float()).to(torch.bfloat16),
    }
    pw = lambda t, layout=_lib.LAYOUT_MFMA16X32: PackedWeight.from_rowmajor(t.to(DEV), layout)  # noqa: E731
    attention = SimpleNamespace(
        layer_idx=0, qkv_proj_weight=pw(w["qkv"]), o_proj_weight=pw(w["o"]), q_norm_weight=w["qn"].to(DEV),
        k_norm_weight=w["kn"].to(DEV), num_attention_heads=G.num_attention_heads,
        num_key_value_heads=G.num_key_value_heads, head_dim=D, attention_scale=D ** -0.5,
        num_key_value_groups=G.num_attention_heads // G.num_key_value_heads)
    layer = SimpleNamespace(
        layer_idx=0, input_layernorm_weight=w["in_ln"].to(DEV), attention=attention,
        post_attention_layernorm_weight=w["post_ln"].to(DEV),
        mlp=SimpleNamespace(gate_up_proj_weight=pw(w["gate_up"], _lib.LAYOUT_MFMA16X32_GATEUP),
                            gate_proj_out_dim=i, down_proj_weight=pw(w["down"])))
    return w, layer


def _cos_sin(pos):
    inv = 1.0 / (G.rope_theta ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    f = pos * inv
    return f.cos().to(torch.bfloat16), f.sin().to(torch.bfloat16)


def test_decode_layer_three_tokens(gpu):
    """semantic_qwen_decode_layer_forward over three consecutive tokens (the
    cache cursor advances) against the oracle's layer on the same caches."""
    w, layer = _layer(9300)
    s_max = 64
    cache = ArenaKVCache(1, G.num_key_value_heads, D, s_max, device=DEV)
    kc = torch.zeros((G.num_key_value_heads, s_max, D), dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    gen = torch.Generator().manual_seed(9301)
    for pos in range(3):
        hidden = (torch.randn(G.hidden_size, generator=gen) * 3).to(torch.bfloat16)
        cos, sin = _cos_sin(pos)
        got = dispatch.semantic_qwen_decode_layer_forward(layer, hidden.to(DEV).view(1, 1, -1), cache,
                                                          (cos.to(DEV).view(1, 1, -1), sin.to(DEV).view(1, 1, -1)),
                                                          EPS)
        torch.cuda.synchronize()
        expect, kc, vc = ref_attn.decode_layer(
            hidden, w["in_ln"], w["qkv"], G.num_attention_heads, G.num_key_value_heads, D, w["qn"], w["kn"], cos, sin,
            kc, vc, pos, D ** -0.5, w["o"], w["post_ln"], w["gate_up"], G.intermediate_size, w["down"], EPS)
        assert got.shape == (1, 1, G.hidden_size)
        assert_parity(got.cpu().view(-1), expect, f"decode layer pos={pos}")
        assert cache.rows(0) == pos + 1 and cache.max_layer_seq_len == pos + 1
        k_layer, v_layer = cache.layer_tensors(0)
        assert_parity(v_layer[:, : pos + 1].cpu(), vc[:, : pos + 1], f"v cache pos={pos}")
        assert_parity(k_layer[:, : pos + 1].cpu(), kc[:, : pos + 1], f"k cache pos={pos}")


def test_attention_decode_forward_matches_oracle(gpu):
    """_semantic_qwen_attention_decode_forward (QKV GEMV, the attention kernel,
    o_proj GEMV) on a normalised hidden state, with a cache of the reference's
    shape [L, B, n_kv, S, d] whose cursor sits at row 5."""
    w, layer = _layer(9400)
    s_max, pos = 32, 5
    gen = torch.Generator().manual_seed(9401)
    kc = torch.randn((G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16)
    vc = torch.randn((G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16)
    cache = SimpleNamespace(key_cache=kc.clone().to(DEV)[None, None], value_cache=vc.clone().to(DEV)[None, None],
                            layer_seq_lens=[pos], max_layer_seq_len=pos)
    hidden = (torch.randn(G.hidden_size, generator=gen)).to(torch.bfloat16)
    cos, sin = _cos_sin(pos)
    got = dispatch._semantic_qwen_attention_decode_forward(layer.attention, hidden.to(DEV), cache,
                                                           (cos.to(DEV).view(1, 1, -1), sin.to(DEV).view(1, 1, -1)),
                                                           EPS)
    torch.cuda.synchronize()
    qkv = torch.mv(w["qkv"], hidden)
    attn, _, _ = ref_attn.decode_attention(qkv, G.num_attention_heads, G.num_key_value_heads, D, w["qn"], w["kn"], EPS,
                                           cos, sin, kc, vc, pos, D ** -0.5)
    assert_parity(got.cpu(), torch.mv(w["o"], attn), "attention decode forward")
    assert cache.layer_seq_lens == [pos + 1] and cache.max_layer_seq_len == pos + 1


def test_decode_step_two_layers_and_head(gpu):
    """stack.DecodeStep (graph-capturable whole token) over two layers at
    position 5 with a filled cache, against the oracle's layer chain and the
    greedy bf16-logit head; the replayed graph gives the same token."""
    from leanstack_amd.stack import DecodeStep, LayerProjections
    from oracle import projections as ref

    n_layers, s_max, pos = 2, 16, 5
    layers_cpu, layers = [], []
    for l in range(n_layers):
        w, layer = _layer(9500 + 10 * l)
        layers_cpu.append(w)
        layers.append(LayerProjections(layer.attention.qkv_proj_weight, layer.attention.o_proj_weight,
                                       layer.mlp.gate_up_proj_weight, layer.mlp.down_proj_weight))
    norms = torch.stack([torch.stack((w["in_ln"], w["post_ln"])) for w in layers_cpu])
    qk = torch.stack([torch.stack((w["qn"], w["kn"])) for w in layers_cpu])
    gen = torch.Generator().manual_seed(9599)
    final = (1 + 0.1 * torch.randn(G.hidden_size, generator=gen)).to(torch.bfloat16)
    lm_w = weight(G.vocab_size, G.hidden_size, seed=9598)
    kc = torch.randn((n_layers, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16)
    vc = torch.randn((n_layers, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16)
    hidden = (torch.randn(G.hidden_size, generator=gen) * 3).to(torch.bfloat16)
    step = DecodeStep(layers, norms.to(DEV), qk.to(DEV), final.to(DEV), PackedWeight.from_rowmajor(lm_w.to(DEV)), G,
                      kc.clone().to(DEV), vc.clone().to(DEV), DEV)
    step.hidden[0, 0] = hidden.to(DEV)
    step.launch(pos)
    torch.cuda.synchronize()
    h = hidden
    cos, sin = step.cos[pos].cpu(), step.sin[pos].cpu()
    for l, w in enumerate(layers_cpu):
        h, kl, vl = ref_attn.decode_layer(
            h, w["in_ln"], w["qkv"], G.num_attention_heads, G.num_key_value_heads, D, w["qn"], w["kn"], cos, sin,
            kc[l], vc[l], pos, D ** -0.5, w["o"], w["post_ln"], w["gate_up"], G.intermediate_size, w["down"], EPS)
        assert_parity(step.k_cache[l, :, : pos + 1].cpu(), kl[:, : pos + 1], f"layer {l} k cache")
    assert_parity(step.hidden[n_layers % 2, 0].cpu(), h, "hidden after two layers")
    scores = ref.logits_scores_fp32(ref.rmsnorm(h.view(1, -1), final, EPS), lm_w)
    got_scores = _gpu_scores(step.hidden[n_layers % 2], step.lm_head, step.final_norm)
    assert_greedy_rows(step.token.cpu(), scores, got_scores, "two-layer step")
    token = step.token.item()
    graph = torch.cuda.CUDAGraph()
    step.hidden[0, 0] = hidden.to(DEV)
    with torch.cuda.graph(graph):
        step.launch(pos)
    for _ in range(3):
        step.hidden[0, 0] = hidden.to(DEV)
        graph.replay()
        torch.cuda.synchronize()
        assert step.token.item() == token


def test_decode_step_one_graph_for_every_position(gpu):
    """DecodeStep.launch() with the position in device memory: one graph,
    captured once, replayed at positions 3, 4, 5 (set_position between
    replays, the output hidden fed back as the next input) gives the tokens,
    hidden states and caches of per-position eager launches, bit for bit."""
    from leanstack_amd.stack import DecodeStep, LayerProjections

    n_layers, s_max = 2, 200
    layers_cpu, layers = [], []
    for l in range(n_layers):
        w, layer = _layer(9700 + 10 * l)
        layers_cpu.append(w)
        layers.append(LayerProjections(layer.attention.qkv_proj_weight, layer.attention.o_proj_weight,
                                       layer.mlp.gate_up_proj_weight, layer.mlp.down_proj_weight))
    norms = torch.stack([torch.stack((w["in_ln"], w["post_ln"])) for w in layers_cpu]).to(DEV)
    qk = torch.stack([torch.stack((w["qn"], w["kn"])) for w in layers_cpu]).to(DEV)
    gen = torch.Generator().manual_seed(9799)
    final = (1 + 0.1 * torch.randn(G.hidden_size, generator=gen)).to(torch.bfloat16).to(DEV)
    lm = PackedWeight.from_rowmajor(weight(G.vocab_size, G.hidden_size, seed=9798).to(DEV))
    kc = torch.randn((n_layers, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((n_layers, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16).to(DEV)
    hidden = (torch.randn(G.hidden_size, generator=gen) * 3).to(torch.bfloat16).to(DEV)
    eager = DecodeStep(layers, norms, qk, final, lm, G, kc.clone(), vc.clone(), DEV)
    graphed = DecodeStep(layers, norms, qk, final, lm, G, kc.clone(), vc.clone(), DEV)
    graphed.set_position(3)
    graphed.hidden[0, 0] = hidden
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graphed.launch()
    # capture ran nothing: reset what the graph will write, then replay per position
    graphed.k_cache.copy_(kc)
    graphed.v_cache.copy_(vc)
    h_eager = h_graph = hidden
    for pos in (3, 4, 5):
        eager.hidden[0, 0] = h_eager
        eager.launch(pos)
        graphed.hidden[0, 0] = h_graph
        graphed.set_position(pos)
        graph.replay()
        torch.cuda.synchronize()
        out_e, out_g = eager.hidden[n_layers % 2, 0].clone(), graphed.hidden[n_layers % 2, 0].clone()
        assert _same_bits(out_e, out_g), f"pos {pos}: hidden differs"
        assert eager.token.item() == graphed.token.item(), f"pos {pos}: token differs"
        h_eager, h_graph = out_e, out_g
    assert _same_bits(eager.k_cache, graphed.k_cache) and _same_bits(eager.v_cache, graphed.v_cache)
    with pytest.raises(ValueError):
        graphed.set_position(s_max)


def test_decode_step_greedy_loop_in_one_graph(gpu):
    """DecodeStep.launch_next captured once: four replays generate the same
    tokens, caches and positions as four eager steps driven from the host
    (embedding lookup, launch(pos), token read back)."""
    from leanstack_amd.stack import DecodeStep, LayerProjections

    n_layers, s_max, start = 2, 64, 7
    layers_cpu, layers = [], []
    for l in range(n_layers):
        w, layer = _layer(9800 + 10 * l)
        layers_cpu.append(w)
        layers.append(LayerProjections(layer.attention.qkv_proj_weight, layer.attention.o_proj_weight,
                                       layer.mlp.gate_up_proj_weight, layer.mlp.down_proj_weight))
    norms = torch.stack([torch.stack((w["in_ln"], w["post_ln"])) for w in layers_cpu]).to(DEV)
    qk = torch.stack([torch.stack((w["qn"], w["kn"])) for w in layers_cpu]).to(DEV)
    gen = torch.Generator().manual_seed(9899)
    final = (1 + 0.1 * torch.randn(G.hidden_size, generator=gen)).to(torch.bfloat16).to(DEV)
    emb = weight(G.vocab_size, G.hidden_size, seed=9897).to(DEV)  # untied, so the tokens change
    lm = PackedWeight.from_rowmajor(weight(G.vocab_size, G.hidden_size, seed=9898).to(DEV))
    kc = torch.randn((n_layers, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16).to(DEV)
    vc = torch.randn((n_layers, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16).to(DEV)
    first = 1234

    eager = DecodeStep(layers, norms, qk, final, lm, G, kc.clone(), vc.clone(), DEV)
    token, expect = first, []
    for pos in range(start, start + 4):
        eager.hidden[0, 0] = emb[token]
        eager.launch(pos)
        token = eager.token.item()
        expect.append(token)

    looped = DecodeStep(layers, norms, qk, final, lm, G, kc.clone(), vc.clone(), DEV)
    tokens = torch.full((s_max,), -1, dtype=torch.long, device=DEV)
    looped.token.fill_(first)
    looped.set_position(start)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        looped.launch_next(emb, tokens)
    for _ in range(4):
        graph.replay()
    torch.cuda.synchronize()
    assert tokens[start:start + 4].tolist() == expect, (tokens[start:start + 4].tolist(), expect)
    assert int(looped.pos_dev.item()) == start + 4
    assert _same_bits(eager.k_cache, looped.k_cache) and _same_bits(eager.v_cache, looped.v_cache)
    assert expect != [first] * 4  # the loop moved on from its first token


def _gpu_scores(hidden, lm_head, final_norm):
    """The fp32 scores DecodeStep's fused head (final RMSNorm, fp32 scores)
    compares for `hidden` ([1, H] on the GPU), on the CPU."""
    scores = torch.empty((1, lm_head.n), device=DEV, dtype=torch.float32)
    kernels.lm_head_argmax(hidden.reshape(1, -1), lm_head, logits_mode=_lib.LOGITS_FP32, logits_out=scores,
                           norm_weight=final_norm, eps=EPS)
    torch.cuda.synchronize()
    return scores.cpu()


def test_one_layer_greedy_decode_matches_oracle_token_by_token(gpu):
    """A one-layer greedy decode of six tokens through DecodeStep.launch_next
    (embedding gather, the layer's five kernels, the fused head, token
    record, position advance), checked after every token against the
    oracle's decode layer (qwen_explicit.py:1247-1272) and the default greedy
    head (final RMSNorm, fp32 scores, first maximum: :1798-1832 with
    cutile_logits.py:17-69) on the same caches: the hidden state and the
    cache rows at the parity bar, the token equal wherever the oracle's score
    margin exceeds twice the largest score difference (assert_greedy_rows),
    else one of the oracle's near-maximal tokens."""
    from leanstack_amd.stack import DecodeStep, LayerProjections
    from oracle import projections as ref

    s_max, start, steps = 64, 9, 6
    w, layer = _layer(9900)
    layers = [LayerProjections(layer.attention.qkv_proj_weight, layer.attention.o_proj_weight,
                               layer.mlp.gate_up_proj_weight, layer.mlp.down_proj_weight)]
    norms = torch.stack((w["in_ln"], w["post_ln"]))[None]
    qk = torch.stack((w["qn"], w["kn"]))[None]
    gen = torch.Generator().manual_seed(9999)
    final = (1 + 0.1 * torch.randn(G.hidden_size, generator=gen)).to(torch.bfloat16)
    emb = (torch.randn((G.vocab_size, G.hidden_size), generator=gen) * 2).to(torch.bfloat16)  # untied
    lm_w = weight(G.vocab_size, G.hidden_size, seed=9998)
    kc = torch.randn((1, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16)
    vc = torch.randn((1, G.num_key_value_heads, s_max, D), generator=gen).to(torch.bfloat16)
    step = DecodeStep(layers, norms.to(DEV), qk.to(DEV), final.to(DEV), PackedWeight.from_rowmajor(lm_w.to(DEV)), G,
                      kc.clone().to(DEV), vc.clone().to(DEV), DEV)
    emb_dev = emb.to(DEV)
    tokens = torch.full((s_max,), -1, dtype=torch.long, device=DEV)
    token = 4321
    step.token.fill_(token)
    step.set_position(start)
    k_ref, v_ref = kc[0].clone(), vc[0].clone()
    exact = exact_own = 0
    margins = []
    for i in range(steps):
        pos = start + i
        step.launch_next(emb_dev, tokens)
        torch.cuda.synchronize()
        cos, sin = step.cos[pos].cpu(), step.sin[pos].cpu()
        h, k_ref, v_ref = ref_attn.decode_layer(
            emb[token], w["in_ln"], w["qkv"], G.num_attention_heads, G.num_key_value_heads, D, w["qn"], w["kn"], cos,
            sin, k_ref, v_ref, pos, D ** -0.5, w["o"], w["post_ln"], w["gate_up"], G.intermediate_size, w["down"],
            EPS)
        assert_parity(step.hidden[1, 0].cpu(), h, f"token {i}: hidden")
        assert_parity(step.k_cache[0, :, pos].cpu(), k_ref[:, pos], f"token {i}: k row")
        assert_parity(step.v_cache[0, :, pos].cpu(), v_ref[:, pos], f"token {i}: v row")
        scores = ref.logits_scores_fp32(ref.rmsnorm(h.view(1, -1), final, EPS), lm_w)
        got = int(tokens[pos].item())
        assert got == int(step.token.item())
        gpu_scores = _gpu_scores(step.hidden[1], step.lm_head, step.final_norm)
        assert_greedy_rows(torch.tensor([got]), scores, gpu_scores, f"token {i}")
        exact += got == int(scores.argmax())
        # The oracle's head on the GPU's own hidden state: the same input, so
        # only the norm's multiplication order and the fp32 summation order
        # differ (|score difference| <= delta_own); the token must be the
        # oracle's argmax exactly unless its top-2 margin is inside that.
        own = ref.logits_scores_fp32(ref.rmsnorm(step.hidden[1].cpu().view(1, -1), final, EPS), lm_w).view(-1)
        delta_own = float((gpu_scores.view(-1) - own).abs().max())
        top = torch.topk(own, 2)
        margin_own = float(top.values[0] - top.values[1])
        margins.append(margin_own)
        assert got == int(top.indices[0]) or margin_own <= 2 * delta_own, (
            f"token {i}: {got} != oracle argmax {int(top.indices[0])} on the GPU's hidden state "
            f"(margin {margin_own:.3g}, delta {delta_own:.3g})")
        exact_own += got == int(top.indices[0])
        token = got  # the oracle follows the decode's own tokens
    assert int(step.pos_dev.item()) == start + steps
    assert exact_own == steps, (f"{exact_own} of {steps} tokens equal the oracle's argmax on the GPU's hidden state "
                                f"(top-2 margins {margins})")
    assert exact >= steps - 1, f"{exact} of {steps} tokens equal the oracle's argmax on the oracle's hidden state"
    print(f"{exact} of {steps} tokens equal to the oracle's argmax on the oracle's hidden state, "
          f"{exact_own} of {steps} on the GPU's own hidden state")
