"""The 36-layer decode projection step that the benchmark times, against the
oracle.

The step (DecodeLinearStack.launch: per layer fused QKV, o_proj, fused
gate_up + SiLU*up, down_proj, 144 launches) is built exactly as the bench
builds it -- 36 distinct random N(0, 0.02) layers packed into one resident
arena, fresh N(0, 1) inputs per layer -- captured as one HIP graph and
replayed.  Every layer writes the same output buffers, so after a replay
they hold the last layer's projections, and down_proj reads the activation
that layer's gate_up kernel wrote: the oracle recomputes that layer (and
layers 0, 1, 17 and 34, through one-layer graphs of the same arena) from the
CPU copies of their weights at the parity bar.  The graph's outputs also equal an eager launch of the same
sequence bit for bit.  The reference's callers are run_semantic_stack_decode /
run_semantic_stack_verify_from_hidden (src/leanstack/runtime/
qwen_explicit.py:1617-1644, :1676-1716).
"""

from __future__ import annotations

import pytest
import torch

from leanstack_amd import _lib
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.leanserve import ResidentArena, build_resident_buffer_plan, layer_entry_names
from leanstack_amd.stack import DecodeLinearStack, LayerProjections
from oracle import projections as ref
from tests.helpers import assert_parity

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
# layers checked through one-layer graphs of the arena (the full step's
# outputs hold only the last layer's)
CHECKED_LAYERS = (0, 1, 17, 34)


@pytest.fixture(scope="module")
def stack36(gpu):
    """The bench's 36-layer arena, with CPU copies of layers 0, 1, 17, 34
    and 35."""
    plan = build_resident_buffer_plan(G, max_rows=16, include_embedding=False, include_lm_head=False, buckets=())
    arena = ResidentArena(plan, DEV)
    gen = torch.Generator(device=DEV).manual_seed(0)
    layers, cpu = [], {}
    last = G.num_hidden_layers - 1
    for l in range(G.num_hidden_layers):
        names = layer_entry_names(l)
        for proj, (n, k) in G.projections().items():
            w = (torch.randn((n, k), generator=gen, device=DEV) * 0.02).to(torch.bfloat16)
            arena.store_rowmajor(names[proj], w)
            if l in CHECKED_LAYERS + (last,):
                cpu[(l, proj)] = w.cpu()
            del w
        layers.append(LayerProjections(arena.packed(names["qkv_proj"]), arena.packed(names["o_proj"]),
                                       arena.packed(names["gate_up_proj"]), arena.packed(names["down_proj"])))
    stack = DecodeLinearStack(layers, G, max_rows=8, device=DEV)
    torch.cuda.synchronize()
    yield stack, cpu
    del stack, arena
    torch.cuda.empty_cache()


def _outputs(stack, m):
    return [t[:m].clone() for t in (stack.y_qkv, stack.y_o, stack.act, stack.y_down)]


def _check_layer(stack, cpu, layer, m, got, what):
    x_qkv, x_o, x_gu = (t[layer, :m].cpu() for t in (stack.x_qkv, stack.x_o, stack.x_gu))
    y_qkv = ref.linear(x_qkv, cpu[(layer, "qkv_proj")])
    y_o = ref.linear(x_o, cpu[(layer, "o_proj")])
    act = ref.silu_mul(ref.linear(x_gu, cpu[(layer, "gate_up_proj")]), G.intermediate_size)
    names = ("qkv", "o", "act", "down")
    for name, g, e in zip(names[:3], got[:3], (y_qkv, y_o, act)):
        assert_parity(g.cpu(), e, f"{what} layer {layer} M={m} {name}")
    # down reads the activation the GPU wrote; checked from that input and
    # from the oracle's own activation
    assert_parity(got[3].cpu(), ref.linear(got[2].cpu(), cpu[(layer, "down_proj")]), f"{what} layer {layer} down")
    assert_parity(got[3].cpu(), ref.linear(act, cpu[(layer, "down_proj")]), f"{what} layer {layer} down (oracle act)")


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_36_layer_graph_matches_oracle(stack36, m):
    stack, cpu = stack36
    for t in (stack.y_qkv, stack.y_o, stack.act, stack.y_down):
        t.fill_(float("nan"))
    graph = stack.capture(lambda: stack.launch(m))
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    got = _outputs(stack, m)
    _check_layer(stack, cpu, G.num_hidden_layers - 1, m, got, "graph")
    del graph
    # eager launches of the same 144 projections give the same bits
    for t in (stack.y_qkv, stack.y_o, stack.act, stack.y_down):
        t.fill_(float("nan"))
    stack.launch(m)
    torch.cuda.synchronize()
    for g, e in zip(got, _outputs(stack, m)):
        assert torch.equal(g.view(torch.int16), e.view(torch.int16))


@pytest.mark.parametrize("layer", CHECKED_LAYERS)
def test_single_layers_of_the_stack(stack36, layer):
    """Layers 0, 1, 17 and 34 through one-layer graphs of the same launches
    on the same arena (their outputs are overwritten by the later layers in
    the full step): every layer's arena views and kernels, not only the
    last one's, meet the oracle."""
    stack, cpu = stack36
    m = 4
    for t in (stack.y_qkv, stack.y_o, stack.act, stack.y_down):
        t.fill_(float("nan"))
    graph = stack.capture(lambda: stack.launch(m, range(layer, layer + 1)))
    graph.replay()
    torch.cuda.synchronize()
    _check_layer(stack, cpu, layer, m, _outputs(stack, m), "one-layer graph")
    assert stack.layers[layer].gate_up.layout == _lib.LAYOUT_MFMA16X32_GATEUP


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("m", [1, 8])
def test_36_layer_graph_with_rmsnorms_matches_oracle(stack36, m, fused):
    """The step with the two RMSNorms of each layer (input_layernorm in front
    of QKV, post_attention_layernorm in front of gate_up,
    qwen_explicit.py:1255 and :941), fused into those kernels or run as
    F.rms_norm launches, captured as one graph: the last layer's outputs
    against the oracle's norm then projection."""
    stack, cpu = stack36
    for t in (stack.y_qkv, stack.y_o, stack.act, stack.y_down):
        t.fill_(float("nan"))
    graph = stack.capture(lambda: stack.launch_with_norms(m, fused))
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    got = _outputs(stack, m)
    del graph
    layer = G.num_hidden_layers - 1
    ln_in, ln_post = (stack.norm_w[layer, i].cpu() for i in (0, 1))
    x_qkv, x_o, x_gu = (t[layer, :m].cpu() for t in (stack.x_qkv, stack.x_o, stack.x_gu))
    y_qkv = ref.linear(ref.rmsnorm(x_qkv, ln_in, stack.eps), cpu[(layer, "qkv_proj")])
    y_o = ref.linear(x_o, cpu[(layer, "o_proj")])
    act = ref.silu_mul(ref.linear(ref.rmsnorm(x_gu, ln_post, stack.eps), cpu[(layer, "gate_up_proj")]),
                       G.intermediate_size)
    what = f"{'fused' if fused else 'separate'} norms, layer {layer} M={m}"
    for name, g, e in zip(("qkv", "o", "act"), got[:3], (y_qkv, y_o, act)):
        assert_parity(g.cpu(), e, f"{what} {name}")
    assert_parity(got[3].cpu(), ref.linear(act, cpu[(layer, "down_proj")]), f"{what} down")


@pytest.mark.parametrize("m", [1, 2, 4, 8])
def test_36_layer_persistent_step_matches_oracle(stack36, m):
    """The same 144-projection step as one persistent launch (the chained
    stack program the bench also times): no wait gives up, and the last
    layer's outputs meet the oracle (the persistent kernel sums in another
    order than the launch kernels, so parity, not bit equality, is the bar)."""
    stack, cpu = stack36
    for t in (stack.y_qkv, stack.y_o, stack.act, stack.y_down):
        t.fill_(float("nan"))
    step = stack.persistent_step(m, chain=True)
    step.launch()
    torch.cuda.synchronize()
    assert step.error() == 0
    _check_layer(stack, cpu, G.num_hidden_layers - 1, m, _outputs(stack, m), "persistent")
    del step
