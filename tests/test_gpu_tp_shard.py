"""One GPU's share of 8-way tensor parallelism, at the real Qwen3-4B shard
shapes, against the oracle: QKV split by output rows (4 q heads + 1 kv head,
768 x 2560), o_proj by its K (2560 x 512), gate_up by output rows keeping the
gate/up pairing (2 x 1216 x 2560, SiLU*up), down by its K (2560 x 1216), and
the tied lm_head by vocab (18992 x 2560: 1187 row-blocks, an odd count).  A
shard runs the same C ABI entry points as the whole projection; the o_proj
and down shards yield the partial sums an all-reduce would add, so they take
no residual here.  Same bar as the full shapes: cosine >= 0.9999 and normwise
max relative error <= 1e-2 for bf16 outputs, greedy tokens by
assert_greedy_rows."""

from __future__ import annotations

import pytest
import torch

from leanstack_amd import _lib, kernels
from leanstack_amd.geometry import QWEN3_4B as G
from leanstack_amd.layout import PackedWeight
from oracle import projections as ref
from tests.helpers import activations, assert_greedy_rows, assert_parity, weight

pytestmark = pytest.mark.gpu

TP = 8
SHARDS = {
    "qkv_proj": (G.qkv_dim // TP, G.hidden_size),  # 768 x 2560
    "o_proj": (G.hidden_size, G.q_dim // TP),  # 2560 x 512
    "down_proj": (G.hidden_size, G.intermediate_size // TP),  # 2560 x 1216
}
GATE_SHARD = G.intermediate_size // TP  # 1216 gate rows and 1216 up rows
VOCAB_SHARD = G.vocab_size // TP  # 18992


def _gpu_linear(x, w, layout=_lib.LAYOUT_MFMA16X32, epilogue=_lib.EPI_NONE):
    dev = torch.device("cuda:0")
    pw = PackedWeight.from_rowmajor(w.to(dev), layout)
    y = kernels.linear(x.to(dev), pw, epilogue=epilogue)
    torch.cuda.synchronize()
    return y.cpu()


def test_shard_geometry():
    assert SHARDS == {"qkv_proj": (768, 2560), "o_proj": (2560, 512), "down_proj": (2560, 1216)}
    assert (GATE_SHARD, VOCAB_SHARD, VOCAB_SHARD // 16, VOCAB_SHARD % 32) == (1216, 18992, 1187, 16)


@pytest.mark.parametrize("name", sorted(SHARDS))
@pytest.mark.parametrize("m", [1, 4, 8, 64, 2048])
def test_shard_projection(gpu, name, m):
    """Decode (M = 1, 4, 8), the 17..128-row kernel (64) and the prefill GEMM
    (2048 tokens, with its split-K workspace) on each shard."""
    n, k = SHARDS[name]
    w = weight(n, k, seed=300 + n % 89 + k % 83)
    x = activations(m, k, seed=3000 + m)
    print(f"case {name} shard {n}x{k} M={m}", flush=True)
    assert_parity(_gpu_linear(x, w), ref.linear(x, w), f"{name} shard M={m}")


@pytest.mark.parametrize("m", [1, 4, 8, 64, 2048])
def test_shard_gate_up_silu(gpu, m):
    n, k = 2 * GATE_SHARD, G.hidden_size
    w = weight(n, k, seed=310)
    x = activations(m, k, seed=3100 + m)
    print(f"case gate_up shard {n}x{k} M={m}", flush=True)
    y = _gpu_linear(x, w, _lib.LAYOUT_MFMA16X32_GATEUP, _lib.EPI_SILU_MUL)
    assert_parity(y, ref.silu_mul(ref.linear(x, w), GATE_SHARD), f"gate_up+silu shard M={m}")


@pytest.mark.parametrize("m", [1, 4])
def test_shard_lm_head(gpu, m):
    """The vocab shard's greedy head (337 pairs of row-blocks, then 513
    single ones): fp32 scores against the oracle's, tokens by the margin
    rule, and a maximum planted in the last row found exactly."""
    dev = torch.device("cuda:0")
    v, k = VOCAB_SHARD, G.hidden_size
    e = weight(v, k, seed=320)
    h = activations(m, k, seed=3200 + m)
    pw = PackedWeight.from_rowmajor(e.to(dev))
    logits = torch.empty((m, v), device=dev, dtype=torch.float32)
    print(f"case lm_head shard {v}x{k} M={m}", flush=True)
    idx = kernels.lm_head_argmax(h.to(dev), pw, logits_out=logits).cpu()
    expect = ref.logits_scores_fp32(h, e)
    got = logits.cpu()
    assert_parity(got, expect, f"lm_head shard logits M={m}")
    assert_greedy_rows(idx, expect, got, f"lm_head shard M={m}")
    e[v - 1] = torch.sign(h[0].float()).to(torch.bfloat16) * 0.5
    pw = PackedWeight.from_rowmajor(e.to(dev))
    assert kernels.lm_head_argmax(h[:1].to(dev), pw).cpu().tolist() == [v - 1]


def test_shard_lm_head_with_final_norm(gpu):
    """The fused final RMSNorm + head on the vocab shard against the oracle's
    greedy head (bf16 logits of the normalised row, first maximum), by the
    margin rule: bf16 logits tie often over 18992 rows."""
    dev = torch.device("cuda:0")
    v, k = VOCAB_SHARD, G.hidden_size
    e = weight(v, k, seed=330)
    h = activations(1, k, seed=3300)
    gen = torch.Generator(device="cpu").manual_seed(331)
    nw = (1.0 + 0.1 * torch.randn(k, generator=gen)).to(torch.bfloat16)
    pw = PackedWeight.from_rowmajor(e.to(dev))
    logits = torch.empty((1, v), device=dev, dtype=torch.float32)
    idx = kernels.lm_head_argmax(h.to(dev), pw, logits_mode=_lib.LOGITS_BF16, logits_out=logits,
                                 norm_weight=nw.to(dev), eps=G.rms_norm_eps).cpu()
    hn = ref.rmsnorm(h, nw, G.rms_norm_eps)
    expect = ref.logits_scores_fp32(hn, e).to(torch.bfloat16).float()
    assert_greedy_rows(idx, expect, logits.cpu(), "lm_head shard with final norm")
