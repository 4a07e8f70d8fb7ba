"""The decode step's projection sequence over all resident layers.

Per layer, in the reference's call order (src/leanstack/runtime/qwen_explicit.py:
1247-1272 for M = 1, :1211-1244 for the verify batch), the step runs the fused
QKV projection, o_proj, the fused gate_up with SiLU(gate)*up and down_proj.
The RMSNorm / q-k norm / RoPE / attention work between them is not part of
this path; each projection reads a fixed input buffer instead (its "fresh"
activations), so the stack measures exactly the projection traffic of a
decode step.  All launches go to one stream in dependency order, and the
whole step can be captured once as a HIP graph and replayed, which takes
host launch cost out of the step time.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib, kernels
from .geometry import QwenGeometry
from .layout import PackedWeight


@dataclass
class LayerProjections:
    qkv: PackedWeight
    o: PackedWeight
    gate_up: PackedWeight
    down: PackedWeight


class DecodeLinearStack:
    def __init__(self, layers: list[LayerProjections], geometry: QwenGeometry, max_rows: int,
                 device: torch.device, inputs: dict[str, torch.Tensor] | None = None) -> None:
        if not 1 <= max_rows <= 16:
            raise ValueError("the decode stack serves M = 1..16 rows")
        self.layers = layers
        self.g = geometry
        self.max_rows = max_rows
        self.device = device
        n = len(layers)
        h, q, i, qkv = geometry.hidden_size, geometry.q_dim, geometry.intermediate_size, geometry.qkv_dim
        if inputs is None:
            gen = torch.Generator(device=device).manual_seed(1)
            inputs = {
                "qkv": torch.randn((n, max_rows, h), generator=gen, device=device).to(torch.bfloat16),
                "o": torch.randn((n, max_rows, q), generator=gen, device=device).to(torch.bfloat16),
                "gate_up": torch.randn((n, max_rows, h), generator=gen, device=device).to(torch.bfloat16),
            }
        self.x_qkv, self.x_o, self.x_gu = inputs["qkv"], inputs["o"], inputs["gate_up"]
        # input_layernorm / post_attention_layernorm weights of each layer
        # (for the step with its RMSNorms, launch_with_norms)
        gen_n = torch.Generator(device=device).manual_seed(2)
        self.norm_w = (1.0 + 0.1 * torch.randn((n, 2, h), generator=gen_n, device=device)).to(torch.bfloat16)
        self.eps = geometry.rms_norm_eps
        self.y_qkv = torch.empty((max_rows, qkv), device=device, dtype=torch.bfloat16)
        self.y_o = torch.empty((max_rows, h), device=device, dtype=torch.bfloat16)
        self.act = torch.empty((max_rows, i), device=device, dtype=torch.bfloat16)
        self.y_down = torch.empty((max_rows, h), device=device, dtype=torch.bfloat16)

    def launch(self, m: int, layers: range | None = None) -> None:
        """Enqueue one step (all layers, or `layers`) at M = m rows."""
        if not 1 <= m <= self.max_rows:
            raise ValueError(f"m={m} outside 1..{self.max_rows}")
        for l in layers if layers is not None else range(len(self.layers)):
            p = self.layers[l]
            kernels.linear(self.x_qkv[l, :m], p.qkv, out=self.y_qkv[:m])
            kernels.linear(self.x_o[l, :m], p.o, out=self.y_o[:m])
            kernels.linear(self.x_gu[l, :m], p.gate_up, epilogue=_lib.EPI_SILU_MUL, out=self.act[:m])
            kernels.linear(self.act[:m], p.down, out=self.y_down[:m])

    def launch_with_norms(self, m: int, fused: bool) -> None:
        """The step with the two RMSNorms of each layer in front of QKV
        (input_layernorm, qwen_explicit.py:1255) and gate_up
        (post_attention_layernorm, :941): inside those projections' kernels
        when `fused`, else as F.rms_norm launches ahead of them."""
        if not 1 <= m <= self.max_rows:
            raise ValueError(f"m={m} outside 1..{self.max_rows}")
        h = self.g.hidden_size
        for l, p in enumerate(self.layers):
            ln_in, ln_post = self.norm_w[l, 0], self.norm_w[l, 1]
            if fused:
                kernels.rmsnorm_linear(self.x_qkv[l, :m], ln_in, self.eps, p.qkv, out=self.y_qkv[:m])
            else:
                normed = torch.nn.functional.rms_norm(self.x_qkv[l, :m], (h,), ln_in, self.eps)
                kernels.linear(normed, p.qkv, out=self.y_qkv[:m])
            kernels.linear(self.x_o[l, :m], p.o, out=self.y_o[:m])
            if fused:
                kernels.rmsnorm_linear(self.x_gu[l, :m], ln_post, self.eps, p.gate_up, epilogue=_lib.EPI_SILU_MUL,
                                       out=self.act[:m])
            else:
                normed = torch.nn.functional.rms_norm(self.x_gu[l, :m], (h,), ln_post, self.eps)
                kernels.linear(normed, p.gate_up, epilogue=_lib.EPI_SILU_MUL, out=self.act[:m])
            kernels.linear(self.act[:m], p.down, out=self.y_down[:m])

    def launch_projection(self, name: str, m: int) -> None:
        """Enqueue one projection kind across all layers (per-kernel timing)."""
        for l, p in enumerate(self.layers):
            if name == "qkv_proj":
                kernels.linear(self.x_qkv[l, :m], p.qkv, out=self.y_qkv[:m])
            elif name == "o_proj":
                kernels.linear(self.x_o[l, :m], p.o, out=self.y_o[:m])
            elif name == "gate_up_proj":
                kernels.linear(self.x_gu[l, :m], p.gate_up, epilogue=_lib.EPI_SILU_MUL, out=self.act[:m])
            elif name == "down_proj":
                kernels.linear(self.act[:m], p.down, out=self.y_down[:m])
            else:
                raise ValueError(name)

    def persistent_step(self, m: int, chain: bool = True) -> kernels.StackStep:
        """The same step as launch(m) as one persistent-kernel program.  With
        `chain`, every projection waits for all earlier ones (the decode
        step's dependency chain: each projection's input is produced from the
        previous one's output); weights still stream ahead of the waits."""
        specs = []
        for l, p in enumerate(self.layers):
            base = len(specs)
            dep = (lambda i: i - 1) if chain else (lambda i: -1)
            specs.append({"x": self.x_qkv[l, :m], "weight": p.qkv, "out": self.y_qkv[:m], "depends_on": dep(base)})
            specs.append({"x": self.x_o[l, :m], "weight": p.o, "out": self.y_o[:m], "depends_on": dep(base + 1)})
            specs.append({"x": self.x_gu[l, :m], "weight": p.gate_up, "out": self.act[:m],
                          "epilogue": _lib.EPI_SILU_MUL, "depends_on": dep(base + 2)})
            specs.append({"x": self.act[:m], "weight": p.down, "out": self.y_down[:m], "depends_on": base + 2})
        return kernels.StackStep(specs, m, self.device)

    def capture(self, fn) -> torch.cuda.CUDAGraph:
        """Capture `fn()` (a launch sequence) as a HIP graph.  The warm-up
        run and the capture use the stack's own capture stream, so workspaces
        that kernels.linear keeps per (device, stream) exist before the
        capture and no other work shares them."""
        if getattr(self, "_capture_stream", None) is None:
            self._capture_stream = torch.cuda.Stream(device=self.device)
        side = self._capture_stream
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            fn()  # warm the launch path outside capture
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            fn()
        torch.cuda.synchronize(self.device)
        return graph


class DecodeStep:
    """One whole decode token (M = 1) over every layer, in the reference's
    order (semantic_qwen_decode_layer_forward, qwen_explicit.py:1247-1272,
    then the greedy head, :1798-1832): per layer input_layernorm + QKV, the
    attention kernel (q/k norms, RoPE, cache append, GQA attention), o_proj
    + residual, post_attention_layernorm + gate_up + SiLU*up, down +
    residual; then the final RMSNorm and the lm_head argmax.  All buffers are
    fixed, so the launch sequence can be captured as one HIP graph.
    launch(pos) bakes the position into the launches; launch() reads it from
    the device (self.pos_dev, set with set_position), so one captured graph
    serves every token of a sequence.

    norms: [n, 2, H] (input / post-attention), qk_norms: [n, 2, d] (q / k),
    k_cache / v_cache: [n, n_kv, max_seq_len, d]."""

    def __init__(self, layers: list[LayerProjections], norms: torch.Tensor, qk_norms: torch.Tensor,
                 final_norm: torch.Tensor, lm_head: PackedWeight, geometry: QwenGeometry, k_cache: torch.Tensor,
                 v_cache: torch.Tensor, device: torch.device, logits_mode: int = _lib.LOGITS_FP32) -> None:
        g = geometry
        # The head compares fp32 scores by default, as the reference's decode
        # loop does with its default "auto" backend (select_semantic_greedy_token
        # -> the cuTile head, qwen_explicit.py:1798-1832); LOGITS_BF16 is the
        # torch.mv head of _semantic_greedy_head_vector (:952-960).
        self.logits_mode = logits_mode
        self.layers, self.norms, self.qk_norms, self.final_norm, self.lm_head = layers, norms, qk_norms, final_norm, \
            lm_head
        self.g, self.k_cache, self.v_cache, self.device = g, k_cache, v_cache, device
        self.eps = g.rms_norm_eps
        self.scale = g.head_dim ** -0.5
        max_seq = k_cache.shape[2]
        inv = 1.0 / (g.rope_theta ** (torch.arange(0, g.head_dim, 2, device=device, dtype=torch.float32) / g.head_dim))
        freqs = torch.outer(torch.arange(max_seq, device=device, dtype=torch.float32), inv)
        # the reference's position cache (build_qwen_position_cache, qwen_explicit.py:664-676)
        self.cos, self.sin = freqs.cos().to(torch.bfloat16), freqs.sin().to(torch.bfloat16)
        h = g.hidden_size
        self.hidden = torch.zeros((2, 1, h), device=device, dtype=torch.bfloat16)  # ping-pong residual stream
        self.mid = torch.empty((1, h), device=device, dtype=torch.bfloat16)
        self.qkv = torch.empty((1, g.qkv_dim), device=device, dtype=torch.bfloat16)
        self.attn = torch.empty((g.q_dim,), device=device, dtype=torch.bfloat16)
        self.act = torch.empty((1, g.intermediate_size), device=device, dtype=torch.bfloat16)
        self.head_ws = kernels.LmHeadWorkspace(1, lm_head.n, lm_head.k, device)
        ws_bytes = _lib.load().lsk_attention_workspace_bytes(g.num_attention_heads, g.num_key_value_heads,
                                                               g.head_dim, max_seq)
        self.attn_ws = torch.zeros(ws_bytes, device=device, dtype=torch.uint8)  # left zeroed by every launch
        self.token = torch.zeros((1,), device=device, dtype=torch.long)
        self.pos_dev = torch.zeros((1,), device=device, dtype=torch.int32)
        # device-side indices of launch_next, clamped into their tables
        self._row = torch.zeros((1,), device=device, dtype=torch.long)
        self._slot = torch.zeros((1,), device=device, dtype=torch.long)

    def set_position(self, pos: int) -> None:
        """Write the position launch() reads, ordered on the current stream
        before whatever is enqueued next (a graph replay included)."""
        if not 0 <= pos < self.k_cache.shape[2]:
            raise ValueError(f"pos={pos} outside 0..{self.k_cache.shape[2] - 1}")
        self.pos_dev.fill_(pos)

    def launch_next(self, embedding: torch.Tensor, tokens_out: torch.Tensor | None = None) -> None:
        """One greedy decode step with no host work, for a graph captured once
        and replayed per token (the loop of qwen_explicit_runtime_loop.py:
        339-352 without its per-token dispatch): the embedding row of
        self.token becomes the input, the token at position self.pos_dev is
        computed (tokens_out[pos] = the new token, when given), and the
        position advances by one.  embedding: [V, H] bf16 (the tied lm_head's
        row-major copy serves).

        Replay bound: a sequence has max_seq_len positions.  Replays past the
        last one leave every cache untouched (the attention kernel ignores a
        position outside the cache) and write their token to the last slot of
        tokens_out; the device indices are clamped, so no replay reads or
        writes outside the embedding table or tokens_out.  The argmax kernels
        always return a valid vocab row (NaN and -inf scores included)."""
        if embedding.dim() != 2 or embedding.shape[1] != self.g.hidden_size or embedding.dtype != torch.bfloat16:
            raise ValueError(f"embedding must be a bfloat16 [V, {self.g.hidden_size}] tensor")
        if tokens_out is not None and (tokens_out.dtype != torch.long or tokens_out.dim() != 1
                                       or tokens_out.numel() < 1 or tokens_out.device != self.pos_dev.device):
            raise ValueError("tokens_out must be a 1-D int64 tensor on the step's device")
        torch.clamp(self.token, 0, embedding.shape[0] - 1, out=self._row)
        torch.index_select(embedding, 0, self._row, out=self.hidden[0])
        self.launch()
        if tokens_out is not None:
            self._slot.copy_(self.pos_dev)
            self._slot.clamp_(0, tokens_out.numel() - 1)
            tokens_out.index_copy_(0, self._slot, self.token)
        self.pos_dev.add_(1)

    def launch(self, pos: int | None = None) -> None:
        """Enqueue the token at position `pos` (rows 0..pos-1 of every layer's
        cache are the context), or, with pos None, at the position in
        self.pos_dev; its input is self.hidden[0], its output token
        self.token."""
        g = self.g
        if pos is None:
            cos, sin, where = self.cos, self.sin, self.pos_dev
        else:
            cos, sin, where = self.cos[pos], self.sin[pos], pos
        for l, p in enumerate(self.layers):
            x, y = self.hidden[l % 2], self.hidden[(l + 1) % 2]
            kernels.rmsnorm_linear(x, self.norms[l, 0], self.eps, p.qkv, out=self.qkv)
            kernels.decode_attention(self.qkv, self.qk_norms[l, 0], self.qk_norms[l, 1], self.eps, cos, sin,
                                     self.k_cache[l], self.v_cache[l], where, self.scale,
                                     num_attention_heads=g.num_attention_heads,
                                     num_key_value_heads=g.num_key_value_heads, out=self.attn,
                                     workspace=self.attn_ws)
            kernels.linear(self.attn.view(1, -1), p.o, epilogue=_lib.EPI_RESIDUAL_ADD, residual=x, out=self.mid)
            kernels.rmsnorm_linear(self.mid, self.norms[l, 1], self.eps, p.gate_up, epilogue=_lib.EPI_SILU_MUL,
                                   out=self.act)
            kernels.linear(self.act, p.down, epilogue=_lib.EPI_RESIDUAL_ADD, residual=self.mid, out=y)
        last = self.hidden[len(self.layers) % 2]
        # final RMSNorm + scores + argmax (qwen_explicit.py:1798-1832 / :952-960) in the lm_head kernel
        kernels.lm_head_argmax(last, self.lm_head, logits_mode=self.logits_mode, workspace=self.head_ws,
                               out=self.token, norm_weight=self.final_norm, eps=self.eps)
