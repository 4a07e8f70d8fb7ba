"""The drop-in boundary: leanstack_amd.dispatch offers the reference's
dispatch names with the reference's parameter lists, so the semantic runtime
binds them unchanged (CPU only; nothing is called).

Each entry is the parameter list of the reference function at
src/leanstack/runtime/qwen_explicit.py:<line> (the *_eager body that the
reference wraps under the same name at :963-971 where one exists)."""

from __future__ import annotations

import inspect

import pytest

from leanstack_amd import dispatch

REFERENCE_SIGNATURES = {
    "_semantic_attention_qkv": (733, ["hidden_states", "qkv_proj_weight", "q_proj_out_dim", "k_proj_out_dim",
                                      "num_attention_heads", "num_key_value_heads", "head_dim", "q_norm_weight",
                                      "k_norm_weight", "cos", "sin", "rms_norm_eps"]),
    "_semantic_attention_qkv_vector": (773, ["hidden_states", "qkv_proj_weight", "q_proj_out_dim", "k_proj_out_dim",
                                             "num_attention_heads", "num_key_value_heads", "head_dim",
                                             "q_norm_weight", "k_norm_weight", "cos", "sin", "rms_norm_eps"]),
    "_semantic_post_attention_mlp": (809, ["attention_output", "residual", "o_proj_weight",
                                           "post_attention_layernorm_weight", "gate_up_proj_weight",
                                           "gate_proj_out_dim", "down_proj_weight", "rms_norm_eps"]),
    "_semantic_mlp_epilogue": (834, ["hidden_states", "post_attention_layernorm_weight", "gate_up_proj_weight",
                                     "gate_proj_out_dim", "down_proj_weight", "rms_norm_eps"]),
    "_semantic_decode_attention_output": (855, ["query_states", "key_states", "value_states", "o_proj_weight",
                                                "attention_scale", "num_key_value_groups"]),
    "_semantic_decode_attention_output_vector": (886, ["query_states", "key_states", "value_states",
                                                       "o_proj_weight", "attention_scale",
                                                       "num_key_value_groups"]),
    "_semantic_greedy_head": (916, ["hidden_states", "final_norm_weight", "lm_head_weight", "rms_norm_eps"]),
    "_semantic_mlp_epilogue_vector": (932, ["hidden_states", "post_attention_layernorm_weight",
                                            "gate_up_proj_weight", "gate_proj_out_dim", "down_proj_weight",
                                            "rms_norm_eps"]),
    "_semantic_greedy_head_vector": (952, ["hidden_states", "final_norm_weight", "lm_head_weight", "rms_norm_eps"]),
    "semantic_qwen_mlp_forward": (1201, ["mlp", "hidden_states"]),
    "project_semantic_hidden_to_logits": (1775, ["runtime", "hidden_states"]),
    "select_semantic_greedy_token": (1814, ["runtime", "hidden_states"]),
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SIGNATURES))
def test_dispatch_name_has_the_reference_parameters(name):
    line, params = REFERENCE_SIGNATURES[name]
    fn = getattr(dispatch, name, None)
    assert callable(fn), f"dispatch.{name} (qwen_explicit.py:{line}) is missing"
    got = [p.name for p in inspect.signature(fn).parameters.values()
           if p.kind in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD)]
    assert got == params, f"dispatch.{name} takes {got}, qwen_explicit.py:{line} takes {params}"
    # No extra required parameter: a call written for the reference binds.
    extra = [p.name for p in inspect.signature(fn).parameters.values()
             if p.name not in params and p.default is inspect.Parameter.empty
             and p.kind not in (p.VAR_POSITIONAL, p.VAR_KEYWORD)]
    assert not extra, f"dispatch.{name} requires {extra} beyond the reference's parameters"
