"""Pin the CPU oracle (oracle/projections.py) before trusting it.

Each check is chosen so that a plausible mistake in the oracle -- a dropped
term, a transposed operand, a wrong sign or split, a wrong rounding chain or
tie rule -- fails it.  None of them restates the oracle's own formula.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute
from oracle import projections as ref
from tests.helpers import bits, from_bits


def _case(n, k, m, seed):
    rng = np.random.default_rng(seed)
    w = brute.f32_to_bf16_bits((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = brute.f32_to_bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    return w, x


def _within_rounding(got: np.ndarray, y64: np.ndarray, bound: np.ndarray) -> bool:
    slack = 0.5 * np.maximum(brute.bf16_ulp(y64), brute.bf16_ulp(got)) + bound + 1e-30
    return bool(np.all(np.abs(got - y64) <= slack))


@pytest.mark.parametrize("n,k,m", [(16, 32, 1), (48, 96, 3), (64, 2560, 2), (32, 9728, 1)])
def test_linear_matches_float64_brute_force(n, k, m):
    w, x = _case(n, k, m, seed=n + k + m)
    y64 = brute.linear64(x, w)
    bound = brute.fp32_sum_bound(x, w)
    got = ref.linear(from_bits(x), from_bits(w)).double().numpy()
    assert _within_rounding(got, y64, bound)
    if m == 1:
        got_mv = ref.mv(from_bits(w), from_bits(x)[0]).double().numpy()
        assert _within_rounding(got_mv[None, :], y64, bound)


def test_one_hot_activation_returns_weight_column_exactly():
    w, _ = _case(64, 128, 1, seed=3)
    wt = from_bits(w)
    for col in (0, 7, 64, 127):
        x = torch.zeros(128, dtype=torch.bfloat16)
        x[col] = 1.0
        assert torch.equal(ref.mv(wt, x), wt[:, col])


def test_power_of_two_scaling_is_exact():
    w, x = _case(32, 256, 2, seed=4)
    wt, xt = from_bits(w), from_bits(x)
    base = ref.linear(xt, wt)
    assert torch.equal(ref.linear(xt * 4, wt), base * 4)
    assert torch.equal(ref.linear(xt, wt * 0.5), base * 0.5)


def test_linearity_in_x():
    w, x = _case(32, 512, 2, seed=5)
    wt = from_bits(w).double()
    a, b = from_bits(x).double()
    ya = torch.mv(wt, a)
    yb = torch.mv(wt, b)
    ysum = torch.mv(wt, a + b)
    assert torch.allclose(ysum, ya + yb, rtol=0, atol=1e-9)
    got = ref.mv(from_bits(w), (a + b).to(torch.bfloat16)).double()
    bf_sum_exact = (a + b).to(torch.bfloat16).double()
    assert torch.allclose(got, torch.mv(wt, bf_sum_exact), rtol=2e-2, atol=1e-2)


def test_rows_are_independent():
    """M stacked GEMVs equal one GEMM (rows do not mix), to fp32-order noise."""
    w, x = _case(64, 256, 4, seed=6)
    wt, xt = from_bits(w), from_bits(x)
    full = ref.linear(xt, wt).double()
    stacked = torch.stack([ref.mv(wt, xt[i]) for i in range(4)]).double()
    y64 = brute.linear64(x, w)
    bound = brute.fp32_sum_bound(x, w)
    assert _within_rounding(full.numpy(), y64, bound)
    assert _within_rounding(stacked.numpy(), y64, bound)
    # Permuting the rows of x permutes the rows of y: no cross-row terms.
    perm = torch.tensor([2, 0, 3, 1])
    assert torch.equal(ref.linear(xt[perm], wt), ref.linear(xt, wt)[perm])


def test_fused_qkv_segment_order():
    """One-hot weight rows pin [q | k | v] along the fused output (pack.py:271-274)."""
    q, kv, k = 8, 4, 16
    w = torch.zeros(q + 2 * kv, k, dtype=torch.bfloat16)
    for r in range(q + 2 * kv):
        w[r, r % k] = 1.0 + r  # row r reads input r % k, scaled by its own index
    x = torch.arange(1, k + 1, dtype=torch.bfloat16)
    y = ref.mv(w, x)
    qs, ks, vs = torch.split(y, (q, kv, kv))
    assert qs.tolist() == [(1.0 + r) * ((r % k) + 1) for r in range(q)]
    assert ks.tolist() == [(1.0 + r) * ((r % k) + 1) for r in range(q, q + kv)]
    assert vs.tolist() == [(1.0 + r) * ((r % k) + 1) for r in range(q + kv, q + 2 * kv)]


def test_silu_mul_applies_silu_to_the_gate_half():
    """SiLU goes on the first (gate) half, the second half multiplies
    (qwen_explicit.py:829-830): swapping the halves changes the result."""
    gate = torch.tensor([[0.0, 8.0, -8.0, 1.0]], dtype=torch.bfloat16)
    up = torch.tensor([[5.0, 3.0, 3.0, 2.0]], dtype=torch.bfloat16)
    out = ref.silu_mul(torch.cat((gate, up), dim=-1), 4).double()
    g = gate.double().numpy()
    u = up.double().numpy()
    expect = brute.silu_mul_chain(g, u)
    assert np.allclose(out.numpy(), expect, rtol=0, atol=0)
    assert out[0, 0] == 0.0                       # silu(0) = 0
    assert abs(out[0, 1] - 8.0 * 3.0) < 0.05 * 24  # large +g -> g * u
    assert abs(out[0, 2]) < 0.01                  # large -g -> 0
    swapped = ref.silu_mul(torch.cat((up, gate), dim=-1), 4)
    assert not torch.equal(swapped, out.to(torch.bfloat16))


def test_silu_over_every_bf16_gate():
    """The oracle's SiLU*up (F.silu on bf16, computed in float32) against the
    float64 chain for every finite bf16 gate and a few up values: within one
    bf16 ulp and identical almost everywhere, except below g = -88.72, where
    exp(-g) overflows float32 and the float32 formula gives -0 while the
    float64 one still gives a value below 2^-121."""
    pat = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    pat = pat[(pat & 0x7F80) != 0x7F80]
    g = brute.bf16_bits_to_f64(pat)
    for u_val in (1.0, -0.75, 0.3125):
        u = np.full_like(g, u_val)
        gate = torch.from_numpy(pat.view(np.int16)).view(torch.bfloat16).view(1, -1)
        up = torch.full_like(gate, u_val)
        out = ref.silu_mul(torch.cat((gate, up), dim=-1), gate.shape[-1]).double().numpy()[0]
        with np.errstate(over="ignore"):
            expect = brute.silu_mul_chain(g, u)
        overflow = g < -88.72
        assert np.all(out[overflow] == 0.0)
        assert np.all(np.abs(expect[overflow]) < 2.0 ** -121)
        o, e = out[~overflow], expect[~overflow]
        assert np.all(np.abs(o - e) <= brute.bf16_ulp(np.maximum(np.abs(o), np.abs(e))))
        assert np.mean(o == e) >= 0.999


def test_silu_matches_closed_form_elementwise():
    rng = np.random.default_rng(8)
    g = brute.round_bf16(rng.standard_normal(4096) * 4)
    u = brute.round_bf16(rng.standard_normal(4096))
    gt = torch.tensor(g, dtype=torch.float64).to(torch.bfloat16)
    ut = torch.tensor(u, dtype=torch.float64).to(torch.bfloat16)
    out = ref.silu_mul(torch.cat((gt, ut)).view(1, -1), 4096).double().numpy()[0]
    expect = brute.silu_mul_chain(g, u)
    # fp32 silu in torch vs float64 silu: equal after bf16 rounding except at
    # rounding ties of the intermediate; allow one bf16 ulp there.
    assert np.mean(out == expect) > 0.995
    assert np.all(np.abs(out - expect) <= brute.bf16_ulp(expect) + 1e-30)


def test_logits_argmax_planted_and_ties():
    v, k = 512, 64
    rng = np.random.default_rng(9)
    w = brute.f32_to_bf16_bits((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    h = brute.f32_to_bf16_bits(rng.standard_normal((1, k)).astype(np.float32))
    hot = brute.f32_to_bf16_bits((np.sign(brute.bf16_bits_to_f64(h[0])) * 0.5).astype(np.float32))
    w[300] = hot
    w[120] = hot  # identical maximal row at a lower index
    wt, ht = from_bits(w), from_bits(h)[0]
    assert ref.logits_argmax(ht, wt).item() == 120
    assert ref.greedy_head_vector(ht, torch.ones(k, dtype=torch.bfloat16), wt, 1e-6).item() == 120
    assert ref.bf16_logits_argmax(ht, wt).item() == 120
    w[120] = brute.f32_to_bf16_bits(np.zeros(k, dtype=np.float32))
    assert ref.logits_argmax(ht, from_bits(w)).item() == 300


def test_greedy_head_vector_applies_the_final_norm_weight():
    """RMSNorm is scale-invariant for the argmax, so a tie test with an
    all-ones weight cannot see the final norm weight.  Here the weight is 4
    on the first half of the hidden dims and 1/4 on the second half, and two
    vocab rows each read one half (the second with 4x the magnitude):
    applied as rmsnorm(h) * w, row 0 wins (4 x 32 against 4 x 0.25 x 32);
    dropped, row 1 wins (128 against 32); divided instead of multiplied or
    applied to the swapped halves, row 1 wins too.  A random case is held to
    the float64 chain of the reference (qwen_explicit.py:952-960)."""
    k = 64
    h = torch.ones(k, dtype=torch.bfloat16)
    w_norm = torch.cat((torch.full((k // 2,), 4.0), torch.full((k // 2,), 0.25))).to(torch.bfloat16)
    lm = torch.zeros((3, k), dtype=torch.float32)
    lm[0, : k // 2] = 1.0
    lm[1, k // 2:] = 4.0
    lm[2] = -1.0
    lm = lm.to(torch.bfloat16)
    assert ref.greedy_head_vector(h, w_norm, lm, 1e-6).item() == 0
    # the plausible mistakes pick row 1
    assert ref.greedy_head_vector(h, torch.ones(k, dtype=torch.bfloat16), lm, 1e-6).item() == 1
    assert ref.greedy_head_vector(h, (1.0 / w_norm.float()).to(torch.bfloat16), lm, 1e-6).item() == 1
    assert ref.greedy_head_vector(h, w_norm.flip(0), lm, 1e-6).item() == 1

    rng = np.random.default_rng(12)
    v, k = 1024, 256
    lm_bits = brute.f32_to_bf16_bits((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    h_bits = brute.f32_to_bf16_bits((rng.standard_normal(k) * 2.0).astype(np.float32))
    wn_bits = brute.f32_to_bf16_bits((1.0 + 0.5 * rng.standard_normal(k)).astype(np.float32))
    h64, wn64, lm64 = (brute.bf16_bits_to_f64(b) for b in (h_bits, wn_bits, lm_bits))
    normed = brute.round_bf16(h64 / np.sqrt(np.mean(h64 * h64) + 1e-6) * wn64)
    logits = lm64 @ normed
    top = np.sort(logits)[-2:]
    got = ref.greedy_head_vector(from_bits(h_bits[None])[0], from_bits(wn_bits[None])[0], from_bits(lm_bits),
                                 1e-6).item()
    # bf16 logits may merge scores closer than one bf16 step at their size
    assert top[1] - top[0] > 2 * brute.bf16_ulp(np.array([top[1]]))[0]
    assert got == int(np.argmax(logits))


def test_logits_scores_are_fp32_accumulated():
    """The cuTile head accumulates f32(W) * f32(h) in fp32 (cutile_logits.py:27):
    the oracle's scores stay within the fp32 summation bound of float64."""
    v, k = 256, 2560
    rng = np.random.default_rng(10)
    w = brute.f32_to_bf16_bits((rng.standard_normal((v, k)) * 0.02).astype(np.float32))
    h = brute.f32_to_bf16_bits(rng.standard_normal((1, k)).astype(np.float32))
    s = ref.logits_scores_fp32(from_bits(h)[0], from_bits(w)).double().numpy()
    s64 = brute.linear64(h, w)[0]
    assert np.all(np.abs(s - s64) <= brute.fp32_sum_bound(h, w)[0] + 1e-12)
    # ... and are NOT rounded to bf16 (a bf16 head would fail this on random data)
    assert np.any(np.abs(s - brute.round_bf16(s)) > 0)


def test_mlp_epilogue_vector_composes_the_reference_steps():
    """_semantic_mlp_epilogue_vector = residual + down(silu_mul(gate_up(rmsnorm(h))))."""
    h_dim, inter = 64, 96
    rng = np.random.default_rng(11)
    hid = torch.tensor(rng.standard_normal(h_dim), dtype=torch.float32).to(torch.bfloat16)
    ln = torch.tensor(1 + 0.1 * rng.standard_normal(h_dim), dtype=torch.float32).to(torch.bfloat16)
    gu = torch.tensor(rng.standard_normal((2 * inter, h_dim)) * 0.05, dtype=torch.float32).to(torch.bfloat16)
    dn = torch.tensor(rng.standard_normal((h_dim, inter)) * 0.05, dtype=torch.float32).to(torch.bfloat16)
    out = ref.mlp_epilogue_vector(hid, ln, gu, inter, dn, 1e-6)
    hf = hid.double()
    normed = (hf / torch.sqrt((hf * hf).mean() + 1e-6) * ln.double())
    g = gu.double() @ normed
    act = torch.nn.functional.silu(g[:inter]) * g[inter:]
    expect = hf + dn.double() @ act
    assert torch.allclose(out.double(), expect, rtol=3e-2, atol=3e-2)
    # the residual is really added: dropping it moves the result by |h|
    assert (out.double() - (expect - hf)).abs().max() > 0.5


def test_rmsnorm_closed_forms():
    """rms_norm of a constant row c with eps = 0 is sign(c) * w exactly (r = 1/|c|
    for a power-of-two c), and eps enters under the square root: with
    x = 1 and eps = 3 the row is scaled by 1/2."""
    k = 2560
    w = torch.tensor(np.random.default_rng(12).standard_normal(k), dtype=torch.float32).to(torch.bfloat16)
    for c in (0.25, 1.0, -8.0, 64.0):
        x = torch.full((1, k), c, dtype=torch.bfloat16)
        out = ref.rmsnorm(x, w, 0.0)
        assert torch.equal(out[0], (w.float() * np.sign(c)).to(torch.bfloat16))
    out = ref.rmsnorm(torch.ones(1, k, dtype=torch.bfloat16), w, 3.0)
    assert torch.equal(out[0], (w.float() * 0.5).to(torch.bfloat16))


def test_rmsnorm_power_of_two_scale_invariance():
    """With eps = 0, scaling a row by 2^j changes neither r * x nor the output
    (a wrong exponent of the mean, or a missing square, breaks this)."""
    rng = np.random.default_rng(13)
    x = torch.tensor(rng.standard_normal((3, 2560)), dtype=torch.float32).to(torch.bfloat16)
    w = torch.tensor(1 + 0.2 * rng.standard_normal(2560), dtype=torch.float32).to(torch.bfloat16)
    base = ref.rmsnorm(x, w, 0.0)
    for j in (-3, 2, 5):
        assert torch.equal(ref.rmsnorm(x * (2.0 ** j), w, 0.0), base)


def test_rmsnorm_matches_float64_one_rounding():
    """Each output is the float64 value (x * r) * w rounded once to bf16, to
    within one bf16 step where the fp32 evaluation lands next to a rounding
    boundary; the two-rounding form bf16(bf16(x * r) * w) of the composite
    fallback (qwen_explicit.py:629-633) differs from it on many elements,
    so the chain is pinned as the single rounding of the cuTile kernel and
    its torch reference (experiments/cutile/qwen_bf16_hot_kernels.py:45-57)."""
    rng = np.random.default_rng(14)
    k = 2560
    xb = brute.f32_to_bf16_bits((rng.standard_normal((4, k)) * np.array([[0.1], [1.0], [7.0], [300.0]]))
                                .astype(np.float32))
    wb = brute.f32_to_bf16_bits((1 + 0.3 * rng.standard_normal(k)).astype(np.float32))
    eps = 1e-6
    x64, w64 = brute.bf16_bits_to_f64(xb), brute.bf16_bits_to_f64(wb)
    r64 = 1.0 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + eps)
    y64 = x64 * r64 * w64
    got = ref.rmsnorm(from_bits(xb), from_bits(wb), eps).double().numpy()
    step = brute.bf16_ulp(y64)
    assert np.all(np.abs(got - y64) <= step * (0.5 + 2e-3) + 1e-30)
    exact = np.mean(got == brute.round_bf16(y64))
    assert exact > 0.995
    two = brute.round_bf16(brute.round_bf16(x64 * r64) * w64)
    assert np.mean(got != two) > 0.1


# ---------------------------------------------------------------- decode attention step


def _bf(x):
    return torch.tensor(np.asarray(x), dtype=torch.float32).to(torch.bfloat16)


def test_rope_closed_forms():
    """cos = 1, sin = 0 is the identity; cos = 0, sin = 1 maps (a, b) to
    (-b, a) exactly: a sign error, swapped halves or a missing term fails."""
    from oracle.attention import rope

    rng = np.random.default_rng(20)
    q = _bf(rng.standard_normal((1, 4, 1, 128)))
    k = _bf(rng.standard_normal((1, 2, 1, 128)))
    one, zero = torch.ones(1, 1, 64, dtype=torch.bfloat16), torch.zeros(1, 1, 64, dtype=torch.bfloat16)
    q1, k1 = rope(q, k, one, zero)
    assert torch.equal(q1, q) and torch.equal(k1, k)
    q2, k2 = rope(q, k, zero, one)
    assert torch.equal(q2, torch.cat((-q[..., 64:], q[..., :64]), dim=-1))
    assert torch.equal(k2, torch.cat((-k[..., 64:], k[..., :64]), dim=-1))


def test_rope_matches_float64_rotation():
    """Random angles: each output is the float64 rotation of the bf16 inputs
    to within the reference's per-op bf16 roundings (two products and one sum)."""
    from oracle.attention import rope

    rng = np.random.default_rng(21)
    q = _bf(rng.standard_normal((1, 3, 1, 128)) * 2)
    ang = rng.uniform(0, 2 * np.pi, 64)
    cos, sin = _bf(np.cos(ang)[None, None]), _bf(np.sin(ang)[None, None])
    out, _ = rope(q, q[:, :1], cos, sin)
    a, b = q[..., :64].double().numpy(), q[..., 64:].double().numpy()
    c, s = cos.double().numpy()[:, None], sin.double().numpy()[:, None]
    exact = np.concatenate((a * c - b * s, b * c + a * s), axis=-1)
    bound = 2.0 ** -8 * (np.abs(np.concatenate((a * c, b * c), -1)) + np.abs(np.concatenate((b * s, a * s), -1))) \
        + 2.0 ** -8 * np.abs(exact)
    assert np.all(np.abs(out.double().numpy() - exact) <= bound + 1e-30)


def test_sdpa_gqa_pins():
    """softmax(q K^T * scale) V with kv head h // G: against a float64 brute
    force, against torch's own scaled_dot_product_attention (fp32, enable_gqa),
    uniform keys give the mean of V, and a planted dominant key returns its row."""
    from oracle.attention import sdpa_gqa

    rng = np.random.default_rng(22)
    n_q, n_kv, S, d = 8, 2, 37, 128
    q = _bf(rng.standard_normal((1, n_q, 1, d)))
    k = _bf(rng.standard_normal((1, n_kv, S, d)))
    v = _bf(rng.standard_normal((1, n_kv, S, d)))
    scale = d ** -0.5
    out = sdpa_gqa(q, k, v, scale, n_q // n_kv).double().numpy()
    q64, k64, v64 = q.double().numpy(), k.double().numpy(), v.double().numpy()
    for h in range(n_q):
        j = h // (n_q // n_kv)
        s = (k64[0, j] @ q64[0, h, 0]) * scale
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ v64[0, j]
        assert np.allclose(out[0, h, 0], ref, rtol=1e-2, atol=1e-2)
    torch_out = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), scale=scale, enable_gqa=True)
    assert torch.allclose(sdpa_gqa(q, k, v, scale, n_q // n_kv).float(), torch_out, rtol=1e-2, atol=1e-2)
    # uniform keys -> mean of V
    ku = k.clone()
    ku[:] = k[:, :, :1]
    mean = v.float().mean(dim=2, keepdim=True).repeat_interleave(n_q // n_kv, dim=1)
    assert torch.allclose(sdpa_gqa(q, ku, v, scale, n_q // n_kv).float(), mean, rtol=0, atol=2e-2)
    # a key aligned with q head 0 at 30x the scale dominates: head 0 returns that V row
    kd = k.clone()
    kd[0, 0, 5] = (q[0, 0, 0].float() * 30).to(torch.bfloat16)
    got = sdpa_gqa(q, kd, v, scale, n_q // n_kv)
    assert torch.allclose(got[0, 0, 0].float(), v[0, 0, 5].float(), atol=1e-2)



def test_decode_attention_appends_one_row():
    """The oracle writes exactly row `pos` of each cache (k rotated, v as is)
    and attends over rows 0..pos only: changing a row past pos changes nothing."""
    from oracle.attention import decode_attention, qk_heads_vector

    rng = np.random.default_rng(23)
    n_q, n_kv, d, S, pos = 4, 2, 128, 32, 9
    qkv = _bf(rng.standard_normal((n_q + 2 * n_kv) * d))
    qn, kn = _bf(1 + 0.1 * rng.standard_normal(d)), _bf(1 + 0.1 * rng.standard_normal(d))
    ang = rng.uniform(0, 6, 64)
    cos, sin = _bf(np.cos(ang)), _bf(np.sin(ang))
    kc, vc = _bf(rng.standard_normal((n_kv, S, d))), _bf(rng.standard_normal((n_kv, S, d)))
    out, kc2, vc2 = decode_attention(qkv, n_q, n_kv, d, qn, kn, 1e-6, cos, sin, kc, vc, pos, d ** -0.5)
    _, k, v = qk_heads_vector(qkv, n_q, n_kv, d, qn, kn, 1e-6, cos, sin)
    rows = [t for t in range(S) if t != pos]
    assert torch.equal(kc2[:, rows], kc[:, rows]) and torch.equal(vc2[:, rows], vc[:, rows])
    assert torch.equal(kc2[:, pos], k.view(n_kv, d)) and torch.equal(vc2[:, pos], v.view(n_kv, d))
    kc_far = kc.clone()
    kc_far[:, pos + 1:] = 100.0
    out_far, _, _ = decode_attention(qkv, n_q, n_kv, d, qn, kn, 1e-6, cos, sin, kc_far, vc, pos, d ** -0.5)
    assert torch.equal(out, out_far)


# ---------------------------------------------------------------- composite functions
#
# The oracle's compositions (post-attention MLP, MLP forward, q/k heads,
# decode layer) against brute's float64 restatements with the same bf16
# rounding points.  Each check also runs the float64 chain with a plausible
# mistake -- a residual joined at the wrong point, a norm on the wrong
# tensor, swapped q/k norm weights, a wrong kv-head mapping, the new row left
# out of attention -- and requires that the oracle does NOT match it, so the
# check is known to catch that mistake.

from oracle import attention as ref_attn  # noqa: E402


def _f64(t: torch.Tensor) -> np.ndarray:
    return brute.bf16_bits_to_f64(bits(t)).reshape(tuple(t.shape))


def _agreement(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    """(fraction of bit-equal values, max |got - want| / max |want|)."""
    return float(np.mean(got == want)), float(np.abs(got - want).max() / np.abs(want).max())


def _matches(got, want) -> bool:
    exact, rel = _agreement(got, want)
    return exact >= 0.98 and rel <= 1e-2


def _differs(got, want) -> bool:
    exact, rel = _agreement(got, want)
    return exact < 0.5 and rel > 3e-2


class _Rand:
    def __init__(self, seed):
        self.rng = np.random.default_rng(seed)

    def __call__(self, *shape, scale=1.0, mean=0.0):
        return _bf(mean + self.rng.standard_normal(shape) * scale)


def test_post_attention_mlp_is_pinned():
    """_semantic_post_attention_mlp_eager (qwen_explicit.py:809-831):
    h = residual + o(attn), then h + MLP(rmsnorm(h))."""
    r = _Rand(21)
    h_dim, q_dim, inter, t = 64, 96, 80, 3
    attn, res = r(t, q_dim), r(t, h_dim)
    o_w, ln = r(h_dim, q_dim, scale=0.1), r(h_dim, scale=0.2, mean=1.0)
    gu, dn = r(2 * inter, h_dim, scale=0.15), r(h_dim, inter, scale=0.15)
    got = _f64(ref.post_attention_mlp(attn, res, o_w, ln, gu, inter, dn, 1e-6))
    A, R, O, L, GU, DN = map(_f64, (attn, res, o_w, ln, gu, dn))
    assert _matches(got, brute.post_attention_mlp64(A, R, O, L, GU, inter, DN, 1e-6))
    h = brute.round_bf16(R + brute.proj64(A, O))
    mlp = lambda x: brute.mlp_forward64(x, GU, inter, DN)  # noqa: E731
    mistakes = {
        "residual joins before o_proj's output": brute.round_bf16(R + mlp(brute.rmsnorm64(h, L, 1e-6))),
        "norm of the residual, not of h": brute.round_bf16(h + mlp(brute.rmsnorm64(R, L, 1e-6))),
        "norm of o_proj's output": brute.round_bf16(h + mlp(brute.rmsnorm64(brute.proj64(A, O), L, 1e-6))),
        "no norm": brute.round_bf16(h + mlp(h)),
        "no final residual": mlp(brute.rmsnorm64(h, L, 1e-6)),
    }
    for what, wrong in mistakes.items():
        assert _differs(got, wrong), what


def test_mlp_forward_is_pinned():
    """semantic_qwen_mlp_forward (qwen_explicit.py:1201-1208): down(SiLU(gate) * up)."""
    r = _Rand(22)
    h_dim, inter, t = 64, 80, 4
    x, gu, dn = r(t, h_dim), r(2 * inter, h_dim, scale=0.15), r(h_dim, inter, scale=0.15)
    got = _f64(ref.mlp_forward(x, gu, inter, dn))
    X, GU, DN = map(_f64, (x, gu, dn))
    assert _matches(got, brute.mlp_forward64(X, GU, inter, DN))
    g = brute.proj64(X, GU)
    swapped = np.concatenate((g[:, inter:], g[:, :inter]), axis=1)
    mistakes = {
        "SiLU on the up half": brute.proj64(brute.silu_mul64(swapped, inter), DN),
        "no SiLU": brute.proj64(brute.round_bf16(g[:, :inter] * g[:, inter:]), DN),
        "down of the gate half alone": brute.proj64(g[:, :inter], DN),
    }
    for what, wrong in mistakes.items():
        assert _differs(got, wrong), what


def _qk_case(seed):
    r = _Rand(seed)
    n_q, n_kv, d = 4, 2, 16
    qkv = r((n_q + 2 * n_kv) * d, scale=2.0)
    qn, kn = r(d, scale=0.3, mean=1.0), r(d, scale=0.3, mean=1.0)
    ang = r.rng.uniform(0.3, 6.0, d // 2)
    return n_q, n_kv, d, qkv, qn, kn, _bf(np.cos(ang)), _bf(np.sin(ang))


def test_qk_heads_vector_is_pinned():
    """The tail of _semantic_attention_qkv_vector_eager (qwen_explicit.py:
    788-806): split [q | k | v], q heads normalised with q_norm_weight and k
    heads with k_norm_weight, each over head_dim, then RoPE."""
    n_q, n_kv, d, qkv, qn, kn, cos, sin = _qk_case(23)
    q, k, v = ref_attn.qk_heads_vector(qkv, n_q, n_kv, d, qn, kn, 1e-6, cos, sin)
    got_q, got_k, got_v = _f64(q).reshape(n_q, d), _f64(k).reshape(n_kv, d), _f64(v).reshape(n_kv, d)
    QKV, QN, KN, C, S = map(_f64, (qkv, qn, kn, cos, sin))
    want_q, want_k, want_v = brute.qk_heads64(QKV, n_q, n_kv, d, QN, KN, 1e-6, C, S)
    assert _matches(got_q, want_q) and _matches(got_k, want_k) and np.array_equal(got_v, want_v)
    swapped_q, swapped_k, _ = brute.qk_heads64(QKV, n_q, n_kv, d, KN, QN, 1e-6, C, S)
    assert _differs(got_q, swapped_q) and _differs(got_k, swapped_k), "q/k norm weights swapped"
    qs = QKV[: n_q * d]
    whole = brute.rope64(brute.round_bf16(qs * QN.repeat(n_q) / np.sqrt((qs * qs).mean() + 1e-6)).reshape(n_q, d),
                         C, S)
    assert _differs(got_q, whole), "q normalised over all heads at once"
    unrotated_q, _, _ = brute.qk_heads64(QKV, n_q, n_kv, d, QN, KN, 1e-6, np.ones_like(C), np.zeros_like(S))
    assert _differs(got_q, unrotated_q), "RoPE left out"
    assert _differs(got_q, brute.qk_heads64(QKV, n_q, n_kv, d, QN, KN, 1e-6, C, -S)[0]), "RoPE sign flipped"


def _layer64_with(mistake, hidden, in_ln, qkv_w, n_q, n_kv, d, qn, kn, cos, sin, kc, vc, pos, scale, o_w, post_ln,
                  gu, inter, dn, eps):
    """brute.decode_layer64's chain with one named mistake (None: none)."""
    if mistake == "q/k norms swapped":
        qn, kn = kn, qn
    x = hidden if mistake != "no input norm" else None
    qkv = brute.proj64(brute.rmsnorm64(hidden, in_ln, eps) if x is not None else hidden, qkv_w)
    q, k, v = brute.qk_heads64(qkv, n_q, n_kv, d, qn, kn, eps, cos, sin)
    kc, vc = kc.copy(), vc.copy()
    kc[:, pos], vc[:, pos] = k, v
    rows = pos if mistake == "new row not attended" else pos + 1
    if mistake == "kv head h % n_kv":
        q = q.reshape(n_q // n_kv, n_kv, d).transpose(1, 0, 2).reshape(n_q, d)
        a = brute.attention64(q, kc[:, :rows], vc[:, :rows], scale)
        attn = a.reshape(n_kv, n_q // n_kv, d).transpose(1, 0, 2).reshape(-1)
    else:
        attn = brute.attention64(q, kc[:, :rows], vc[:, :rows], scale).reshape(-1)
    h = brute.round_bf16(hidden + brute.proj64(attn, o_w))
    normed = brute.rmsnorm64(hidden if mistake == "post norm of the layer input" else h, post_ln, eps)
    base = hidden if mistake == "final residual is the layer input" else h
    return brute.round_bf16(base + brute.mlp_forward64(normed, gu, inter, dn)), kc, vc


def test_decode_layer_is_pinned():
    """semantic_qwen_decode_layer_forward (qwen_explicit.py:1247-1272) with a
    filled cache: the output and the appended cache row against brute's
    float64 chain, and five plausible mistakes that the check rejects."""
    r = _Rand(24)
    h_dim, n_q, n_kv, d, inter, s_max, pos = 64, 4, 2, 16, 80, 8, 5
    hidden = r(h_dim, scale=2.0)
    in_ln, post_ln = r(h_dim, scale=0.2, mean=1.0), r(h_dim, scale=0.2, mean=1.0)
    qkv_w = r((n_q + 2 * n_kv) * d, h_dim, scale=0.2)
    qn, kn = r(d, scale=0.3, mean=1.0), r(d, scale=0.3, mean=1.0)
    o_w, gu, dn = r(h_dim, n_q * d, scale=0.15), r(2 * inter, h_dim, scale=0.15), r(h_dim, inter, scale=0.15)
    kc, vc = r(n_kv, s_max, d, scale=2.0), r(n_kv, s_max, d)
    ang = r.rng.uniform(0.3, 6.0, d // 2)
    cos, sin = _bf(np.cos(ang)), _bf(np.sin(ang))
    scale = d ** -0.5
    out, kc_new, vc_new = ref_attn.decode_layer(hidden, in_ln, qkv_w, n_q, n_kv, d, qn, kn, cos, sin, kc, vc, pos,
                                                scale, o_w, post_ln, gu, inter, dn, 1e-6)
    args = [_f64(hidden), _f64(in_ln), _f64(qkv_w), n_q, n_kv, d, _f64(qn), _f64(kn), _f64(cos), _f64(sin), _f64(kc),
            _f64(vc), pos, scale, _f64(o_w), _f64(post_ln), _f64(gu), inter, _f64(dn), 1e-6]
    want, want_kc, want_vc = brute.decode_layer64(*args)
    got = _f64(out)
    assert _matches(got, want)
    assert _matches(_f64(kc_new)[:, pos], want_kc[:, pos]) and np.array_equal(_f64(vc_new), want_vc)
    assert np.array_equal(_f64(kc_new)[:, :pos], _f64(kc)[:, :pos])  # only row pos changes
    assert np.array_equal(_layer64_with(None, *args)[0], want)
    for mistake in ("q/k norms swapped", "new row not attended", "kv head h % n_kv", "post norm of the layer input",
                    "final residual is the layer input", "no input norm"):
        assert _differs(got, _layer64_with(mistake, *args)[0]), mistake
