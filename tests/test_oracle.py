"""Pins the CPU oracle (oracle/decode_oracle.py) with checks that do not
restate its own formulas: library routines (torch, float64), closed forms,
invariants, and the committed golden vectors (tests/golden/, written by an
independent float64 torch composition).  CPU only.
"""

import math
import pathlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
rng = np.random.default_rng(1234)


def randn(*shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def t64(a):
    return torch.from_numpy(np.asarray(a, dtype=np.float64))


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------

def test_bf16_helpers_match_torch():
    a = randn(4096, scale=3.0)
    a[:4] = [0.0, -0.0, 1e-40, 65504.0]
    ours = oracle.bf16_bits(a)
    theirs = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(oracle.bf16_round(a), torch.from_numpy(a).to(torch.bfloat16).float().numpy())
    assert np.array_equal(oracle.as_f32(ours), oracle.bf16_round(a))


# ---------------------------------------------------------------------------
# small pieces
# ---------------------------------------------------------------------------

def test_rms_norm_matches_torch_library():
    x, w = randn(3, 257), randn(257, scale=0.1) + 1
    ref = F.rms_norm(t64(x), (257,), weight=t64(w), eps=1e-6).numpy()
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-6), ref, rtol=2e-6, atol=2e-6)


def test_topk_matches_torch_on_distinct_values():
    logits = randn(5, 300)
    v, i = oracle.topk_desc(logits, 8)
    tv, ti = torch.topk(torch.from_numpy(logits), 8, dim=-1)
    assert np.array_equal(i, ti.numpy())
    assert np.array_equal(v, tv.numpy())


def test_topk_tie_rule_lower_index_first():
    v, i = oracle.topk_desc(np.array([[1.0, 3.0, 3.0, 2.0, 3.0]], np.float32), 4)
    assert i.tolist() == [[1, 2, 4, 3]]


def test_softmax_and_silu_match_torch():
    a = randn(4, 9, scale=4)
    np.testing.assert_allclose(oracle.softmax(a), torch.softmax(t64(a), -1).numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(oracle.silu(a), F.silu(t64(a)).numpy(), rtol=1e-6, atol=1e-6)


# ---------------------------------------------------------------------------
# MoE
# ---------------------------------------------------------------------------

def _moe_inputs(B=2, H=24, E=6, I=10, Is=14, scale=0.3):
    return dict(
        x=randn(B, H), norm_weight=randn(H, scale=0.1) + 1, router_weight=randn(E, H, scale=scale),
        expert_gate=randn(E, I, H, scale=scale), expert_up=randn(E, I, H, scale=scale),
        expert_down=randn(E, H, I, scale=scale), shared_gate=randn(Is, H, scale=scale),
        shared_up=randn(Is, H, scale=scale), shared_down=randn(H, Is, scale=scale))


def _moe(d, **kw):
    return oracle.moe_decode(d["x"], d["norm_weight"], d["router_weight"], d["expert_gate"], d["expert_up"],
                             d["expert_down"], d["shared_gate"], d["shared_up"], d["shared_down"], **kw)


def _swiglu64(xn, g, u, dn):
    return F.linear(F.silu(F.linear(xn, g)) * F.linear(xn, u), dn)


def test_moe_matches_float64_library_composition():
    d = _moe_inputs()
    k = 3
    out, idx, w = _moe(d, top_k=k)
    x = t64(d["x"])
    xn = F.rms_norm(x, (x.shape[1],), weight=t64(d["norm_weight"]), eps=1e-6)
    logits = F.linear(xn, t64(d["router_weight"]))
    tv, ti = torch.topk(logits, k, dim=-1)
    tw = torch.softmax(tv, -1)
    ref = x + _swiglu64(xn, t64(d["shared_gate"]), t64(d["shared_up"]), t64(d["shared_down"]))
    for b in range(x.shape[0]):
        for s in range(k):
            e = int(ti[b, s])
            ref[b] += tw[b, s] * _swiglu64(xn[b:b + 1], t64(d["expert_gate"][e]), t64(d["expert_up"][e]),
                                           t64(d["expert_down"][e]))[0]
    assert idx.tolist() == ti.tolist()
    np.testing.assert_allclose(w, tw.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-4, atol=1e-4)


def test_moe_single_expert_reduces_to_dense_ffn():
    d = _moe_inputs(E=1)
    out, idx, w = _moe(d, top_k=1)
    assert idx.tolist() == [[0], [0]] and np.all(w == 1.0)
    dense = oracle.dense_ffn_decode(d["x"], d["norm_weight"], d["expert_gate"][0], d["expert_up"][0],
                                    d["expert_down"][0])
    shared = oracle.dense_ffn_decode(d["x"], d["norm_weight"], d["shared_gate"], d["shared_up"],
                                     d["shared_down"], add_residual=False)
    np.testing.assert_allclose(out, dense + shared, rtol=1e-5, atol=1e-5)


def test_moe_identical_experts_routing_independent():
    d = _moe_inputs(E=5)
    for key in ("expert_gate", "expert_up", "expert_down"):
        d[key] = np.repeat(d[key][:1], 5, axis=0)
    out_k2, _, _ = _moe(d, top_k=2)
    out_k4, _, _ = _moe(d, top_k=4)
    np.testing.assert_allclose(out_k2, out_k4, rtol=1e-5, atol=1e-5)


def test_moe_shared_gate_zero_is_half():
    d = _moe_inputs()
    ungated, idx0, _ = _moe(d, top_k=2)
    gated0, idx1, _ = _moe(d, top_k=2, shared_expert_gate=np.zeros(d["x"].shape[1], np.float32))
    no_shared = dict(d, shared_down=np.zeros_like(d["shared_down"]))
    routed, _, _ = _moe(no_shared, top_k=2)
    assert idx0.tolist() == idx1.tolist()
    np.testing.assert_allclose(gated0 - routed, 0.5 * (ungated - routed), rtol=1e-5, atol=1e-5)


def test_moe_shared_gate_reads_post_norm_activation():
    d = _moe_inputs()
    wsg = randn(d["x"].shape[1], scale=0.5)
    gated, _, _ = _moe(d, top_k=2, shared_expert_gate=wsg)
    ungated, _, _ = _moe(d, top_k=2)
    routed, _, _ = _moe(dict(d, shared_down=np.zeros_like(d["shared_down"])), top_k=2)
    xn = F.rms_norm(t64(d["x"]), (d["x"].shape[1],), weight=t64(d["norm_weight"]), eps=1e-6)
    factor = torch.sigmoid(xn @ t64(wsg)).numpy()[:, None]
    np.testing.assert_allclose(gated - routed, factor * (ungated - routed), rtol=1e-4, atol=1e-5)


def test_moe_router_weights_sum_to_one_and_sorted():
    d = _moe_inputs(B=4, E=9)
    _, idx, w = _moe(d, top_k=4)
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-6)
    assert np.all(np.diff(w, axis=-1) <= 0)


# ---------------------------------------------------------------------------
# dense FFN
# ---------------------------------------------------------------------------

def test_dense_matches_float64_library_and_zero_gate():
    x, nw = randn(3, 20), randn(20, scale=0.1) + 1
    g, u, dn = randn(33, 20, scale=0.3), randn(33, 20, scale=0.3), randn(20, 33, scale=0.3)
    out = oracle.dense_ffn_decode(x, nw, g, u, dn)
    xn = F.rms_norm(t64(x), (20,), weight=t64(nw), eps=1e-6)
    ref = t64(x) + _swiglu64(xn, t64(g), t64(u), t64(dn))
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(oracle.dense_ffn_decode(x, nw, np.zeros_like(g), u, dn), x)


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(2, 4, 2, 16, 9), (1, 24, 4, 32, 50), (3, 6, 6, 8, 5)])
def test_attention_matches_sdpa_library(shape):
    b, hq, hkv, d, t = shape
    q, k, v = randn(b, hq, d), randn(b, t, hkv, d), randn(b, t, hkv, d)
    out = oracle.full_attention_decode(q, k, v)
    ref = F.scaled_dot_product_attention(t64(q)[:, :, None], t64(k).transpose(1, 2), t64(v).transpose(1, 2),
                                         enable_gqa=True)[:, :, 0]
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-5, atol=1e-5)


def test_attention_known_answers():
    q, k, v = randn(1, 6, 16), randn(1, 1, 2, 16), randn(1, 1, 2, 16)
    out = oracle.full_attention_decode(q, k, v)
    np.testing.assert_allclose(out[0, :3], np.repeat(v[0, 0, :1], 3, 0), rtol=1e-6)
    np.testing.assert_allclose(out[0, 3:], np.repeat(v[0, 0, 1:], 3, 0), rtol=1e-6)
    k = np.repeat(randn(1, 1, 1, 16), 40, axis=1)
    v = randn(1, 40, 1, 16)
    out = oracle.full_attention_decode(randn(1, 3, 16), k, v, scale=0.7)
    np.testing.assert_allclose(out[0], np.repeat(v.mean(axis=1)[0], 3, 0), rtol=1e-5, atol=1e-6)
    with pytest.raises(ValueError, match="query_heads must be divisible by kv_heads"):
        oracle.full_attention_decode(randn(1, 3, 8), randn(1, 4, 2, 8), randn(1, 4, 2, 8))


def test_partial_rope_is_a_complex_rotation():
    q, k = randn(2, 3, 16), randn(2, 5, 3, 16)
    theta = randn(4, scale=2.0)
    cos = np.concatenate([np.cos(theta)] * 2).astype(np.float32)
    sin = np.concatenate([np.sin(theta)] * 2).astype(np.float32)
    qo, ko = oracle.apply_partial_rope(q, k, cos, sin, 8)
    z = (q[..., :4] + 1j * q[..., 4:8]) * np.exp(1j * theta)
    np.testing.assert_allclose(qo[..., :4], z.real, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(qo[..., 4:8], z.imag, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(qo[..., 8:], q[..., 8:])
    np.testing.assert_allclose(np.linalg.norm(ko[..., :8], axis=-1), np.linalg.norm(k[..., :8], axis=-1), rtol=1e-5)
    q2, k2 = oracle.apply_partial_rope(q, k, None, None, 8)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)


# ---------------------------------------------------------------------------
# linear attention
# ---------------------------------------------------------------------------

def test_linear_reference_rule_closed_forms():
    q, k, v, s = randn(2, 3, 5), randn(2, 3, 5), randn(2, 3, 7), randn(2, 3, 5, 7)
    o, s2 = oracle.linear_attention_decode(q, k, v, s, decay=0.0)
    np.testing.assert_allclose(s2, k[..., :, None] * v[..., None, :], rtol=1e-6)
    o, s2 = oracle.linear_attention_decode(q, k, v, s, decay=0.9)
    qk = (q * k).sum(-1, keepdims=True)
    expect = qk * v + 0.9 * np.einsum("bhd,bhdv->bhv", q.astype(np.float64), s.astype(np.float64))
    np.testing.assert_allclose(o, expect, rtol=1e-5, atol=1e-5)


def _unit(a):
    return (a / np.linalg.norm(a, axis=-1, keepdims=True)).astype(np.float32)


def test_gated_delta_invariants():
    b, hk, hv, dk, dv = 2, 2, 4, 8, 6
    q, k, v = randn(b, hk, dk), _unit(randn(b, hk, dk)), randn(b, hv, dv)
    s, g, beta = randn(b, hv, dk, dv), -np.abs(randn(b, hv)), np.abs(randn(b, hv)) % 1
    kk = np.repeat(k, hv // hk, axis=1)
    # beta = 0 => S' = e^g S
    _, s2 = oracle.gated_delta_decode(q, k, v, s, g, np.zeros_like(beta))
    np.testing.assert_allclose(s2, s * np.exp(g)[..., None, None], rtol=1e-6)
    # g = 0, beta = 0 => S' = S
    _, s2 = oracle.gated_delta_decode(q, k, v, s, np.zeros_like(g), np.zeros_like(beta))
    np.testing.assert_array_equal(s2, s)
    # |k| = 1, beta = 1 => S'^T k = v
    _, s2 = oracle.gated_delta_decode(q, k, v, s, g, np.ones_like(beta))
    np.testing.assert_allclose(np.einsum("bhd,bhdv->bhv", kk, s2), v, rtol=1e-4, atol=1e-5)
    # S = 0, beta = 1 => S' = k v^T
    _, s2 = oracle.gated_delta_decode(q, k, v, np.zeros_like(s), g, np.ones_like(beta))
    np.testing.assert_allclose(s2, kk[..., :, None] * v[..., None, :], rtol=1e-6)


def test_gated_delta_matches_transformers_recurrent_rule():
    tr = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    b, hk, hv, dk, dv = 2, 2, 4, 16, 8
    q, k, v = randn(b, hk, dk), _unit(randn(b, hk, dk)), randn(b, hv, dv)
    s, g, beta = randn(b, hv, dk, dv, scale=0.1), -np.abs(randn(b, hv)), 1 / (1 + np.exp(-randn(b, hv)))
    o, s2 = oracle.gated_delta_decode(q, k, v, s, g, beta.astype(np.float32))
    rep = hv // hk
    qq = torch.from_numpy(np.repeat(q, rep, 1) * math.sqrt(dk))[:, None]  # their rule scales q by 1/sqrt(dk)
    kk = torch.from_numpy(np.repeat(k, rep, 1))[:, None]
    out, state = tr.torch_recurrent_gated_delta_rule(
        qq, kk, torch.from_numpy(v)[:, None], torch.from_numpy(g)[:, None],
        torch.from_numpy(beta.astype(np.float32))[:, None], torch.from_numpy(s), True)
    np.testing.assert_allclose(o, out[:, 0].float().numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(s2, state.float().numpy(), rtol=1e-5, atol=1e-6)


def test_gated_delta_qk_l2norm_invariants():
    """In-kernel q/k L2 normalisation: outputs do not change when q and k are
    scaled by positive factors; with beta = 1 the new state maps the unit key
    to v for keys of any length; from S = 0 with beta = 1 the output is
    scale * cos(q, k) * v."""
    b, hk, hv, dk, dv = 2, 2, 4, 16, 6
    q, k, v = randn(b, hk, dk), randn(b, hk, dk), randn(b, hv, dv)
    s, g, beta = randn(b, hv, dk, dv), -np.abs(randn(b, hv)), np.abs(randn(b, hv)) % 1
    o1, s1 = oracle.gated_delta_decode(q, k, v, s, g, beta, qk_l2norm=True)
    o2, s2 = oracle.gated_delta_decode(q * 7.5, k * 0.5, v, s, g, beta, qk_l2norm=True)
    np.testing.assert_allclose(o2, o1, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(s2, s1, rtol=1e-4, atol=1e-5)
    o_raw, _ = oracle.gated_delta_decode(q, k, v, s, g, beta)
    assert not np.allclose(o_raw, o1, rtol=1e-2)  # the flag changes the result
    ku = np.repeat(_unit(k), hv // hk, axis=1)
    _, s3 = oracle.gated_delta_decode(q, k * 3.0, v, s, g, np.ones_like(beta), qk_l2norm=True)
    np.testing.assert_allclose(np.einsum("bhd,bhdv->bhv", ku, s3), v, rtol=1e-4, atol=1e-4)
    o4, _ = oracle.gated_delta_decode(q, k, v, np.zeros_like(s), g, np.ones_like(beta), qk_l2norm=True, q_scale=0.5)
    cos = np.repeat((_unit(q) * _unit(k)).sum(-1), hv // hk, axis=1)
    np.testing.assert_allclose(o4, 0.5 * cos[..., None] * v, rtol=1e-4, atol=1e-5)


def test_gated_delta_qk_l2norm_matches_transformers():
    tr = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    b, hk, hv, dk, dv = 2, 2, 4, 16, 8
    q, k, v = randn(b, hk, dk), randn(b, hk, dk) * 3.0, randn(b, hv, dv)
    s, g, beta = randn(b, hv, dk, dv, scale=0.1), -np.abs(randn(b, hv)), 1 / (1 + np.exp(-randn(b, hv)))
    o, s2 = oracle.gated_delta_decode(q, k, v, s, g, beta.astype(np.float32), qk_l2norm=True)
    rep = hv // hk
    out, state = tr.torch_recurrent_gated_delta_rule(
        torch.from_numpy(np.repeat(q, rep, 1))[:, None], torch.from_numpy(np.repeat(k, rep, 1))[:, None],
        torch.from_numpy(v)[:, None], torch.from_numpy(g)[:, None], torch.from_numpy(beta.astype(np.float32))[:, None],
        torch.from_numpy(s), True, use_qk_l2norm_in_kernel=True)
    np.testing.assert_allclose(o, out[:, 0].float().numpy(), rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(s2, state.float().numpy(), rtol=1e-5, atol=1e-5)


def test_gated_delta_qk_l2norm_bf16_inputs_vs_transformers_bf16_loop():
    """The in-kernel q/k L2 norm is taken in FP32 on the upcast inputs, as the
    fused recurrent kernel of flash-linear-attention does with
    use_qk_l2norm_in_kernel.  transformers' torch fallback normalises in the
    input dtype (x*x, the sum, rsqrt and the product each rounded to bf16)
    before its float32 cast.  On bf16 config-5 inputs the two agree on the
    output within the bf16 tolerance (measured max 1.6e-4 abs) and on the
    FP32 state within 5e-3 abs (measured 3.0e-3): the difference is the bf16
    rounding of the normalised q and k, which the FP32 target does not do."""
    tr = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    r = np.random.default_rng(0)
    b, hk, hv, dk, dv = 2, 16, 32, 128, 128
    q, k, v = (oracle.bf16_round(r.standard_normal(sh).astype(np.float32))
               for sh in ((b, hk, dk), (b, hk, dk), (b, hv, dv)))
    s = (r.standard_normal((b, hv, dk, dv)) * 0.1).astype(np.float32)
    g = -np.log1p(np.exp(r.standard_normal((b, hv)))).astype(np.float32)
    beta = (1 / (1 + np.exp(-r.standard_normal((b, hv))))).astype(np.float32)
    o, s2 = oracle.gated_delta_decode(q, k, v, s, g, beta, qk_l2norm=True)
    rep, bf = hv // hk, torch.bfloat16
    out, state = tr.torch_recurrent_gated_delta_rule(
        torch.from_numpy(np.repeat(q, rep, 1))[:, None].to(bf), torch.from_numpy(np.repeat(k, rep, 1))[:, None].to(bf),
        torch.from_numpy(v)[:, None].to(bf), torch.from_numpy(g)[:, None], torch.from_numpy(beta)[:, None],
        torch.from_numpy(s), True, use_qk_l2norm_in_kernel=True)
    np.testing.assert_allclose(o, out[:, 0].float().numpy(), rtol=1e-2, atol=1e-2)
    np.testing.assert_allclose(s2, state.float().numpy(), rtol=0, atol=5e-3)
    assert not np.allclose(s2, state.float().numpy(), rtol=0, atol=1e-4)  # the rounding is visible


def test_causal_conv1d_update_identity_tap_and_shift():
    """With only the newest tap set to 1 and no activation the output is the
    input, and the state shifts by one token with the input appended."""
    b, c, sl = 2, 12, 3
    x, st = randn(b, c), randn(b, c, sl)
    w = np.zeros((c, sl + 1), np.float32)
    w[:, -1] = 1.0
    out, new_state = oracle.causal_conv1d_update(x, st, w, silu_activation=False, bf16=False)
    np.testing.assert_array_equal(out, x)
    np.testing.assert_array_equal(new_state, np.concatenate([st[..., 1:], x[..., None]], -1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_causal_conv1d_update_matches_transformers(dtype):
    tr = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    b, c, sl = 2, 40, 3
    x, st, w, bias = randn(b, c), randn(b, c, sl), randn(c, sl + 1, scale=0.5), randn(c)
    bf = dtype == torch.bfloat16
    if bf:
        x, st, w, bias = (oracle.bf16_round(a) for a in (x, st, w, bias))
    for bias_ in (None, bias):
        out, new_state = oracle.causal_conv1d_update(x, st, w, bias_, bf16=bf)
        ts = torch.from_numpy(st.copy()).to(dtype)
        ref = tr.causal_conv1d_update(torch.from_numpy(x).to(dtype)[..., None], ts, torch.from_numpy(w).to(dtype),
                                      None if bias_ is None else torch.from_numpy(bias_).to(dtype), "silu")
        tol = 8e-3 if bf else 1e-5
        np.testing.assert_allclose(out, ref[..., 0].float().numpy(), rtol=tol, atol=tol)
        np.testing.assert_array_equal(new_state, ts.float().numpy())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gated_rms_norm_matches_transformers(dtype):
    tr = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    rows, d = 6, 128
    x, z, w = randn(rows, d), randn(rows, d), randn(d, scale=0.5) + 1.0
    bf = dtype == torch.bfloat16
    if bf:
        x, z, w = (oracle.bf16_round(a) for a in (x, z, w))
    out = oracle.gated_rms_norm(x, z, w, eps=1e-6, bf16=bf)
    mod = tr.Qwen3NextRMSNormGated(d, eps=1e-6).to(dtype)
    with torch.no_grad():
        mod.weight.copy_(torch.from_numpy(w).to(dtype))
        ref = mod(torch.from_numpy(x).to(dtype), torch.from_numpy(z).to(dtype)).float().numpy()
    tol = 8e-3 if bf else 1e-5
    np.testing.assert_allclose(out, ref, rtol=tol, atol=tol)


def test_gated_rms_norm_constant_rows():
    """A constant row normalises to its sign, so out = weight * sign * silu(gate)."""
    d = 16
    x = np.stack([np.full(d, 3.0), np.full(d, -0.25)]).astype(np.float32)
    z, w = randn(2, d), randn(d)
    out = oracle.gated_rms_norm(x, z, w, eps=0.0, bf16=False)
    silu = z / (1 + np.exp(-z))
    np.testing.assert_allclose(out, np.sign(x) * w * silu, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# golden vectors
# ---------------------------------------------------------------------------

def _golden(name):
    path = GOLDEN / f"{name}.npz"
    if not path.exists():
        pytest.skip(f"{path} missing (run tests/golden/make_golden.py)")
    return dict(np.load(path, allow_pickle=False))


def test_golden_moe():
    g = _golden("moe_small")
    out, idx, w = oracle.moe_decode(g["x"], g["norm_weight"], g["router_weight"], g["expert_gate"], g["expert_up"],
                                    g["expert_down"], g["shared_gate"], g["shared_up"], g["shared_down"],
                                    top_k=int(g["top_k"]), shared_expert_gate=g["shared_expert_gate"])
    assert idx.tolist() == g["out_idx"].tolist()
    np.testing.assert_allclose(w, g["out_w"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out, g["out"], rtol=1e-4, atol=1e-5)


def test_golden_dense():
    g = _golden("dense_small")
    out = oracle.dense_ffn_decode(g["x"], g["norm_weight"], g["gate_weight"], g["up_weight"], g["down_weight"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-4, atol=1e-5)


def test_golden_attention():
    g = _golden("attention_small")
    out = oracle.full_attention_decode(g["q"], g["k_cache"], g["v_cache"])
    np.testing.assert_allclose(out, g["out"], rtol=1e-5, atol=1e-6)


def test_golden_linear():
    g = _golden("linear_small")
    o, s = oracle.linear_attention_decode(g["q"], g["k"], g["v"], g["state"], decay=float(g["decay"]))
    np.testing.assert_allclose(o, g["out"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s, g["new_state"], rtol=1e-6, atol=1e-7)


def test_golden_gated_delta():
    g = _golden("gated_delta_small")
    o, s = oracle.gated_delta_decode(g["q"], g["k"], g["v"], g["state"], g["g"], g["beta"])
    np.testing.assert_allclose(o, g["out"], rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(s, g["new_state"], rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------------------
# attention cache layouts (KV append, paged KV)
# ---------------------------------------------------------------------------

def test_attention_cache_view_append_writes_one_row():
    b, cap, hkv, d = 2, 7, 2, 8
    kc, vc = randn(b, cap, hkv, d), randn(b, cap, hkv, d)
    kn, vn = randn(b, hkv, d), randn(b, hkv, d)
    for pos in (None, 3, 0):
        k, v = oracle.attention_cache_view(dict(k_cache=kc, v_cache=vc, k_new=kn, v_new=vn, cache_seqlen=pos))
        p = cap - 1 if pos is None else pos
        assert k.shape == (b, p + 1, hkv, d)
        np.testing.assert_array_equal(k[:, p], kn)
        np.testing.assert_array_equal(v[:, p], vn)
        np.testing.assert_array_equal(k[:, :p], kc[:, :p])
        np.testing.assert_array_equal(v[:, :p], vc[:, :p])
    np.testing.assert_array_equal(oracle.attention_cache_view(dict(k_cache=kc, v_cache=vc))[0], kc)
    with pytest.raises(ValueError, match="cache_seqlen must leave room"):
        oracle.attention_cache_view(dict(k_cache=kc, v_cache=vc, k_new=kn, v_new=vn, cache_seqlen=cap))
    with pytest.raises(ValueError, match="given together"):
        oracle.attention_cache_view(dict(k_cache=kc, v_cache=vc, k_new=kn))


def test_attention_cache_view_paged_gathers_the_cut_cache():
    """Cut a contiguous cache into blocks, scatter them over a shuffled pool
    with garbage in the unused blocks: the paged view gathers the original
    back; an out-of-pool id reads as zeros; an append lands in its block."""
    b, t, hkv, d, bs = 2, 40, 2, 8, 16
    nb_row = (t + bs - 1) // bs
    kc, vc = randn(b, nb_row * bs, hkv, d), randn(b, nb_row * bs, hkv, d)
    pool_n = 2 * b * nb_row
    perm = np.random.default_rng(5).permutation(pool_n)[: b * nb_row].reshape(b, nb_row)
    kp, vp = randn(pool_n, bs, hkv, d), randn(pool_n, bs, hkv, d)
    for r in range(b):
        for j in range(nb_row):
            kp[perm[r, j]] = kc[r, j * bs:(j + 1) * bs]
            vp[perm[r, j]] = vc[r, j * bs:(j + 1) * bs]
    k, v = oracle.attention_cache_view(dict(k_cache=kp, v_cache=vp, block_table=perm.astype(np.int32), seq_len=t))
    np.testing.assert_array_equal(k, kc[:, :t])
    np.testing.assert_array_equal(v, vc[:, :t])
    bad = perm.copy()
    bad[1, 1] = pool_n + 3
    k, _ = oracle.attention_cache_view(dict(k_cache=kp, v_cache=vp, block_table=bad, seq_len=t))
    assert np.all(k[1, bs:2 * bs] == 0) and np.array_equal(k[0], kc[0, :t])
    kn, vn = randn(b, hkv, d), randn(b, hkv, d)
    k, v = oracle.attention_cache_view(dict(k_cache=kp, v_cache=vp, block_table=perm, seq_len=t, k_new=kn, v_new=vn))
    np.testing.assert_array_equal(k[:, t - 1], kn)
    np.testing.assert_array_equal(k[:, : t - 1], kc[:, : t - 1])


# ---------------------------------------------------------------------------
# decode_layer: an independent float64 torch composition of ops.py:701-748
# ---------------------------------------------------------------------------

def _bf(t, on):
    return t.to(torch.bfloat16).to(torch.float64) if on else t


def _moe64(x, m, k):
    """MoE in float64 torch (library ops), shared gate on the post-norm input."""
    xn = F.rms_norm(x, (x.shape[1],), weight=t64(m["norm_weight"]), eps=1e-6)
    tv, ti = torch.topk(F.linear(xn, t64(m["router_weight"])), k, dim=-1)
    tw = torch.softmax(tv, -1)
    shared = _swiglu64(xn, t64(m["shared_gate"]), t64(m["shared_up"]), t64(m["shared_down"]))
    if m.get("shared_expert_gate") is not None:
        shared = shared * torch.sigmoid(xn @ t64(m["shared_expert_gate"]).reshape(-1, 1))
    out = x + shared
    for b in range(x.shape[0]):
        for s in range(k):
            e = int(ti[b, s])
            out[b] += tw[b, s] * _swiglu64(xn[b:b + 1], t64(m["expert_gate"][e]), t64(m["expert_up"][e]),
                                           t64(m["expert_down"][e]))[0]
    return out, ti


def _gdr64(la):
    """Gated delta rule through transformers' recurrent loop (it scales q by
    1/sqrt(dk), undone here when q/k are not normalised in the kernel)."""
    tr = pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    q, k, v = t64(la["q"]), t64(la["k"]), t64(la["v"])
    rep = v.shape[1] // q.shape[1]
    dk = q.shape[-1]
    l2 = bool(la.get("qk_l2norm", False))
    if l2:
        scale = la.get("q_scale") or 1.0 / math.sqrt(dk)
        q = q * (scale * math.sqrt(dk))  # q's own length is normalised away; only the scale remains
    else:
        q = q * math.sqrt(dk)
    out, state = tr.torch_recurrent_gated_delta_rule(
        q.repeat_interleave(rep, 1)[:, None], k.repeat_interleave(rep, 1)[:, None], v[:, None],
        t64(la["g"])[:, None], t64(la["beta"])[:, None], t64(la["state"]), True, use_qk_l2norm_in_kernel=l2)
    return out[:, 0], state


def _decode_layer64(hidden, kind, *, moe=None, dense=None, attn=None, lin=None, k=8, rounding=False):
    h = t64(hidden)
    if kind == "full_attention":
        q, kc, vc = t64(attn["q"]), t64(attn["k_cache"]), t64(attn["v_cache"])
        a = F.scaled_dot_product_attention(q[:, :, None], kc.transpose(1, 2), vc.transpose(1, 2),
                                           scale=attn.get("scale"), enable_gqa=True)[:, :, 0]
        mixer = _bf(a, rounding)
    else:
        mixer, state = _gdr64(lin)
        mixer = _bf(mixer, rounding)
    proj = (attn if kind == "full_attention" else lin).get("out_proj")
    mixer = mixer.reshape(h.shape[0], -1)
    if proj is not None:
        mixer = _bf(F.linear(mixer, t64(proj)), rounding)
    mixer = mixer.reshape(h.shape)
    resid = _bf(h + mixer, rounding)
    if dense is not None:
        xn = F.rms_norm(resid, (h.shape[1],), weight=t64(dense["norm_weight"]), eps=1e-6)
        return resid + _swiglu64(xn, t64(dense["gate_weight"]), t64(dense["up_weight"]), t64(dense["down_weight"])), \
            None, mixer
    out, idx = _moe64(resid, moe, k)
    return out, idx, mixer


def _layer_inputs(B=2, H=32, heads=4, dk=8, dv=16, seed=0):
    r = np.random.default_rng(seed)

    def rn(*shape, scale=1.0):
        return (r.standard_normal(shape) * scale).astype(np.float32)

    moe = dict(norm_weight=rn(H, scale=0.1) + 1, router_weight=rn(12, H, scale=0.3),
               expert_gate=rn(12, 10, H, scale=0.3), expert_up=rn(12, 10, H, scale=0.3),
               expert_down=rn(12, H, 10, scale=0.3), shared_gate=rn(14, H, scale=0.3),
               shared_up=rn(14, H, scale=0.3), shared_down=rn(H, 14, scale=0.3),
               shared_expert_gate=rn(H, scale=0.3))
    dense = dict(norm_weight=rn(H, scale=0.1) + 1, gate_weight=rn(40, H, scale=0.3), up_weight=rn(40, H, scale=0.3),
                 down_weight=rn(H, 40, scale=0.3))
    lin = dict(q=_unit(rn(B, heads // 2, dk)), k=_unit(rn(B, heads // 2, dk)), v=rn(B, heads, dv),
               state=rn(B, heads, dk, dv, scale=0.1), g=-np.abs(rn(B, heads)),
               beta=(1 / (1 + np.exp(-rn(B, heads)))).astype(np.float32), out_proj=rn(H, heads * dv, scale=0.2))
    attn = dict(q=rn(B, 8, dk), k_cache=rn(B, 9, 2, dk), v_cache=rn(B, 9, 2, dk), scale=0.4,
                out_proj=rn(H, 8 * dk, scale=0.2))
    return rn(B, H), moe, dense, lin, attn


@pytest.mark.parametrize("rounding", [False, True])
@pytest.mark.parametrize("ffn", ["moe", "dense"])
@pytest.mark.parametrize("kind", ["linear_attention", "full_attention"])
def test_decode_layer_matches_float64_composition(kind, ffn, rounding):
    """oracle.decode_layer against ops.py:701-748 composed from library ops in
    float64: mixer, then out_proj, then the residual add, then the FFN/MoE
    with its own residual.  With rounding, both round to bfloat16 at the same
    points (mixer output, projection, residual sum)."""
    pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    x, moe, dense, lin, attn = _layer_inputs(seed=3)
    if rounding:
        x = oracle.bf16_round(x)
    mix = dict(linear_attention=lin) if kind == "linear_attention" else dict(full_attention=attn)
    ffn_kw = dict(moe=moe) if ffn == "moe" else dict(dense_ffn=dense)
    res = oracle.decode_layer(x, kind=kind, top_k=3, round_to_bf16=rounding, **mix, **ffn_kw)
    ref, idx, mixer = _decode_layer64(x, kind, moe=moe if ffn == "moe" else None, dense=dense if ffn == "dense" else None,
                                      attn=attn, lin=lin, k=3, rounding=rounding)
    tol = 2e-2 if rounding else 2e-4
    np.testing.assert_allclose(res["hidden"], ref.numpy(), rtol=tol, atol=tol)
    mixer_out = res["linear_output"] if kind == "linear_attention" else res["attention_output"]
    np.testing.assert_allclose(mixer_out, mixer.numpy(), rtol=tol, atol=tol)
    if ffn == "moe":
        assert res["router_indices"].tolist() == idx.tolist()
    else:
        assert res["router_indices"] is None


def test_decode_layer_wiring_mistakes_are_caught():
    """The float64 composition separates the plausible wiring mistakes: the
    residual added after the FFN instead of before it, the projection
    skipped, and the mixer output dropped."""
    pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    x, moe, dense, lin, attn = _layer_inputs(seed=4)
    ref, _, mixer = _decode_layer64(x, "linear_attention", dense=dense, lin=lin)
    h = t64(x)
    xn = F.rms_norm(h, (h.shape[1],), weight=t64(dense["norm_weight"]), eps=1e-6)
    late_residual = h + mixer + _swiglu64(xn, t64(dense["gate_weight"]), t64(dense["up_weight"]),
                                          t64(dense["down_weight"]))
    no_mixer = torch.from_numpy(oracle.dense_ffn_decode(x, *(dense[n] for n in (
        "norm_weight", "gate_weight", "up_weight", "down_weight")))).double()
    res = oracle.decode_layer(x, kind="linear_attention", dense_ffn=dense, linear_attention=lin, round_to_bf16=False)
    np.testing.assert_allclose(res["hidden"], ref.numpy(), rtol=2e-4, atol=2e-4)
    for wrong in (late_residual, no_mixer):
        assert not np.allclose(res["hidden"], wrong.numpy(), rtol=1e-2, atol=1e-2)


def test_decode_layer_special_cases():
    x, moe, dense, lin, attn = _layer_inputs(seed=5)
    x = oracle.bf16_round(x)
    # zero out_proj: the mixer adds nothing, so the layer is the MoE of its input
    lin0 = dict(lin, out_proj=np.zeros_like(lin["out_proj"]))
    res = oracle.decode_layer(x, kind="linear_attention", moe=moe, linear_attention=lin0, top_k=3)
    out, idx, w = oracle.moe_decode(x, *(moe[n] for n in ("norm_weight", "router_weight", "expert_gate", "expert_up",
                                                          "expert_down", "shared_gate", "shared_up", "shared_down")),
                                    top_k=3, shared_expert_gate=moe["shared_expert_gate"])
    np.testing.assert_array_equal(res["hidden"], out)
    assert res["router_indices"].tolist() == idx.tolist()
    np.testing.assert_array_equal(res["router_weights"], w)
    # zero-gate dense FFN: the FFN adds nothing, so hidden = round(x + mixer output)
    d0 = dict(dense, gate_weight=np.zeros_like(dense["gate_weight"]))
    res = oracle.decode_layer(x, kind="full_attention", dense_ffn=d0, full_attention=attn)
    np.testing.assert_array_equal(res["hidden"], oracle.bf16_round(x + res["attention_output"]))
    # the state of the linear layer is the gated delta rule's
    res = oracle.decode_layer(x, kind="linear_attention", dense_ffn=dense, linear_attention=lin)
    _, s = oracle.gated_delta_decode(lin["q"], lin["k"], lin["v"], lin["state"], lin["g"], lin["beta"])
    np.testing.assert_array_equal(res["linear_state"], s)
    # without out_proj the output is reshaped onto the hidden size (8 heads x 4 = 32 = H)
    attn_r = dict(q=randn(2, 8, 4), k_cache=randn(2, 5, 2, 4), v_cache=randn(2, 5, 2, 4))
    res = oracle.decode_layer(x, kind="full_attention", dense_ffn=d0, full_attention=attn_r)
    a = oracle.bf16_round(oracle.full_attention_decode(attn_r["q"], attn_r["k_cache"], attn_r["v_cache"]))
    np.testing.assert_array_equal(res["attention_output"], a.reshape(x.shape))
    # qk_l2norm and q_scale reach the recurrence
    lin_n = dict(lin, q=lin["q"] * 3.0, qk_l2norm=True, q_scale=0.25)
    res = oracle.decode_layer(x, kind="linear_attention", dense_ffn=dense, linear_attention=lin_n)
    o, s = oracle.gated_delta_decode(lin_n["q"], lin["k"], lin["v"], lin["state"], lin["g"], lin["beta"],
                                     qk_l2norm=True, q_scale=0.25)
    np.testing.assert_array_equal(res["linear_state"], s)
    # KV append through decode_layer reads the new row
    kn, vn = randn(2, 2, 8), randn(2, 2, 8)
    res = oracle.decode_layer(x, kind="full_attention", dense_ffn=d0,
                              full_attention=dict(attn, k_new=kn, v_new=vn, cache_seqlen=4))
    kc = attn["k_cache"].copy()
    vc = attn["v_cache"].copy()
    kc[:, 4], vc[:, 4] = kn, vn
    a = oracle.bf16_round(oracle.full_attention_decode(attn["q"], kc[:, :5], vc[:, :5], scale=attn["scale"]))
    a = oracle.bf16_round(a.reshape(2, -1) @ attn["out_proj"].T)
    np.testing.assert_array_equal(res["attention_output"], a)


def test_decode_layer_errors_match_ops():
    """The ValueError texts of ops.py:720-721, 725-726, 730-731, 738-739."""
    x, moe, dense, lin, attn = _layer_inputs(seed=6)
    with pytest.raises(ValueError, match="full_attention inputs are required for full_attention layers"):
        oracle.decode_layer(x, kind="full_attention", moe=moe)
    with pytest.raises(ValueError, match="linear_attention inputs are required for linear_attention layers"):
        oracle.decode_layer(x, kind="linear_attention", moe=moe)
    with pytest.raises(ValueError, match="unsupported layer_type: vision"):
        oracle.decode_layer(x, kind="vision", moe=moe)
    with pytest.raises(ValueError, match="either moe or dense_ffn weights are required"):
        oracle.decode_layer(x, kind="linear_attention", linear_attention=lin)
    with pytest.raises(ValueError, match="qk_l2norm needs the gated delta rule"):
        oracle.decode_layer(x, kind="linear_attention", moe=moe,
                            linear_attention=dict(q=lin["q"], k=lin["k"], v=lin["v"][:, :2], state=lin["state"],
                                                  qk_l2norm=True))


def test_rms_norm_linear_matches_float64_torch():
    """rms_norm_linear against F.linear(F.rms_norm(x).to(bf16)) in float64
    torch (the reference's rms_norm rounds its result to the input dtype,
    reference.py:10-13), unrounded and rounded; an identity projection gives
    the (rounded) norm itself; scaling x leaves the output unchanged."""
    r = np.random.default_rng(11)
    x = r.standard_normal((3, 48)).astype(np.float32)
    nw = (1 + 0.1 * r.standard_normal(48)).astype(np.float32)
    w = (0.2 * r.standard_normal((20, 48))).astype(np.float32)
    xn64 = F.rms_norm(t64(x), (48,), weight=t64(nw), eps=1e-6)
    np.testing.assert_allclose(oracle.rms_norm_linear(x, nw, w, round_to_bf16=False),
                               F.linear(xn64, t64(w)).numpy(), rtol=1e-5, atol=1e-5)
    ref_b = F.linear(xn64.to(torch.bfloat16).double(), t64(w)).to(torch.bfloat16).double()
    np.testing.assert_allclose(oracle.rms_norm_linear(x, nw, w), ref_b.numpy(), rtol=1e-2, atol=1e-2)
    eye = np.eye(48, dtype=np.float32)
    np.testing.assert_array_equal(oracle.rms_norm_linear(x, nw, eye), oracle.bf16_round(oracle.rms_norm(x, nw)))
    np.testing.assert_allclose(oracle.rms_norm_linear(4.0 * x, nw, w, round_to_bf16=False),
                               oracle.rms_norm_linear(x, nw, w, round_to_bf16=False), rtol=1e-5, atol=1e-5)
    # a dropped norm weight or a transposed projection fails
    assert not np.allclose(oracle.rms_norm_linear(x, np.ones_like(nw), w), ref_b.numpy(), rtol=1e-2, atol=1e-2)


def test_decode_layer_projects_its_own_inputs():
    """With qkv_proj / in_proj, decode_layer computes the mixer's inputs from
    the layer input: a full-attention layer equals the layer given q, k_new
    and v_new cut from rms_norm(hidden) @ qkv_proj^T (in that order), and a
    linear layer equals the layer given q, k, v cut the same way; both
    against an independent float64 torch composition of the cuts too."""
    pytest.importorskip("transformers.models.qwen3_next.modeling_qwen3_next")
    x, moe, dense, lin, attn = _layer_inputs(seed=8)
    x = oracle.bf16_round(x)
    r = np.random.default_rng(12)
    nw = (1 + 0.1 * r.standard_normal(32)).astype(np.float32)
    # full attention: 8 q heads and 2 kv heads of 8 -> 96 rows
    wqkv = (0.3 * r.standard_normal((96, 32))).astype(np.float32)
    a_in = dict(attn, q=None, qkv_proj=wqkv, input_norm=nw, cache_seqlen=6)
    res = oracle.decode_layer(x, kind="full_attention", dense_ffn=dense, full_attention=a_in)
    qkv = oracle.rms_norm_linear(x, nw, wqkv)
    cut = dict(attn, q=qkv[:, :64].reshape(2, 8, 8), k_new=qkv[:, 64:80].reshape(2, 2, 8),
               v_new=qkv[:, 80:].reshape(2, 2, 8), cache_seqlen=6)
    want = oracle.decode_layer(x, kind="full_attention", dense_ffn=dense, full_attention=cut)
    np.testing.assert_array_equal(res["hidden"], want["hidden"])
    np.testing.assert_array_equal(res["attention_output"], want["attention_output"])
    xn = F.rms_norm(t64(x), (32,), weight=t64(nw), eps=1e-6).to(torch.bfloat16).double()
    qkv64 = F.linear(xn, t64(wqkv)).to(torch.bfloat16).double()
    np.testing.assert_allclose(qkv, qkv64.numpy(), rtol=1e-2, atol=1e-2)
    swapped = dict(cut, k_new=cut["v_new"], v_new=cut["k_new"])
    wrong = oracle.decode_layer(x, kind="full_attention", dense_ffn=dense, full_attention=swapped)
    assert not np.allclose(res["attention_output"], wrong["attention_output"], rtol=1e-2, atol=1e-2)
    # linear attention: 2 k heads of 8 (q, k) and 4 v heads of 16 -> 96 rows
    win = (0.3 * r.standard_normal((96, 32))).astype(np.float32)
    l_in = dict(lin, q=None, k=None, v=None, in_proj=win, input_norm=nw, qk_l2norm=True)
    res = oracle.decode_layer(x, kind="linear_attention", moe=moe, linear_attention=l_in, top_k=3)
    qkv = oracle.rms_norm_linear(x, nw, win)
    cut = dict(lin, q=qkv[:, :16].reshape(2, 2, 8), k=qkv[:, 16:32].reshape(2, 2, 8),
               v=qkv[:, 32:].reshape(2, 4, 16), qk_l2norm=True)
    want = oracle.decode_layer(x, kind="linear_attention", moe=moe, linear_attention=cut, top_k=3)
    np.testing.assert_array_equal(res["hidden"], want["hidden"])
    np.testing.assert_array_equal(res["linear_state"], want["linear_state"])
    with pytest.raises(ValueError, match="qkv_proj must have"):
        oracle.decode_layer(x, kind="full_attention", dense_ffn=dense,
                            full_attention=dict(a_in, qkv_proj=wqkv[:30]))
    with pytest.raises(ValueError, match="in_proj must have"):
        oracle.decode_layer(x, kind="linear_attention", moe=moe, linear_attention=dict(l_in, in_proj=win[:70]))


def test_pinning_table_covers_every_function():
    for name in oracle.decode_oracle.__all__:
        if name in ("as_f32", "bf16_bits", "bf16_round", "PINNING", "silu", "softmax"):
            continue
        assert name in oracle.PINNING, name
