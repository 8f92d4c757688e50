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


def test_pinning_table_covers_every_function():
    for name in ("rms_norm", "topk_desc", "moe_decode", "dense_ffn_decode", "apply_partial_rope",
                 "full_attention_decode", "linear_attention_decode", "gated_delta_decode", "decode_layer"):
        assert name in oracle.PINNING
