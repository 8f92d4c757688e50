"""GPU parity: linear-attention decode (reference rule and gated delta rule).

Tolerances (task): bf16 outputs atol/rtol 1e-2; FP32 recurrent state 1e-4.
"""

import numpy as np
import pytest
import torch

import mega_kernel_qwen36 as mk
import oracle
from tests.inputs import (assert_close_out, assert_close_state, make_gated_delta, make_linear_reference_rule, np32)

pytestmark = pytest.mark.gpu


def _oracle_ref(inp):
    return oracle.linear_attention_decode(np32(inp.q), np32(inp.k), np32(inp.v), np32(inp.state), decay=inp.decay)


def _oracle_gated(inp):
    return oracle.gated_delta_decode(np32(inp.q), np32(inp.k), np32(inp.v), np32(inp.state), np32(inp.g),
                                     np32(inp.beta))


def test_linear_attention_reference_rule_reference_shape():
    # test_cuda_ops.py:93-111 shape: B 2, H 3, Dk 8, Dv 10, decay 0.92
    inp = make_linear_reference_rule()
    state_before = inp.state.clone()
    out, new_state = mk.linear_attention_decode(inp)
    ref_out, ref_state = _oracle_ref(inp)
    assert out.dtype == inp.q.dtype
    assert_close_out(out, ref_out)
    assert_close_state(new_state, ref_state)
    assert torch.equal(inp.state, state_before)  # functional: input state untouched


@pytest.mark.parametrize("shape", [(1, 4, 128, 128), (3, 5, 64, 200), (2, 2, 256, 33)])
def test_linear_attention_reference_rule_shapes(shape):
    b, h, dk, dv = shape
    inp = make_linear_reference_rule(batch=b, heads=h, key_dim=dk, value_dim=dv, decay=0.8, seed=sum(shape))
    out, new_state = mk.linear_attention_decode(inp)
    ref_out, ref_state = _oracle_ref(inp)
    assert_close_out(out, ref_out)
    assert_close_state(new_state, ref_state)


@pytest.mark.parametrize("batch", [1, 8])
def test_gated_delta_config5(batch):
    """Config 5: 16 q/k heads, 32 v heads, D 128, FP32 state."""
    inp = make_gated_delta(batch=batch)
    out, new_state = mk.linear_attention_decode(inp)
    ref_out, ref_state = _oracle_gated(inp)
    assert out.shape == inp.v.shape
    assert_close_out(out, ref_out)
    assert_close_state(new_state, ref_state)


def test_gated_delta_in_place_matches_functional():
    inp = make_gated_delta(batch=2, seed=3)
    out, new_state = mk.linear_attention_decode(inp)
    st = inp.state.clone()
    out2 = mk._C.gated_delta_decode_(inp.q, inp.k, inp.v, st, inp.g, inp.beta)
    assert torch.equal(out, out2)
    assert torch.equal(new_state, st)


def test_gated_delta_invariants_on_gpu():
    # beta = 0 => S' = e^g S ; |k| = 1, beta = 1 => S'^T k = v
    inp = make_gated_delta(batch=1, k_heads=2, v_heads=4, key_dim=64, value_dim=32, seed=4)
    zero_beta = mk.LinearAttentionInputs(q=inp.q, k=inp.k, v=inp.v, state=inp.state, g=inp.g,
                                         beta=torch.zeros_like(inp.beta))
    _, s = mk.linear_attention_decode(zero_beta)
    expect = np32(inp.state) * np.exp(np32(inp.g))[:, :, None, None]
    assert_close_state(s, expect)
    k32 = torch.nn.functional.normalize(inp.k.float(), dim=-1)
    one_beta = mk.LinearAttentionInputs(q=inp.q, k=k32, v=inp.v.float(), state=inp.state, g=inp.g,
                                        beta=torch.ones_like(inp.beta))
    qf = inp.q.float()
    one_beta = mk.LinearAttentionInputs(q=qf, k=k32, v=inp.v.float(), state=inp.state, g=inp.g,
                                        beta=torch.ones_like(inp.beta))
    _, s = mk.linear_attention_decode(one_beta)
    kk = k32.repeat_interleave(2, dim=1)  # v head j reads k head j // 2
    stk = torch.einsum("bhd,bhdv->bhv", kk, s)
    torch.testing.assert_close(stk.cpu(), inp.v.float().cpu(), atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("batch,hk,hv,dk,dv,q_scale", [
    (1, 16, 32, 128, 128, None),   # config 5, default scale 1/sqrt(128)
    (8, 16, 32, 128, 128, None),
    (2, 2, 4, 64, 200, 0.3),       # ragged value columns
    (3, 1, 3, 256, 40, None),      # key_dim at the kernel's maximum
    (1, 2, 2, 40, 64, 1.0),        # key_dim below one wave
])
def test_gated_delta_qk_l2norm_in_kernel(batch, hk, hv, dk, dv, q_scale):
    """q and k of arbitrary length, L2-normalised inside the kernel (FP32)
    and q scaled: output and state against the oracle's qk_l2norm form, and
    the in-place entry point agrees with the functional one bit for bit."""
    inp = make_gated_delta(batch=batch, k_heads=hk, v_heads=hv, key_dim=dk, value_dim=dv, seed=dk + dv)
    g = torch.Generator().manual_seed(batch * 31 + dk)
    fq = (torch.rand(batch, hk, 1, generator=g) * 5 + 0.2).to("cuda")
    fk = (torch.rand(batch, hk, 1, generator=g) * 5 + 0.2).to("cuda")
    q = (inp.q.float() * fq).to(inp.q.dtype)
    k = (inp.k.float() * fk).to(inp.k.dtype)
    normed = mk.LinearAttentionInputs(q=q, k=k, v=inp.v, state=inp.state, g=inp.g, beta=inp.beta, qk_l2norm=True,
                                      q_scale=q_scale)
    out, new_state = mk.linear_attention_decode(normed)
    ref_out, ref_state = oracle.gated_delta_decode(np32(q), np32(k), np32(inp.v), np32(inp.state), np32(inp.g),
                                                   np32(inp.beta), qk_l2norm=True, q_scale=q_scale)
    assert_close_out(out, ref_out)
    assert_close_state(new_state, ref_state)
    st = inp.state.clone()
    scale = q_scale if q_scale is not None else dk ** -0.5
    out2 = mk._C.gated_delta_decode_(q, k, inp.v, st, inp.g, inp.beta, qk_l2norm=True, q_scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    assert torch.equal(new_state, st)


def test_gated_delta_qk_l2norm_requires_gated_rule():
    inp = make_linear_reference_rule()
    with pytest.raises(ValueError, match="qk_l2norm"):
        mk.linear_attention_decode(mk.LinearAttentionInputs(q=inp.q, k=inp.k, v=inp.v, state=inp.state,
                                                            qk_l2norm=True))
