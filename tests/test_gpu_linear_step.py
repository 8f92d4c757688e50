"""GPU parity: the ops around the gated delta recurrence in the Qwen3.6
linear-attention step -- the causal conv1d state update (width 4, SiLU) and
the gated RMS norm on the output -- against the oracle's restatements, which
are pinned against transformers' own functions on the CPU.

Tolerances (task): bf16 outputs atol/rtol 1e-2; the conv state is a copy of
inputs and must match bit for bit.
"""

import numpy as np
import pytest
import torch

import mega_kernel_qwen36 as mk
import oracle
from mega_kernel_qwen36 import _lib
from tests.inputs import assert_close_out, np32

pytestmark = pytest.mark.gpu

# Qwen3.6-35B-A3B: q and k 16 heads x 128, v 32 heads x 128 -> 8192 conv channels.
QWEN_CHANNELS = 2 * 16 * 128 + 32 * 128


def _rand(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to("cuda", dtype)


@pytest.mark.parametrize("batch,channels,state_len,dtype,bias,act", [
    (1, QWEN_CHANNELS, 3, torch.bfloat16, False, True),
    (8, QWEN_CHANNELS, 3, torch.bfloat16, False, True),
    (3, 1000, 3, torch.float16, True, True),
    (2, 300, 5, torch.float32, True, False),
    (1, 64, 1, torch.bfloat16, False, True),
])
def test_causal_conv1d_update(batch, channels, state_len, dtype, bias, act):
    x = _rand((batch, channels), 1 + channels, dtype)
    st = _rand((batch, channels, state_len), 2 + channels, dtype)
    w = _rand((channels, state_len + 1), 3 + channels, dtype, 0.5)
    b = _rand((channels,), 4 + channels, dtype) if bias else None
    ref_out, ref_state = oracle.causal_conv1d_update(np32(x), np32(st), np32(w), None if b is None else np32(b),
                                                     silu_activation=act, bf16=dtype == torch.bfloat16)
    out = mk.causal_conv1d_update(x, st, w, b, activation="silu" if act else None)
    torch.cuda.synchronize()
    assert out.shape == x.shape and out.dtype == dtype
    assert_close_out(out, ref_out)
    np.testing.assert_array_equal(np32(st), ref_state)  # the window shifted by one token


def test_causal_conv1d_update_two_steps_through_c_abi():
    """Two tokens in a row through mkq_causal_conv1d_update: the second step
    convolves over the state the first one left."""
    lib = _lib.load_library()
    b, c, sl = 2, QWEN_CHANNELS, 3
    st = _rand((b, c, sl), 11, torch.bfloat16)
    w = _rand((c, sl + 1), 12, torch.bfloat16, 0.5)
    ref_state = np32(st)
    for step in range(2):
        x = _rand((b, c), 13 + step, torch.bfloat16)
        out = torch.empty_like(x)
        rc = lib.mkq_causal_conv1d_update(_lib.MKQ_DTYPE_BF16, x.data_ptr(), st.data_ptr(), w.data_ptr(), None,
                                          out.data_ptr(), b, c, sl, 1, torch.cuda.current_stream().cuda_stream)
        assert rc == _lib.MKQ_OK, lib.mkq_last_error()
        torch.cuda.synchronize()
        ref_out, ref_state = oracle.causal_conv1d_update(np32(x), ref_state, np32(w))
        assert_close_out(out, ref_out)
        np.testing.assert_array_equal(np32(st), ref_state)


@pytest.mark.parametrize("rows,dim,dtype", [
    (32, 128, torch.bfloat16),     # config 5 at batch 1: 32 v heads of 128
    (256, 128, torch.bfloat16),    # batch 8
    (7, 100, torch.float16),       # dim not a multiple of the wave
    (5, 384, torch.float32),
])
def test_gated_rms_norm(rows, dim, dtype):
    x = _rand((rows, dim), 21 + dim, dtype)
    z = _rand((rows, dim), 22 + dim, dtype, 2.0)
    w = _rand((dim,), 23 + dim, dtype, 0.3) + 1.0
    out = mk.gated_rms_norm(x, z, w, eps=1e-6)
    torch.cuda.synchronize()
    ref = oracle.gated_rms_norm(np32(x), np32(z), np32(w), eps=1e-6, bf16=dtype == torch.bfloat16)
    assert out.shape == x.shape and out.dtype == dtype
    assert_close_out(out, ref)


def test_gated_rms_norm_head_layout():
    """[batch, heads, dim] input, as the linear-attention output is laid out:
    each (batch, head) row is normalised on its own."""
    x = _rand((2, 32, 128), 31, torch.bfloat16)
    z = _rand((2, 32, 128), 32, torch.bfloat16)
    w = _rand((128,), 33, torch.bfloat16, 0.3) + 1.0
    out = mk.gated_rms_norm(x, z, w)
    torch.cuda.synchronize()
    ref = oracle.gated_rms_norm(np32(x).reshape(-1, 128), np32(z).reshape(-1, 128), np32(w))
    assert_close_out(out.reshape(-1, 128), ref)


def _step_case(batch, hk, hv, dk, dv, dtype, seed):
    c = 2 * hk * dk + hv * dv
    g = torch.Generator().manual_seed(seed)

    def r(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to("cuda", dtype)

    x = r(batch, c)
    conv_state = r(batch, c, 3)
    conv_w = r(c, 4, scale=0.5)
    state = (torch.randn(batch, hv, dk, dv, generator=g) * 0.1).cuda()
    gg = -torch.nn.functional.softplus(torch.randn(batch, hv, generator=g)).cuda()
    beta = torch.sigmoid(torch.randn(batch, hv, generator=g)).cuda()
    z = r(batch, hv, dv)
    nw = r(dv, scale=0.2) + 1.0
    return x, conv_state, conv_w, state, gg, beta, z, nw


@pytest.mark.parametrize("batch,hk,hv,dk,dv,dtype", [
    (1, 16, 32, 128, 128, torch.bfloat16),   # Qwen3.6-35B-A3B linear attention
    (8, 16, 32, 128, 128, torch.bfloat16),
    (3, 2, 4, 64, 32, torch.float16),
])
def test_linear_attention_step_equals_composition(batch, hk, hv, dk, dv, dtype):
    """The one-call step (q/k/v read from the conv output in place, states
    updated in place) is bit-identical to composing the separate ops on
    copies, and agrees with the oracle's chain of restatements."""
    x, cs, cw, st, gg, beta, z, nw = _step_case(batch, hk, hv, dk, dv, dtype, 700 + batch)
    cs2, st2 = cs.clone(), st.clone()
    np_cs, np_st = np32(cs), np32(st)
    out = mk.linear_attention_step(x, cs, cw, st, gg, beta, z, nw, k_heads=hk)
    mixed = mk.causal_conv1d_update(x, cs2, cw)
    q = mixed[:, :hk * dk].reshape(batch, hk, dk)
    k = mixed[:, hk * dk:2 * hk * dk].reshape(batch, hk, dk)
    v = mixed[:, 2 * hk * dk:].reshape(batch, hv, dv)
    o, new_state = mk.linear_attention_decode(mk.LinearAttentionInputs(q=q, k=k, v=v, state=st2, g=gg, beta=beta,
                                                                       qk_l2norm=True))
    want = mk.gated_rms_norm(o, z, nw)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    assert torch.equal(cs, cs2)
    assert torch.equal(st, new_state)
    bf = dtype == torch.bfloat16
    rnd = oracle.bf16_round if bf else (lambda a: a)
    m, ref_cs = oracle.causal_conv1d_update(np32(x), np_cs, np32(cw), bf16=bf)
    rq = m[:, :hk * dk].reshape(batch, hk, dk)
    rk = m[:, hk * dk:2 * hk * dk].reshape(batch, hk, dk)
    rv = m[:, 2 * hk * dk:].reshape(batch, hv, dv)
    ro, _ = oracle.gated_delta_decode(rq, rk, rv, np_st, np32(gg), np32(beta), qk_l2norm=True)
    ref = oracle.gated_rms_norm(rnd(ro), np32(z), np32(nw), bf16=bf)
    assert_close_out(out, ref)
    np.testing.assert_array_equal(np32(cs), ref_cs)
    # The state against the oracle's recurrence on the device's own conv
    # output (the conv is pinned on its own above; the oracle does not round
    # to f16 between the ops), to the FP32 state tolerance.
    _, ref_st = oracle.gated_delta_decode(np32(q), np32(k), np32(v), np_st, np32(gg), np32(beta), qk_l2norm=True)
    np.testing.assert_allclose(st.cpu().numpy(), ref_st, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("batch,hk,hv,dk,dv,state_len,bias,dtype", [
    (2, 16, 32, 128, 128, 3, False, torch.bfloat16),  # Qwen3.6 heads, two rows
    (2, 2, 6, 64, 96, 3, True, torch.bfloat16),       # a ragged last column slice, rep 3
    (1, 1, 2, 200, 40, 5, True, torch.float16),       # width 6 (the 8-tap variant), key_dim > 128
    (2, 1, 3, 64, 320, 3, False, torch.bfloat16),     # value_dim > 256: the row norm reads z and the weight itself
])
def test_linear_attention_step_two_steps_equal_composition(batch, hk, hv, dk, dv, state_len, bias, dtype):
    """Two steps in a row through the one launch (conv state rewritten by the
    last workgroup reading each q/k head, the arrival counts left at zero by
    the first call) are bit-identical to two rounds of the separate ops."""
    c = 2 * hk * dk + hv * dv
    g = torch.Generator().manual_seed(900 + dk)

    def r(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to("cuda", dtype)

    cs = r(batch, c, state_len)
    cw = r(c, state_len + 1, scale=0.5)
    cb = r(c, scale=0.1) if bias else None
    st = (torch.randn(batch, hv, dk, dv, generator=g) * 0.1).cuda()
    nw = r(dv, scale=0.2) + 1.0
    cs2, st2 = cs.clone(), st.clone()
    for step in range(2):
        x = r(batch, c)
        z = r(batch, hv, dv)
        gg = -torch.nn.functional.softplus(torch.randn(batch, hv, generator=g)).cuda()
        beta = torch.sigmoid(torch.randn(batch, hv, generator=g)).cuda()
        out = mk.linear_attention_step(x, cs, cw, st, gg, beta, z, nw, k_heads=hk, conv_bias=cb)
        mixed = mk.causal_conv1d_update(x, cs2, cw, bias=cb)
        q = mixed[:, :hk * dk].reshape(batch, hk, dk)
        k = mixed[:, hk * dk:2 * hk * dk].reshape(batch, hk, dk)
        v = mixed[:, 2 * hk * dk:].reshape(batch, hv, dv)
        o, st2 = mk.linear_attention_decode(mk.LinearAttentionInputs(q=q, k=k, v=v, state=st2, g=gg, beta=beta,
                                                                     qk_l2norm=True))
        want = mk.gated_rms_norm(o, z, nw)
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"step {step}"
        assert torch.equal(cs, cs2), f"step {step}"
        assert torch.equal(st, st2), f"step {step}"


def test_linear_attention_step_graph_replay():
    """The one-launch step captured in a HIP graph: each replay advances the
    conv and recurrent states in place exactly as an eager step on copies
    does (outputs and both states bit for bit), and eager steps of another
    shape on the capture stream, which share the step's workspace and its
    arrival counts, run between the replays."""
    hk, hv, dk, dv = 16, 32, 128, 128
    x, cs, cw, st, gg, beta, z, nw = _step_case(1, hk, hv, dk, dv, torch.bfloat16, 811)
    ox, ocs, ocw, ost, ogg, obeta, oz, onw = _step_case(2, 2, 4, 64, 32, torch.bfloat16, 812)
    cs_e, st_e = cs.clone(), st.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # warm-up on copies: the captured buffers keep their initial states
        mk.linear_attention_step(x, cs.clone(), cw, st.clone(), gg, beta, z, nw, k_heads=hk)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out_g = mk.linear_attention_step(x, cs, cw, st, gg, beta, z, nw, k_heads=hk)
    ocs_e, ost_e = ocs.clone(), ost.clone()
    for step in range(3):
        graph.replay()
        torch.cuda.synchronize()
        out_e = mk.linear_attention_step(x, cs_e, cw, st_e, gg, beta, z, nw, k_heads=hk)
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {step}"
        assert torch.equal(cs, cs_e) and torch.equal(st, st_e), f"replay {step}"
        with torch.cuda.stream(s):
            other = mk.linear_attention_step(ox, ocs, ocw, ost, ogg, obeta, oz, onw, k_heads=2)
        other_e = mk.linear_attention_step(ox, ocs_e, ocw, ost_e, ogg, obeta, oz, onw, k_heads=2)
        torch.cuda.synchronize()
        assert torch.equal(other, other_e) and torch.equal(ost, ost_e), f"replay {step}"
