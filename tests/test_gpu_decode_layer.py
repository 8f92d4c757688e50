"""GPU parity: decode_layer (reference ops.py:701-748) composed from the HIP ops,
against the oracle's restatement of the same composition.

Config 5 (gated delta rule: 16 q/k heads, 32 v heads of dim 128) and the GQA
attention of config 4 feed the config-2 MoE (35B-A3B shape) or a dense FFN,
with an ``out_proj`` onto the hidden size.  The oracle rounds each op's output
to bfloat16 before the next op, as the device path does.

Tolerances (task): bf16 outputs atol/rtol 1e-2, FP32 recurrent state 1e-4,
top-k indices bit-exact.
"""

import dataclasses

import numpy as np
import pytest
import torch

import mega_kernel_qwen36 as mk
import oracle
from mega_kernel_qwen36 import _lib
from tests.inputs import (assert_close_out, assert_close_state, make_attention, make_dense, make_gated_delta,
                          make_moe, np32)

pytestmark = pytest.mark.gpu

MOE_FIELDS = ("norm_weight", "router_weight", "expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up",
              "shared_down", "shared_expert_gate")
DENSE_FIELDS = ("norm_weight", "gate_weight", "up_weight", "down_weight")


def _proj(out_features, in_features, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(out_features, in_features, generator=g) * 0.02).to("cuda", torch.bfloat16)


def _np_fields(obj, names):
    return {n: np32(getattr(obj, n)) for n in names if getattr(obj, n, None) is not None}


def _router_gap(ref, moe_np, k):
    """Smallest gap between consecutive logits among the top k + 1 of every
    row, for the oracle's MoE input.  The device's MoE input differs from it
    by the bf16 roundings upstream (one ulp of the residual sum flips here and
    there, ~1e-3 on a logit), so a composed layer pins the exact top-k order
    only where the gaps are wider than that."""
    xn = oracle.rms_norm(ref["residual"], moe_np["norm_weight"])
    lg = np.sort(xn @ moe_np["router_weight"].T, axis=-1)[:, ::-1][:, : k + 1]
    return float(np.min(lg[:, :-1] - lg[:, 1:]))


@pytest.mark.parametrize("batch", [1, 8])
def test_decode_layer_gated_delta_with_moe(batch):
    """Config 5 composed with the config-2 MoE (layer 0 is a linear-attention layer)."""
    x, w, k = make_moe(batch=batch, seed=60 + batch)
    lin = make_gated_delta(batch=batch, seed=70 + batch)
    lin = dataclasses.replace(lin, out_proj=_proj(x.shape[1], 32 * 128, 80 + batch))
    state_before = lin.state.clone()
    res = mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)
    ref = oracle.decode_layer(
        np32(x), kind="linear_attention", moe=_np_fields(w, MOE_FIELDS), top_k=k,
        linear_attention=dict(q=np32(lin.q), k=np32(lin.k), v=np32(lin.v), state=np32(lin.state), g=np32(lin.g),
                              beta=np32(lin.beta), out_proj=np32(lin.out_proj)))
    assert _router_gap(ref, _np_fields(w, MOE_FIELDS), k) > 1e-3
    assert res.router_indices.cpu().tolist() == ref["router_indices"].tolist()
    assert_close_out(res.linear_output, ref["linear_output"])
    assert_close_state(res.linear_state, ref["linear_state"])
    assert_close_out(res.hidden, ref["hidden"])
    assert torch.equal(lin.state, state_before)  # the layer returns a new state


@pytest.mark.parametrize("batch", [1, 8])
def test_decode_layer_gated_delta_qk_l2norm_with_moe(batch):
    """Config 5 with the model's in-kernel q/k L2 norm (unnormalised q and k,
    q scaled by 1/sqrt(Dk)) composed with the config-2 MoE."""
    x, w, k = make_moe(batch=batch, seed=160 + batch)
    lin = make_gated_delta(batch=batch, seed=170 + batch)
    g = torch.Generator().manual_seed(180 + batch)
    q = (torch.randn(batch, 16, 128, generator=g) * 2.0).to("cuda", torch.bfloat16)
    kk = (torch.randn(batch, 16, 128, generator=g) * 0.5).to("cuda", torch.bfloat16)
    lin = dataclasses.replace(lin, q=q, k=kk, qk_l2norm=True, out_proj=_proj(x.shape[1], 32 * 128, 190 + batch))
    res = mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)
    ref = oracle.decode_layer(
        np32(x), kind="linear_attention", moe=_np_fields(w, MOE_FIELDS), top_k=k,
        linear_attention=dict(q=np32(q), k=np32(kk), v=np32(lin.v), state=np32(lin.state), g=np32(lin.g),
                              beta=np32(lin.beta), out_proj=np32(lin.out_proj), qk_l2norm=True))
    assert res.router_indices.cpu().tolist() == ref["router_indices"].tolist()
    assert_close_state(res.linear_state, ref["linear_state"])
    assert_close_out(res.linear_output, ref["linear_output"])
    assert_close_out(res.hidden, ref["hidden"])


@pytest.mark.parametrize("layout", ["append", "paged_append"])
def test_decode_layer_attention_append_with_moe(layout):
    """A full-attention layer whose new token is appended inside the attention
    kernel, contiguous or paged (16-token blocks in a shuffled pool), against
    the oracle's decode_layer over the same cache layout."""
    _, w, k = make_moe(batch=2, seed=200)
    att = make_attention(batch=2, seq_len=1000, seed=201)
    g = torch.Generator().manual_seed(202)
    k_new = torch.randn(2, 4, 256, generator=g).to("cuda", torch.bfloat16)
    v_new = torch.randn(2, 4, 256, generator=g).to("cuda", torch.bfloat16)
    proj = _proj(w.norm_weight.shape[0], 24 * 256, 203)
    if layout == "append":
        kc, vc = att.k_cache.clone(), att.v_cache.clone()
        fields = dict(k_cache=kc, v_cache=vc, k_new=k_new, v_new=v_new, cache_seqlen=700)
    else:
        bs, nb = 16, (1000 + 15) // 16
        perm = torch.randperm(4 * nb, generator=g)[: 2 * nb].reshape(2, nb).to(torch.int32)
        kp = torch.randn(4 * nb, bs, 4, 256, generator=g).to("cuda", torch.bfloat16)
        vp = torch.randn(4 * nb, bs, 4, 256, generator=g).to("cuda", torch.bfloat16)
        fields = dict(k_cache=kp, v_cache=vp, k_new=k_new, v_new=v_new, block_table=perm.to("cuda"), seq_len=977)
    ref_fields = {n: (np32(t) if isinstance(t, torch.Tensor) else t) for n, t in fields.items()}
    att = dataclasses.replace(att, out_proj=proj, **fields)
    moe_np = _np_fields(w, MOE_FIELDS)
    for seed in range(210, 230):  # hidden states whose routing has no near-tie (see _router_gap)
        x = torch.randn(2, 2048, generator=torch.Generator().manual_seed(seed)).to("cuda", torch.bfloat16)
        ref = oracle.decode_layer(
            np32(x), kind="full_attention", moe=moe_np, top_k=k,
            full_attention=dict(q=np32(att.q), scale=att.scale, out_proj=np32(proj), **ref_fields))
        if _router_gap(ref, moe_np, k) > 3e-3:
            break
    assert _router_gap(ref, moe_np, k) > 3e-3
    res = mk.decode_layer(3, x, w, full_attention=att, top_k=k)
    assert res.router_indices.cpu().tolist() == ref["router_indices"].tolist()
    assert_close_out(res.attention_output, ref["attention_output"])
    assert_close_out(res.hidden, ref["hidden"])


def test_decode_layer_full_attention_with_moe():
    """Layer 3 is a full-attention layer: config-4 GQA (T = 4096) then the MoE."""
    x, w, k = make_moe(batch=1, seed=91)
    att = make_attention(batch=1, seq_len=4096, seed=92)
    att = dataclasses.replace(att, out_proj=_proj(x.shape[1], 24 * 256, 93))
    res = mk.decode_layer(3, x, w, full_attention=att, top_k=k)
    ref = oracle.decode_layer(
        np32(x), kind="full_attention", moe=_np_fields(w, MOE_FIELDS), top_k=k,
        full_attention=dict(q=np32(att.q), k_cache=np32(att.k_cache), v_cache=np32(att.v_cache), scale=att.scale,
                            out_proj=np32(att.out_proj)))
    assert res.router_indices.cpu().tolist() == ref["router_indices"].tolist()
    assert_close_out(res.attention_output, ref["attention_output"])
    assert_close_out(res.hidden, ref["hidden"])


@pytest.mark.parametrize("batch", [1, 4])
def test_decode_layer_gated_delta_with_dense_ffn(batch):
    x, d = make_dense(batch=batch, hidden=2048, intermediate=6144, seed=100 + batch)
    lin = make_gated_delta(batch=batch, seed=110 + batch)
    lin = dataclasses.replace(lin, out_proj=_proj(2048, 32 * 128, 120 + batch))
    res = mk.decode_layer(0, x, dense_ffn=d, linear_attention=lin)
    ref = oracle.decode_layer(
        np32(x), kind="linear_attention", dense_ffn=_np_fields(d, DENSE_FIELDS),
        linear_attention=dict(q=np32(lin.q), k=np32(lin.k), v=np32(lin.v), state=np32(lin.state), g=np32(lin.g),
                              beta=np32(lin.beta), out_proj=np32(lin.out_proj)))
    assert res.router_indices is None
    assert_close_state(res.linear_state, ref["linear_state"])
    assert_close_out(res.hidden, ref["hidden"])


def test_decode_layer_without_out_proj_reshapes():
    """Without out_proj the attention output is reshaped onto the hidden size,
    as in the reference (ops.py:722,728): 8 q heads x 256 = 2048 = hidden."""
    x, w, k = make_moe(batch=1, seed=131)
    att = make_attention(batch=1, q_heads=8, kv_heads=2, seq_len=300, seed=132)
    res = mk.decode_layer(3, x, w, full_attention=att, top_k=k)
    ref = oracle.decode_layer(
        np32(x), kind="full_attention", moe=_np_fields(w, MOE_FIELDS), top_k=k,
        full_attention=dict(q=np32(att.q), k_cache=np32(att.k_cache), v_cache=np32(att.v_cache), scale=att.scale))
    assert res.router_indices.cpu().tolist() == ref["router_indices"].tolist()
    np.testing.assert_array_equal(res.attention_output.shape, x.shape)
    assert_close_out(res.hidden, ref["hidden"])


def test_decode_layer_graph_replay():
    """A captured decode_layer (gated delta + out_proj + MoE) replays bit-identically
    to eager calls.  The capture stream's workspaces exist before capture, so the
    graph holds no workspace fill: every replay relies on the MoE generation word
    and the arrival counters left by the previous call."""
    x, w, k = make_moe(batch=1, seed=141)
    lin = make_gated_delta(batch=1, seed=142)
    lin = dataclasses.replace(lin, out_proj=_proj(x.shape[1], 32 * 128, 143))
    eager = mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        res = mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(res.hidden, eager.hidden)
        assert torch.equal(res.router_indices, eager.router_indices)
        assert torch.equal(res.linear_state, eager.linear_state)
        mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("batch,dtype", [(1, torch.bfloat16), (5, torch.bfloat16), (3, torch.float16),
                                         (2, torch.float32)])
def test_gemv_add_matches_separate_add(batch, dtype):
    """mkq_gemv_add through the C ABI, the fused residual add of decode_layer:
    y is bit-identical to mkq_gemv without a residual, sum is bit-identical to
    the reference's separate add (torch's `residual + y`), and y agrees with an
    FP64 product within the output tolerance.  Batch 5 takes two launches
    (4 rows, then 1)."""
    lib = _lib.load_library()
    g = torch.Generator().manual_seed(300 + batch)
    kdim, n = 4096, 2048
    x = torch.randn(batch, kdim, generator=g).to("cuda", dtype)
    w = (torch.randn(n, kdim, generator=g) * 0.02).to("cuda", dtype)
    r = torch.randn(batch, n, generator=g).to("cuda", dtype)
    y, summed, y0 = (torch.empty(batch, n, dtype=dtype, device="cuda") for _ in range(3))
    code = {torch.bfloat16: _lib.MKQ_DTYPE_BF16, torch.float16: _lib.MKQ_DTYPE_F16,
            torch.float32: _lib.MKQ_DTYPE_F32}[dtype]
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.mkq_gemv_add(code, x.data_ptr(), w.data_ptr(), r.data_ptr(), y.data_ptr(), summed.data_ptr(), batch,
                          kdim, n, stream)
    assert rc == _lib.MKQ_OK, lib.mkq_last_error()
    rc = lib.mkq_gemv(code, x.data_ptr(), w.data_ptr(), None, y0.data_ptr(), batch, kdim, n, stream)
    assert rc == _lib.MKQ_OK, lib.mkq_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y, y0)
    assert torch.equal(summed, r + y)
    ref = x.cpu().double() @ w.cpu().double().T
    torch.testing.assert_close(y.cpu().double(), ref, atol=1e-2, rtol=1e-2)


def test_decode_layer_projected_residual_equals_separate_add():
    """decode_layer with an out_proj fuses the residual add into the
    projection; its hidden output equals the unfused composition (projection,
    torch add, MoE) bit for bit."""
    x, w, k = make_moe(batch=2, seed=151)
    lin = make_gated_delta(batch=2, seed=152)
    lin = dataclasses.replace(lin, out_proj=_proj(x.shape[1], 32 * 128, 153))
    res = mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)
    out, _ = mk.linear_attention_decode(lin)
    y = mk.ops._C.gemv(out.reshape(2, -1).contiguous(), lin.out_proj, None)
    hidden, idx, _ = mk.moe_decode(x + y, w, top_k=k, add_residual=True)
    torch.cuda.synchronize()
    assert torch.equal(res.linear_output, y)
    assert torch.equal(res.router_indices, idx)
    assert torch.equal(res.hidden, hidden)


@pytest.mark.gpu
@pytest.mark.parametrize("batch,dtype,kdim,n", [(1, torch.bfloat16, 2048, 8192), (3, torch.bfloat16, 5120, 512),
                                                (5, torch.float16, 1000, 300), (2, torch.float32, 777, 65)])
def test_rms_norm_gemv_matches_oracle(batch, dtype, kdim, n):
    """mkq_rms_norm_gemv (input RMSNorm and projection in one launch) against
    the oracle's rms_norm_linear: bf16/f16 round the norm and the product to
    the dtype as the reference's rms_norm does; f32 keeps both.  Batch 5 takes
    two launches; in_features 1000 / 777 take the element-wise path."""
    g = torch.Generator().manual_seed(500 + batch)
    x = torch.randn(batch, kdim, generator=g).to("cuda", dtype)
    nw = (1 + 0.02 * torch.randn(kdim, generator=g)).to("cuda", dtype)
    w = (torch.randn(n, kdim, generator=g) * 0.02).to("cuda", dtype)
    print(f"rms_norm_gemv: batch {batch}, {dtype}, {kdim} -> {n}", flush=True)
    y = mk.ops._C.rms_norm_gemv(x, nw, w, 1e-6)
    torch.cuda.synchronize()
    ref = oracle.rms_norm_linear(np32(x), np32(nw), np32(w), 1e-6, round_to_bf16=dtype == torch.bfloat16)
    if dtype == torch.float16:
        ref = (torch.from_numpy(oracle.rms_norm(np32(x), np32(nw))).half().float().numpy() @ np32(w).T)
    assert_close_out(y, ref)
    # through the C ABI, same result bit for bit
    lib = _lib.load_library()
    y2 = torch.empty_like(y)
    code = {torch.bfloat16: _lib.MKQ_DTYPE_BF16, torch.float16: _lib.MKQ_DTYPE_F16,
            torch.float32: _lib.MKQ_DTYPE_F32}[dtype]
    rc = lib.mkq_rms_norm_gemv(code, x.data_ptr(), nw.data_ptr(), 1e-6, w.data_ptr(), y2.data_ptr(), batch, kdim, n,
                               torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.MKQ_OK, lib.mkq_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y, y2)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["append", "paged_append"])
def test_decode_layer_projects_qkv_with_moe(layout):
    """A full-attention layer from its pre-norm input: q, k_new and v_new come
    from rms_norm(hidden) @ qkv_proj^T (config-4 heads, hidden 2048), the new
    token is appended into the cache inside the attention kernel, then out_proj,
    the residual and the config-2 MoE; against the oracle's decode_layer with
    the same projection."""
    _, w, k = make_moe(batch=2, seed=600)
    att = make_attention(batch=2, seq_len=1000, seed=601)
    g = torch.Generator().manual_seed(602)
    H = w.norm_weight.shape[0]
    qkv_proj = (torch.randn((24 + 8) * 256, H, generator=g) * 0.02).to("cuda", torch.bfloat16)
    in_norm = (1 + 0.02 * torch.randn(H, generator=g)).to("cuda", torch.bfloat16)
    proj = _proj(H, 24 * 256, 603)
    if layout == "append":
        fields = dict(k_cache=att.k_cache.clone(), v_cache=att.v_cache.clone(), cache_seqlen=700)
    else:
        bs, nb = 16, (1000 + 15) // 16
        perm = torch.randperm(4 * nb, generator=g)[: 2 * nb].reshape(2, nb).to(torch.int32)
        kp = torch.randn(4 * nb, bs, 4, 256, generator=g).to("cuda", torch.bfloat16)
        vp = torch.randn(4 * nb, bs, 4, 256, generator=g).to("cuda", torch.bfloat16)
        fields = dict(k_cache=kp, v_cache=vp, block_table=perm.to("cuda"), seq_len=977)
    ref_fields = {n: (np32(t) if isinstance(t, torch.Tensor) else t) for n, t in fields.items()}
    att = dataclasses.replace(att, q=None, out_proj=proj, qkv_proj=qkv_proj, input_norm=in_norm, **fields)
    moe_np = _np_fields(w, MOE_FIELDS)
    for seed in range(610, 640):  # hidden states whose routing has no near-tie (see _router_gap)
        x = torch.randn(2, H, generator=torch.Generator().manual_seed(seed)).to("cuda", torch.bfloat16)
        ref = oracle.decode_layer(
            np32(x), kind="full_attention", moe=moe_np, top_k=k,
            full_attention=dict(scale=att.scale, out_proj=np32(proj), qkv_proj=np32(qkv_proj),
                                input_norm=np32(in_norm), **ref_fields))
        if _router_gap(ref, moe_np, k) > 3e-3:
            break
    assert _router_gap(ref, moe_np, k) > 3e-3
    print(f"decode_layer qkv projection: {layout}, seed {seed}", flush=True)
    res = mk.decode_layer(3, x, w, full_attention=att, top_k=k)
    assert res.router_indices.cpu().tolist() == ref["router_indices"].tolist()
    assert_close_out(res.attention_output, ref["attention_output"])
    assert_close_out(res.hidden, ref["hidden"])


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 8])
def test_decode_layer_projects_linear_inputs_with_moe(batch):
    """A linear-attention layer from its pre-norm input: q, k and v (config 5:
    16 q/k heads and 32 v heads of 128) come from rms_norm(hidden) @ in_proj^T,
    then the gated delta rule with the in-kernel q/k L2 norm, out_proj, the
    residual and the config-2 MoE; against the oracle's decode_layer."""
    _, w, k = make_moe(batch=batch, seed=650 + batch)
    lin = make_gated_delta(batch=batch, seed=660 + batch)
    g = torch.Generator().manual_seed(670 + batch)
    H = w.norm_weight.shape[0]
    in_proj = (torch.randn(2 * 16 * 128 + 32 * 128, H, generator=g) * 0.02).to("cuda", torch.bfloat16)
    in_norm = (1 + 0.02 * torch.randn(H, generator=g)).to("cuda", torch.bfloat16)
    lin = dataclasses.replace(lin, q=None, k=None, v=None, in_proj=in_proj, input_norm=in_norm, qk_l2norm=True,
                              out_proj=_proj(H, 32 * 128, 680 + batch))
    moe_np = _np_fields(w, MOE_FIELDS)
    for seed in range(690, 720):
        x = torch.randn(batch, H, generator=torch.Generator().manual_seed(seed)).to("cuda", torch.bfloat16)
        # The projection is checked against the oracle's at the bf16 tolerance;
        # the recurrence then runs in the oracle on the device's projected q/k/v,
        # since one bf16 ulp of k moves the FP32 state by more than 1e-4.
        qkv = mk.ops._C.rms_norm_gemv(x, in_norm, in_proj, 1e-6)
        assert_close_out(qkv, oracle.rms_norm_linear(np32(x), np32(in_norm), np32(in_proj)))
        q_np = np32(qkv)
        ref = oracle.decode_layer(
            np32(x), kind="linear_attention", moe=moe_np, top_k=k,
            linear_attention=dict(q=q_np[:, :2048].reshape(batch, 16, 128),
                                  k=q_np[:, 2048:4096].reshape(batch, 16, 128),
                                  v=q_np[:, 4096:].reshape(batch, 32, 128), state=np32(lin.state), g=np32(lin.g),
                                  beta=np32(lin.beta), out_proj=np32(lin.out_proj), qk_l2norm=True))
        if _router_gap(ref, moe_np, k) > 3e-3:
            break
    assert _router_gap(ref, moe_np, k) > 3e-3
    print(f"decode_layer linear in_proj: batch {batch}, seed {seed}", flush=True)
    res = mk.decode_layer(0, x, w, linear_attention=lin, top_k=k)
    assert res.router_indices.cpu().tolist() == ref["router_indices"].tolist()
    assert_close_state(res.linear_state, ref["linear_state"])
    assert_close_out(res.linear_output, ref["linear_output"])
    assert_close_out(res.hidden, ref["hidden"])
