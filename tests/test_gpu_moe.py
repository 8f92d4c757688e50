"""GPU parity: persistent MoE decode (one HIP launch) vs the CPU oracle.

Task tolerances: top-k indices bit-exact; bf16 outputs atol 1e-2 / rtol 1e-2
against the oracle run on FP32 upcasts of the inputs; router weights (FP32)
atol 1e-5 / rtol 1e-4.
"""

import dataclasses

import numpy as np
import pytest
import torch

import mega_kernel_qwen36 as mk
import oracle
from tests.inputs import assert_close_out, make_moe, moe_oracle_args, small_moe_reference_shape

pytestmark = pytest.mark.gpu


def _oracle(x, w, k, add_residual=True):
    args, sg = moe_oracle_args(x, w)
    return oracle.moe_decode(*args, top_k=k, add_residual=add_residual, shared_expert_gate=sg)


def _topk_margin(x, w, k):
    """Gap between the k-th and (k+1)-th router logit per row (oracle arithmetic)."""
    args, _ = moe_oracle_args(x, w)
    xn = oracle.rms_norm(args[0], args[1])
    logits = np.sort(xn @ args[2].T, axis=-1)[:, ::-1]
    if logits.shape[1] <= k:
        return np.inf
    return float(np.min(logits[:, k - 1] - logits[:, k]))


def _check(x, w, k, backend="persistent", add_residual=True):
    out, idx, rw = mk.moe_decode(x, w, top_k=k, backend=backend, add_residual=add_residual)
    ref, ref_idx, ref_w = _oracle(x, w, k, add_residual)
    assert out.shape == x.shape and out.dtype == x.dtype
    assert idx.dtype == torch.int64 and rw.dtype == torch.float32
    assert idx.cpu().tolist() == ref_idx.tolist()
    # FP32 softmax over FP32 logits: only the summation order differs.
    torch.testing.assert_close(rw.cpu(), torch.from_numpy(np.asarray(ref_w, dtype=np.float32)), atol=1e-5, rtol=1e-4)
    assert_close_out(out, ref)
    return out, idx, rw


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
@pytest.mark.parametrize("backend", ["auto", "persistent"])
def test_moe_reference_test_shape(batch, backend):
    # test_cuda_ops.py:23-36: _small_moe shape (H 16, E 6, I 12, k 3), row 0 replicated
    x, w, k = small_moe_reference_shape()
    x = x[:1].repeat(batch, 1).contiguous()
    _check(x, w, k, backend)


@pytest.mark.parametrize("batch", [1, 2])
def test_moe_config1_small(batch):
    """Config 1 shape: H 512, E 8, top-2, I 256, shared 256 with a sigmoid gate."""
    x, w, k = make_moe(batch=batch, hidden=512, experts=8, intermediate=256, shared_intermediate=256, top_k=2, seed=1)
    _check(x, w, k)


def test_moe_config1_fp32():
    x, w, k = make_moe(batch=1, hidden=512, experts=8, intermediate=256, shared_intermediate=256, top_k=2, seed=1,
                       dtype=torch.float32)
    _check(x, w, k)


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_moe_config2(batch):
    """Config 2: 35B-A3B MoE layer, independent rows, gated shared expert."""
    x, w, k = make_moe(batch=batch)
    assert _topk_margin(x, w, k) > 1e-4
    _check(x, w, k)


def test_moe_config2_replicated_rows():
    x, w, k = make_moe(batch=4, replicate_rows=True)
    _, idx, _ = _check(x, w, k)
    assert all(row == idx[0].tolist() for row in idx.tolist())


def test_moe_batch_over_eight():
    x, w, k = make_moe(batch=11, hidden=256, experts=32, intermediate=128, shared_intermediate=64, top_k=4, seed=6)
    _check(x, w, k)


@pytest.mark.parametrize("add_residual", [False])
def test_moe_no_residual_ungated(add_residual):
    x, w, k = make_moe(batch=3, hidden=1024, experts=64, intermediate=256, shared_intermediate=384, top_k=6,
                       gated=False, seed=2)
    _check(x, w, k, add_residual=add_residual)


def test_moe_fp16():
    x, w, k = make_moe(batch=2, hidden=1024, experts=32, intermediate=512, shared_intermediate=512, top_k=4, seed=3,
                       dtype=torch.float16)
    _check(x, w, k)


def test_moe_rejects_mixed_weight_dtype():
    # test_cuda_ops.py:52-65
    x, w, k = small_moe_reference_shape()
    mixed = mk.MoeWeights(
        norm_weight=w.norm_weight, router_weight=w.router_weight, expert_gate=w.expert_gate.float(),
        expert_up=w.expert_up, expert_down=w.expert_down, shared_gate=w.shared_gate, shared_up=w.shared_up,
        shared_down=w.shared_down)
    with pytest.raises(RuntimeError, match="expert_gate dtype mismatch"):
        mk.moe_decode(x, mixed, top_k=k, backend="persistent")


def test_moe_deterministic_and_repeated_launches():
    # back-to-back launches exercise the flag generations; results must be bit-identical
    x, w, k = make_moe(batch=2)
    first = mk.moe_decode(x, w, top_k=k)
    for _ in range(20):
        again = mk.moe_decode(x, w, top_k=k)
        assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1]) and torch.equal(first[2], again[2])
    # interleave another shape on the same stream/workspace, then come back
    xs, ws, ks = small_moe_reference_shape()
    _check(xs, ws, ks)
    again = mk.moe_decode(x, w, top_k=k)
    assert torch.equal(first[0], again[0])


def test_moe_grouped_backend_agrees():
    x, w, k = make_moe(batch=2, hidden=512, experts=16, intermediate=256, shared_intermediate=256, top_k=4, seed=4)
    out, idx, rw = mk.moe_decode(x, w, top_k=k)
    g_out, g_idx, g_rw = mk.moe_decode(x, w, top_k=k, backend="grouped")
    assert idx.tolist() == g_idx.tolist()
    torch.testing.assert_close(out.float(), g_out.float(), atol=3e-2, rtol=3e-2)


def test_moe_cuda_graph_replay():
    x, w, k = make_moe(batch=1)
    eager = mk.moe_decode(x, w, top_k=k)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = mk.moe_decode(x, w, top_k=k)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured[0], eager[0]) and torch.equal(captured[1], eager[1])
        again = mk.moe_decode(x, w, top_k=k)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(again[0], eager[0])


@pytest.mark.parametrize("batch", [1, 4])
def test_moe_many_launches_bit_identical(batch):
    """Cross-WG hand-offs (router logits, act) must never read stale data: every
    one of many back-to-back launches returns the same bits, and parity holds."""
    x, w, k = make_moe(batch=batch, seed=40 + batch)
    first = mk.moe_decode(x, w, top_k=k)
    outs = [mk.moe_decode(x, w, top_k=k) for _ in range(300)]
    torch.cuda.synchronize()
    for o in outs:
        assert torch.equal(o[0], first[0]) and torch.equal(o[1], first[1]) and torch.equal(o[2], first[2])
    ref, ref_idx, _ = _oracle(x, w, k)
    assert first[1].cpu().tolist() == ref_idx.tolist()
    assert_close_out(first[0], ref)


# ---------------------------------------------------------------------------
# top-k ties: descending logit, the lower expert index first (the strict `>`
# of the reference kernel's scan, persistent_moe_decode.cu:333; torch.topk
# order, reference.py:44)
# ---------------------------------------------------------------------------

def _exact_logits(x, w):
    """Router logits in float64, one dot per (row, expert), so identical router
    rows give identical values."""
    args, _ = moe_oracle_args(x, w)
    xn = oracle.rms_norm(args[0], args[1]).astype(np.float64)
    r = args[2].astype(np.float64)
    return np.array([[float(np.dot(xn[b], r[e])) for e in range(r.shape[0])] for b in range(xn.shape[0])])


def _with_router(w, router):
    return dataclasses.replace(w, router_weight=router.contiguous())


@pytest.mark.parametrize("shape", ["config1", "config2"])
@pytest.mark.parametrize("batch", [1, 3])
def test_moe_all_router_rows_tied(shape, batch):
    """Identical router rows: every logit ties, so the selection is experts
    0 .. k-1 in that order with equal weights 1/k."""
    if shape == "config1":
        x, w, k = make_moe(batch=batch, hidden=512, experts=8, intermediate=256, shared_intermediate=256, top_k=2,
                           seed=21)
    else:
        x, w, k = make_moe(batch=batch, seed=22)
    w = _with_router(w, w.router_weight[:1].repeat(w.router_weight.shape[0], 1))
    out, idx, rw = mk.moe_decode(x, w, top_k=k)
    assert idx.cpu().tolist() == [list(range(k))] * batch
    torch.testing.assert_close(rw.cpu(), torch.full((batch, k), 1.0 / k), atol=1e-6, rtol=0)
    ref, ref_idx, _ = _oracle(x, w, k)
    assert ref_idx.tolist() == idx.cpu().tolist()
    assert_close_out(out, ref)


def _tied_case(batch, seed):
    """Config 2 with three tie groups planted in row 0's ranking: the top
    expert duplicated at a higher index, the third at a lower index (both
    pairs inside the selection) and the expert that lands on rank k
    duplicated at a lower and a higher index (a tie across the selection
    boundary).  Returns None when the seed's logits have accidental near-ties
    (within 1e-4) among the top k + 4, which FP32 could order differently."""
    x, w, k = make_moe(batch=batch, seed=seed)
    lg = _exact_logits(x, w)
    r = np.argsort(-lg[0], kind="stable")
    far = [int(e) for e in r[k + 4:]]
    e1, e3, eb = int(r[0]), int(r[2]), int(r[k - 3])
    try:
        j_hi = next(e for e in far if e > e1)
        j_lo = next(e for e in far if e < e3 and e != j_hi)
        j_blo = next(e for e in far if e < eb and e not in (j_hi, j_lo))
        j_bhi = next(e for e in far if e > eb and e not in (j_hi, j_lo, j_blo))
    except StopIteration:
        return None
    router = w.router_weight.clone()
    for dst, src in ((j_hi, e1), (j_lo, e3), (j_blo, eb), (j_bhi, eb)):
        router[dst] = router[src]
    w = _with_router(w, router)
    lg = _exact_logits(x, w)
    for b in range(batch):
        top = np.unique(np.sort(lg[b])[::-1][: k + 4])
        if np.min(np.diff(top)) <= 1e-4:
            return None
    expect = np.argsort(-lg, axis=-1, kind="stable")[:, :k]
    row0 = expect[0].tolist()
    # the planted structure is where it was meant to be
    assert row0.index(j_hi) == row0.index(e1) + 1 and row0.index(e3) == row0.index(j_lo) + 1
    assert row0[k - 1] == j_blo and eb not in row0 and j_bhi not in row0
    assert lg[0, eb] == lg[0, j_blo]
    return x, w, k, expect


@pytest.mark.parametrize("batch", [1, 4])
def test_moe_topk_ties_lower_index_first(batch):
    case = None
    for seed in range(500, 540):
        case = _tied_case(batch, seed)
        if case is not None:
            break
    assert case is not None, "no seed without accidental near-ties"
    x, w, k, expect = case
    out, idx, rw = mk.moe_decode(x, w, top_k=k)
    assert idx.cpu().tolist() == expect.tolist()
    rw = rw.cpu()
    row0 = expect[0].tolist()
    lg = _exact_logits(x, w)[0]
    for a, b in zip(row0, row0[1:]):
        if lg[a] == lg[b]:  # tied slots carry bit-identical weights
            assert rw[0, row0.index(a)] == rw[0, row0.index(b)]
    ref, ref_idx, ref_w = _oracle(x, w, k)
    assert ref_idx.tolist() == expect.tolist()
    torch.testing.assert_close(rw, torch.from_numpy(np.asarray(ref_w, np.float32)), atol=1e-5, rtol=1e-4)
    assert_close_out(out, ref)


# ---------------------------------------------------------------------------
# failure reporting: the workspace's error word (a timed-out cross-workgroup
# wait) is reported, makes every later call write NaN instead of reading stale
# words, and a reset restores normal calls.  The error is planted by the host;
# no test makes a wait time out.
# ---------------------------------------------------------------------------

def _moe_capi(lib, x, w, k, out, idx, rw, ws):
    from mega_kernel_qwen36 import _lib as L
    b, h = x.shape
    e, i, _ = w.expert_gate.shape
    return lib.mkq_moe_decode(L.MKQ_DTYPE_BF16, x.data_ptr(), w.norm_weight.data_ptr(), w.router_weight.data_ptr(),
                              w.expert_gate.data_ptr(), w.expert_up.data_ptr(), w.expert_down.data_ptr(),
                              w.shared_gate.data_ptr(), w.shared_up.data_ptr(), w.shared_down.data_ptr(),
                              w.shared_expert_gate.data_ptr(), out.data_ptr(), idx.data_ptr(), rw.data_ptr(), b, h, e,
                              i, w.shared_gate.shape[0], k, 1e-6, 1, ws.data_ptr(), ws.numel(),
                              torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("batch", [1, 3])
def test_moe_error_word_is_sticky_until_reset(batch):
    import ctypes

    from mega_kernel_qwen36 import _lib as L
    lib = L.load_library()
    x, w, k = make_moe(batch=batch, hidden=512, experts=16, intermediate=256, shared_intermediate=256, top_k=4,
                       seed=30 + batch)
    nbytes = lib.mkq_moe_decode_workspace_bytes(batch, 512, 16, 256, 256, k)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    out = torch.empty_like(x)
    idx = torch.empty(batch, k, dtype=torch.int64, device="cuda")
    rw = torch.empty(batch, k, dtype=torch.float32, device="cuda")
    code = ctypes.c_int(-1)
    stream = torch.cuda.current_stream().cuda_stream

    def status(reset):
        assert lib.mkq_moe_decode_status(ws.data_ptr(), ws.numel(), reset, ctypes.byref(code), stream) == L.MKQ_OK
        return code.value

    assert _moe_capi(lib, x, w, k, out, idx, rw, ws) == L.MKQ_OK, lib.mkq_last_error()
    good = (out.clone(), idx.clone(), rw.clone())
    assert status(0) == 0
    ws[256] = 1  # the error word, as a timed-out wait leaves it
    for _ in range(2):
        assert _moe_capi(lib, x, w, k, out, idx, rw, ws) == L.MKQ_OK
        torch.cuda.synchronize()
        assert torch.isnan(out.float()).all() and torch.isnan(rw).all() and (idx == 0).all()
    assert status(0) == 1 and status(1) == 1 and status(0) == 0
    assert int(ws.count_nonzero()) == 0
    assert _moe_capi(lib, x, w, k, out, idx, rw, ws) == L.MKQ_OK
    torch.cuda.synchronize()
    assert torch.equal(out, good[0]) and torch.equal(idx, good[1]) and torch.equal(rw, good[2])


def test_moe_decode_status_through_python(monkeypatch):
    x, w, k = make_moe(batch=1, hidden=512, experts=16, intermediate=256, shared_intermediate=256, top_k=4, seed=35)
    first = mk.moe_decode(x, w, top_k=k)
    assert mk.moe_decode_status() == 0
    monkeypatch.setenv("MKQ_MOE_CHECK", "1")
    again = mk.moe_decode(x, w, top_k=k)
    assert torch.equal(first[0], again[0])
