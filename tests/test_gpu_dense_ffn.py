"""GPU parity: dense SwiGLU FFN decode (HIP) vs the CPU oracle.

Tolerance (task): bf16 outputs atol 1e-2, rtol 1e-2 against the oracle run on
FP32 upcasts of the same bf16 inputs.
"""

import pytest
import torch

import mega_kernel_qwen36 as mk
import oracle
from tests.inputs import assert_close_out, dense_oracle_args, make_dense

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_dense_ffn_reference_shape(batch):
    # the reference test's tiny shape (test_reference.py:36-47): H 16, I 24, scale 0.08,
    # rows replicated as in test_cuda_ops.py:43
    x, w = make_dense(batch=1, hidden=16, intermediate=24, seed=23, x_scale=0.08, w_scale=0.08)
    x = x[:1].repeat(batch, 1).contiguous()
    out = mk.dense_ffn_decode(x, w)
    ref = oracle.dense_ffn_decode(*dense_oracle_args(x, w))
    assert out.dtype == x.dtype and out.shape == x.shape
    assert_close_out(out, ref)


@pytest.mark.parametrize("hidden,intermediate", [(64, 96), (520, 1000), (1000, 264)])
def test_dense_ffn_odd_shapes(hidden, intermediate):
    x, w = make_dense(batch=3, hidden=hidden, intermediate=intermediate, seed=5)
    out = mk.dense_ffn_decode(x, w)
    assert_close_out(out, oracle.dense_ffn_decode(*dense_oracle_args(x, w)))


@pytest.mark.parametrize("add_residual", [True, False])
def test_dense_ffn_no_residual(add_residual):
    x, w = make_dense(batch=2, hidden=256, intermediate=512, seed=9)
    out = mk.dense_ffn_decode(x, w, add_residual=add_residual)
    ref = oracle.dense_ffn_decode(*dense_oracle_args(x, w), add_residual=add_residual)
    assert_close_out(out, ref)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_dense_ffn_other_dtypes(dtype):
    x, w = make_dense(batch=2, hidden=512, intermediate=768, seed=3, dtype=dtype)
    out = mk.dense_ffn_decode(x, w)
    assert out.dtype == dtype
    assert_close_out(out, oracle.dense_ffn_decode(*dense_oracle_args(x, w)))


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_dense_ffn_27b_shape(batch):
    """Config 3: 27B dense FFN, 5120 -> 17408 -> 5120, bf16."""
    x, w = make_dense(batch=batch)
    out = mk.dense_ffn_decode(x, w)
    ref = oracle.dense_ffn_decode(*dense_oracle_args(x, w))
    assert_close_out(out, ref)


def test_dense_ffn_deterministic():
    x, w = make_dense(batch=2, hidden=1024, intermediate=2048, seed=11)
    a = mk.dense_ffn_decode(x, w)
    b = mk.dense_ffn_decode(x, w)
    assert torch.equal(a, b)


def test_dense_ffn_torch_backend_agrees():
    x, w = make_dense(batch=2, hidden=512, intermediate=1024, seed=13)
    out = mk.dense_ffn_decode(x, w)
    ref = mk.dense_ffn_decode(x, w, backend="torch")
    torch.testing.assert_close(out.float(), ref.float(), atol=3e-2, rtol=3e-2)


# Batches of 3 and more take the MFMA path (16-row weight tiles, x_norm and act
# as 16-bit high part + remainder); 9 and 16 run it in passes of 8 rows.
@pytest.mark.parametrize("batch", [3, 5, 7, 9, 16])
def test_dense_ffn_batched_path(batch):
    x, w = make_dense(batch=batch, hidden=1536, intermediate=4104, seed=31)
    out = mk.dense_ffn_decode(x, w)
    assert_close_out(out, oracle.dense_ffn_decode(*dense_oracle_args(x, w)))


def test_dense_ffn_batched_path_fp16():
    x, w = make_dense(batch=4, hidden=512, intermediate=1032, seed=37, dtype=torch.float16)
    out = mk.dense_ffn_decode(x, w)
    assert out.dtype == torch.float16
    assert_close_out(out, oracle.dense_ffn_decode(*dense_oracle_args(x, w)))


def test_dense_ffn_batched_path_matches_rows():
    """The batched path keeps about 16 mantissa bits of x_norm and act: its rows
    agree with the one-row kernels (FP32 x_norm and act) to bf16 rounding."""
    x, w = make_dense(batch=6, hidden=1024, intermediate=2816, seed=41)
    out = mk.dense_ffn_decode(x, w).float()
    rows = torch.cat([mk.dense_ffn_decode(x[i:i + 1].contiguous(), w).float() for i in range(x.shape[0])])
    torch.testing.assert_close(out, rows, atol=1.6e-2, rtol=8e-3)


def test_dense_ffn_batched_state_across_shapes():
    """Arrival counters return to zero: repeated calls, interleaved with other
    shapes on the same workspace, give bit-identical results."""
    x, w = make_dense(batch=4, hidden=512, intermediate=1000, seed=43)
    x2, w2 = make_dense(batch=8, hidden=1024, intermediate=3000, seed=44)
    first = mk.dense_ffn_decode(x, w)
    for _ in range(3):
        other = mk.dense_ffn_decode(x2, w2)
        assert torch.equal(mk.dense_ffn_decode(x, w), first)
    assert_close_out(other, oracle.dense_ffn_decode(*dense_oracle_args(x2, w2)))
    assert_close_out(first, oracle.dense_ffn_decode(*dense_oracle_args(x, w)))


def test_dense_ffn_batched_graph_replay():
    x, w = make_dense(batch=4, hidden=1024, intermediate=2048, seed=47)
    eager = mk.dense_ffn_decode(x, w)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mk.dense_ffn_decode(x, w)  # warm the workspace on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    # Captured on the stream whose workspace already exists, so the graph holds
    # no workspace fill and each replay relies on the counters returning to zero.
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = mk.dense_ffn_decode(x, w)
    for _ in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        mk.dense_ffn_decode(x, w)  # eager work between replays
        torch.cuda.synchronize()
