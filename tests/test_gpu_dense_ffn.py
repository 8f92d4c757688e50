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
