"""Seeded synthetic inputs for the decode ops, shared by the tests and bench.py.

Values are drawn in FP32 with a CPU ``torch.Generator``, scaled, cast to the
requested dtype and only then moved to the device, so that the CPU oracle can
be run on exact FP32 upcasts of the very values the GPU sees.  Shapes and
distributions follow the task's five configurations:

1. small MoE (H 512, E 8, k 2, I 256, shared 256 + sigmoid gate), FP32
2. 35B-A3B MoE (H 2048, E 256, k 8, I 512, shared 512 + sigmoid gate)
3. 27B dense SwiGLU FFN (5120 -> 17408 -> 5120)
4. GQA attention decode (24 q / 4 kv heads, D 256, T 4K/32K/128K)
5. gated-delta linear attention (16 q/k heads, 32 v heads, D 128)
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from mega_kernel_qwen36 import (
    DenseFfnWeights,
    FullAttentionInputs,
    GatedMoeWeights,
    LinearAttentionInputs,
    MoeWeights,
)

SEED_MOE = 123
SEED_DENSE = 456
SEED_ATTN = 321
SEED_LINEAR = 789


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def _randn(gen, shape, scale=1.0, shift=0.0):
    t = torch.randn(*shape, generator=gen, dtype=torch.float32)
    if scale != 1.0:
        t.mul_(scale)
    if shift != 0.0:
        t.add_(shift)
    return t


def _dev(t: torch.Tensor, device, dtype) -> torch.Tensor:
    return t.to(dtype).to(device)


def np32(t: torch.Tensor) -> np.ndarray:
    """Exact FP32 upcast of a tensor as a numpy array (the oracle's input)."""
    return t.detach().float().cpu().numpy()


# ---------------------------------------------------------------------------
# MoE
# ---------------------------------------------------------------------------

def make_moe(
    *,
    batch=1,
    hidden=2048,
    experts=256,
    intermediate=512,
    shared_intermediate=512,
    top_k=8,
    gated=True,
    seed=SEED_MOE,
    x_scale=1.0,
    w_scale=0.02,
    replicate_rows=False,
    device="cuda",
    dtype=torch.bfloat16,
):
    """Returns (x [B,H], weights, top_k).  Rows are independent unless ``replicate_rows``."""
    g = _gen(seed)
    x = _randn(g, (batch, hidden), x_scale)
    if replicate_rows:
        x = x[:1].repeat(batch, 1)
    fields = dict(
        norm_weight=_randn(g, (hidden,), w_scale, 1.0),
        router_weight=_randn(g, (experts, hidden), w_scale),
        expert_gate=_randn(g, (experts, intermediate, hidden), w_scale),
        expert_up=_randn(g, (experts, intermediate, hidden), w_scale),
        expert_down=_randn(g, (experts, hidden, intermediate), w_scale),
        shared_gate=_randn(g, (shared_intermediate, hidden), w_scale),
        shared_up=_randn(g, (shared_intermediate, hidden), w_scale),
        shared_down=_randn(g, (hidden, shared_intermediate), w_scale),
    )
    if gated:
        fields["shared_expert_gate"] = _randn(g, (hidden,), w_scale)
        w = GatedMoeWeights(**{k: _dev(v, device, dtype) for k, v in fields.items()})
    else:
        w = MoeWeights(**{k: _dev(v, device, dtype) for k, v in fields.items()})
    return _dev(x, device, dtype), w, top_k


def small_moe_reference_shape(device="cuda", dtype=torch.bfloat16, batch=2):
    """The reference test's tiny odd MoE shape (test_reference.py:18-33: H 16, E 6, I 12, k 3, scale 0.08)."""
    return make_moe(batch=batch, hidden=16, experts=6, intermediate=12, shared_intermediate=12, top_k=3,
                    gated=False, seed=7, x_scale=0.08, w_scale=0.08, device=device, dtype=dtype)


def moe_oracle_args(x, w):
    args = [np32(x)] + [np32(getattr(w, f)) for f in (
        "norm_weight", "router_weight", "expert_gate", "expert_up", "expert_down",
        "shared_gate", "shared_up", "shared_down")]
    sg = getattr(w, "shared_expert_gate", None)
    return args, (None if sg is None else np32(sg))


# ---------------------------------------------------------------------------
# dense FFN
# ---------------------------------------------------------------------------

def make_dense(*, batch=1, hidden=5120, intermediate=17408, seed=SEED_DENSE, x_scale=1.0, w_scale=0.02,
               device="cuda", dtype=torch.bfloat16):
    g = _gen(seed)
    x = _randn(g, (batch, hidden), x_scale)
    w = DenseFfnWeights(
        norm_weight=_dev(_randn(g, (hidden,), w_scale, 1.0), device, dtype),
        gate_weight=_dev(_randn(g, (intermediate, hidden), w_scale), device, dtype),
        up_weight=_dev(_randn(g, (intermediate, hidden), w_scale), device, dtype),
        down_weight=_dev(_randn(g, (hidden, intermediate), w_scale), device, dtype),
    )
    return _dev(x, device, dtype), w


def dense_oracle_args(x, w):
    return [np32(x), np32(w.norm_weight), np32(w.gate_weight), np32(w.up_weight), np32(w.down_weight)]


# ---------------------------------------------------------------------------
# GQA attention
# ---------------------------------------------------------------------------

def make_attention(*, batch=1, q_heads=24, kv_heads=4, head_dim=256, seq_len=32768, seed=SEED_ATTN, scale=1.0,
                   device="cuda", dtype=torch.bfloat16):
    g = _gen(seed)
    q = _randn(g, (batch, q_heads, head_dim), scale)
    k = _randn(g, (batch, seq_len, kv_heads, head_dim), scale)
    v = _randn(g, (batch, seq_len, kv_heads, head_dim), scale)
    return FullAttentionInputs(q=_dev(q, device, dtype), k_cache=_dev(k, device, dtype),
                               v_cache=_dev(v, device, dtype), scale=1.0 / math.sqrt(head_dim))


# ---------------------------------------------------------------------------
# linear attention (gated delta rule, config 5)
# ---------------------------------------------------------------------------

def make_gated_delta(*, batch=1, k_heads=16, v_heads=32, key_dim=128, value_dim=128, seed=SEED_LINEAR,
                     device="cuda", dtype=torch.bfloat16):
    g = _gen(seed)
    q = torch.nn.functional.normalize(_randn(g, (batch, k_heads, key_dim)), dim=-1)
    k = torch.nn.functional.normalize(_randn(g, (batch, k_heads, key_dim)), dim=-1)
    v = _randn(g, (batch, v_heads, value_dim))
    gg = -torch.nn.functional.softplus(_randn(g, (batch, v_heads)))
    beta = torch.sigmoid(_randn(g, (batch, v_heads)))
    state = _randn(g, (batch, v_heads, key_dim, value_dim), 0.1)
    return LinearAttentionInputs(q=_dev(q, device, dtype), k=_dev(k, device, dtype), v=_dev(v, device, dtype),
                                 state=state.to(device), g=gg.to(device), beta=beta.to(device))


def make_linear_reference_rule(*, batch=2, heads=3, key_dim=8, value_dim=10, decay=0.92, seed=19, device="cuda",
                               dtype=torch.bfloat16):
    """The reference test's linear-attention shape (test_cuda_ops.py:93-111)."""
    g = _gen(seed)
    q = _randn(g, (batch, heads, key_dim), 0.1)
    k = _randn(g, (batch, heads, key_dim), 0.1)
    v = _randn(g, (batch, heads, value_dim), 0.1)
    state = _randn(g, (batch, heads, key_dim, value_dim), 0.1)
    return LinearAttentionInputs(q=_dev(q, device, dtype), k=_dev(k, device, dtype), v=_dev(v, device, dtype),
                                 state=state.to(device), decay=decay)


@dataclass(frozen=True)
class Tol:
    """Parity tolerances of the task: bf16 outputs 1e-2/1e-2, FP32 state 1e-4."""

    out_atol: float = 1e-2
    out_rtol: float = 1e-2
    state_atol: float = 1e-4
    state_rtol: float = 1e-4


TOL = Tol()


def assert_close_out(actual: torch.Tensor, expected: np.ndarray, atol=TOL.out_atol, rtol=TOL.out_rtol):
    torch.testing.assert_close(actual.detach().float().cpu(), torch.from_numpy(np.asarray(expected, np.float32)),
                               atol=atol, rtol=rtol)


def assert_close_state(actual: torch.Tensor, expected: np.ndarray, atol=TOL.state_atol, rtol=TOL.state_rtol):
    torch.testing.assert_close(actual.detach().float().cpu(), torch.from_numpy(np.asarray(expected, np.float32)),
                               atol=atol, rtol=rtol)
