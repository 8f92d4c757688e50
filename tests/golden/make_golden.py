"""Writes the golden vectors in tests/golden/*.npz.

Inputs are seeded and rounded to bfloat16-representable values (so the same
vectors can be fed to the bf16 GPU kernels exactly); expected outputs come
from a float64 composition of torch library routines (F.rms_norm, F.linear,
F.silu, torch.topk, torch.softmax, F.scaled_dot_product_attention with
enable_gqa, einsum) -- independent of the numpy oracle they check.  Shapes are
the reference test suite's tiny shapes (test_reference.py:18-47,
test_cuda_ops.py:79-111) plus a small gated-delta case.

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import pathlib

import numpy as np
import torch
import torch.nn.functional as F

OUT = pathlib.Path(__file__).resolve().parent


def bf(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.bfloat16).to(torch.float64)


def rnd(g, *shape, scale=1.0, shift=0.0):
    return bf(torch.randn(*shape, generator=g, dtype=torch.float32) * scale + shift)


def save(name, **arrays):
    np.savez(OUT / f"{name}.npz", **{k: np.asarray(v.numpy() if torch.is_tensor(v) else v, dtype=(
        np.int64 if (torch.is_tensor(v) and v.dtype == torch.int64) or isinstance(v, int) else np.float32))
        for k, v in arrays.items()})


def swiglu(xn, g, u, d):
    return F.linear(F.silu(F.linear(xn, g)) * F.linear(xn, u), d)


def moe_small():
    g = torch.Generator().manual_seed(7)
    B, H, E, I, Is, K, s = 2, 16, 6, 12, 12, 3, 0.08
    x = rnd(g, B, H, scale=s)
    nw = rnd(g, H, scale=s, shift=1.0)
    r = rnd(g, E, H, scale=s)
    eg, eu, ed = rnd(g, E, I, H, scale=s), rnd(g, E, I, H, scale=s), rnd(g, E, H, I, scale=s)
    sg, su, sd = rnd(g, Is, H, scale=s), rnd(g, Is, H, scale=s), rnd(g, H, Is, scale=s)
    wsg = rnd(g, H, scale=s)
    xn = F.rms_norm(x, (H,), weight=nw, eps=1e-6)
    tv, ti = torch.topk(F.linear(xn, r), K, dim=-1)
    tw = torch.softmax(tv, -1)
    out = x + torch.sigmoid(xn @ wsg)[:, None] * swiglu(xn, sg, su, sd)
    for b in range(B):
        for k in range(K):
            e = int(ti[b, k])
            out[b] += tw[b, k] * swiglu(xn[b:b + 1], eg[e], eu[e], ed[e])[0]
    save("moe_small", x=x, norm_weight=nw, router_weight=r, expert_gate=eg, expert_up=eu, expert_down=ed,
         shared_gate=sg, shared_up=su, shared_down=sd, shared_expert_gate=wsg, top_k=K, out=out, out_idx=ti,
         out_w=tw)


def dense_small():
    g = torch.Generator().manual_seed(23)
    B, H, I, s = 2, 16, 24, 0.08
    x = rnd(g, B, H, scale=s)
    nw = rnd(g, H, scale=s, shift=1.0)
    wg, wu, wd = rnd(g, I, H, scale=s), rnd(g, I, H, scale=s), rnd(g, H, I, scale=s)
    out = x + swiglu(F.rms_norm(x, (H,), weight=nw, eps=1e-6), wg, wu, wd)
    save("dense_small", x=x, norm_weight=nw, gate_weight=wg, up_weight=wu, down_weight=wd, out=out)


def attention_small():
    g = torch.Generator().manual_seed(11)
    B, Hq, Hkv, D, T = 2, 4, 2, 32, 9
    q, k, v = rnd(g, B, Hq, D), rnd(g, B, T, Hkv, D), rnd(g, B, T, Hkv, D)
    out = F.scaled_dot_product_attention(q[:, :, None], k.transpose(1, 2), v.transpose(1, 2), enable_gqa=True)
    save("attention_small", q=q, k_cache=k, v_cache=v, out=out[:, :, 0])


def linear_small():
    g = torch.Generator().manual_seed(13)
    B, H, Dk, Dv, decay = 2, 3, 8, 10, 0.92
    q, k, v = rnd(g, B, H, Dk, scale=0.1), rnd(g, B, H, Dk, scale=0.1), rnd(g, B, H, Dv, scale=0.1)
    st = torch.randn(B, H, Dk, Dv, generator=g, dtype=torch.float32).to(torch.float64) * 0.1
    st = st.float().double()
    new = decay * st + torch.einsum("bhd,bhv->bhdv", k, v)
    out = torch.einsum("bhd,bhdv->bhv", q, new)
    save("linear_small", q=q, k=k, v=v, state=st, decay=np.float32(decay), out=out, new_state=new)


def gated_delta_small():
    g = torch.Generator().manual_seed(29)
    B, Hk, Hv, Dk, Dv = 2, 2, 4, 16, 12
    q = bf(F.normalize(torch.randn(B, Hk, Dk, generator=g), dim=-1))
    k = bf(F.normalize(torch.randn(B, Hk, Dk, generator=g), dim=-1))
    v = rnd(g, B, Hv, Dv)
    gg = (-F.softplus(torch.randn(B, Hv, generator=g))).float().double()
    beta = torch.sigmoid(torch.randn(B, Hv, generator=g)).float().double()
    st = (torch.randn(B, Hv, Dk, Dv, generator=g) * 0.1).float().double()
    rep = Hv // Hk
    kk, qq = k.repeat_interleave(rep, 1), q.repeat_interleave(rep, 1)
    s = st * torch.exp(gg)[..., None, None]
    u = v - torch.einsum("bhd,bhdv->bhv", kk, s)
    s = s + beta[..., None, None] * torch.einsum("bhd,bhv->bhdv", kk, u)
    out = torch.einsum("bhd,bhdv->bhv", qq, s)
    save("gated_delta_small", q=q, k=k, v=v, state=st, g=gg, beta=beta, out=out, new_state=s)


if __name__ == "__main__":
    moe_small()
    dense_small()
    attention_small()
    linear_small()
    gated_delta_small()
    print("wrote", sorted(p.name for p in OUT.glob("*.npz")))
