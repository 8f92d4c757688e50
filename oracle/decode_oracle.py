"""CPU oracle for the single-token decode hot path (numpy, FP32).

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
module: only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use it, and only as the checker (or, for the CPU
baseline, as the thing timed on the host cores).  The HIP path never routes
through it.

Each function restates one function of the reference's
``mega_kernel_qwen36/reference.py`` from its text, keeping its op structure
(FP32 upcast of every weight on every call, the Python loop over
batch x top-k in MoE, the per-query-head loop in attention) so that timing it
is a fair "reference CPU path" figure.  Inputs are numpy arrays:

* ``float32`` arrays are used as is;
* ``uint16`` arrays are bfloat16 bit patterns and are upcast on every call,
  as ``tensor.float()`` does in the reference.

Two behaviours are added where the task's shapes need them and the reference
has no code for them; both are documented at their functions:

* the sigmoid-gated shared expert (``shared_expert_gate``), applied to the
  post-RMSNorm activation, as the HF ``Qwen3NextSparseMoeBlock`` does;
* the gated delta rule for linear attention (``gated_delta_decode``), with
  v-head ``j`` reading q/k head ``j // (Hv // Hk)``.

Pinning (what checks each function independently of its own text) is listed
in ``PINNING`` at the bottom of this file and exercised by
``tests/test_oracle.py``: closed forms, invariants, torch library routines
(``torch.topk``, ``F.scaled_dot_product_attention(enable_gqa=True)``,
``F.rms_norm``) and committed golden vectors written by an independent
float64 torch composition (``tests/golden/make_golden.py``).
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np

__all__ = [
    "as_f32",
    "bf16_bits",
    "bf16_round",
    "rms_norm",
    "silu",
    "topk_desc",
    "softmax",
    "moe_decode",
    "dense_ffn_decode",
    "apply_partial_rope",
    "full_attention_decode",
    "linear_attention_decode",
    "gated_delta_decode",
    "causal_conv1d_update",
    "gated_rms_norm",
    "rms_norm_linear",
    "attention_cache_view",
    "decode_layer",
    "PINNING",
]


# ---------------------------------------------------------------------------
# dtype helpers
# ---------------------------------------------------------------------------

def as_f32(a) -> np.ndarray:
    """Upcast to float32.  ``uint16`` input is taken as bfloat16 bits."""
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return (a.astype(np.uint32) << np.uint32(16)).view(np.float32)
    return a.astype(np.float32, copy=False)


def bf16_bits(a) -> np.ndarray:
    """Round float32 to bfloat16 (nearest-even) and return the bit patterns."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    rounding = np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    out = ((u + rounding) >> np.uint64(16)).astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.uint16(0x7FC0)
    return out


def bf16_round(a) -> np.ndarray:
    """float32 -> bfloat16 -> float32 (what ``.to(torch.bfloat16).float()`` does)."""
    return as_f32(bf16_bits(a))


# ---------------------------------------------------------------------------
# elementwise / small pieces
# ---------------------------------------------------------------------------

def rms_norm(x, weight, eps: float = 1e-6) -> np.ndarray:
    """``(x * rsqrt(mean(x^2) + eps)) * weight`` in FP32 (reference.py:10-13).

    reference.py ends with ``.to(x.dtype)``, which rounds x_norm to bf16 for
    bf16 inputs.  The CUDA kernels this path replaces keep x_norm in FP32
    (persistent_moe_decode.cu:28-30, 280), and so do the HIP kernels, so the
    oracle keeps it in FP32 too.  The difference is below the bf16 output
    tolerance; the reference's own GPU tests compare its FP32-x_norm kernel with
    reference.py the same way (tests/test_cuda_ops.py:25-36).
    """
    xf = as_f32(x)
    var = np.mean(xf * xf, axis=-1, keepdims=True, dtype=np.float32)
    inv = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return (xf * inv * as_f32(weight)).astype(np.float32)


def rms_norm_linear(x, norm_weight, w, eps: float = 1e-6, *, round_to_bf16: bool = True) -> np.ndarray:
    """An input RMSNorm then a projection: ``rms_norm(x).to(dtype) @ w^T``.

    This is the reference planner's ``rmsnorm`` -> ``linear`` task pair in
    front of a layer's mixer (mega_kernel_qwen36/mpk_graph.py:349-373), with
    the norm of reference.py:10-13, whose ``.to(x.dtype)`` rounds x_norm to
    bf16 before the matmul.  With ``round_to_bf16`` x_norm and the product are
    rounded to bfloat16, as on the bf16 device path; x [B, K], w [N, K].
    """
    rnd = bf16_round if round_to_bf16 else (lambda a: as_f32(a))
    xn = rnd(rms_norm(x, norm_weight, eps))
    return rnd(xn @ as_f32(w).T)


def silu(a: np.ndarray) -> np.ndarray:
    a = a.astype(np.float32, copy=False)
    return (a / (np.float32(1.0) + np.exp(-a))).astype(np.float32)


def sigmoid(a):
    a = np.asarray(a, dtype=np.float32)
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-a))).astype(np.float32)


def topk_desc(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Top-k along the last axis, descending, ties to the lower index.

    ``torch.topk(..., sorted=True)`` order (reference.py:44).  The tie rule is
    the one the reference CUDA kernel implements with a strict ``>`` while
    scanning indices upward (persistent_moe_decode.cu:333).
    """
    order = np.argsort(-logits, axis=-1, kind="stable")[..., :k]
    vals = np.take_along_axis(logits, order, axis=-1)
    return vals.astype(np.float32), order.astype(np.int64)


def softmax(a: np.ndarray, axis: int = -1) -> np.ndarray:
    a = a.astype(np.float32, copy=False)
    m = np.max(a, axis=axis, keepdims=True)
    e = np.exp(a - m)
    return (e / np.sum(e, axis=axis, keepdims=True)).astype(np.float32)


# ---------------------------------------------------------------------------
# MoE  (reference.py:16-62)
# ---------------------------------------------------------------------------

def moe_decode(
    x,
    norm_weight,
    router_weight,
    expert_gate,
    expert_up,
    expert_down,
    shared_gate,
    shared_up,
    shared_down,
    *,
    eps: float = 1e-6,
    top_k: int = 8,
    add_residual: bool = True,
    shared_expert_gate=None,
) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Restates ``moe_decode_reference`` (reference.py:16-62).

    x [B,H]; router [E,H]; expert_gate/up [E,I,H]; expert_down [E,H,I];
    shared_gate/up [Is,H]; shared_down [H,Is].

    ``shared_expert_gate`` ([H] or [1,H]) is the extension for the Qwen3.6
    shape: the shared expert's output is scaled by ``sigmoid(x_norm . w_sg)``
    per row, with ``x_norm`` the post-RMSNorm activation.  ``None`` keeps the
    reference behaviour exactly.

    Returns (out [B,H] f32, indices [B,k] int64, weights [B,k] f32).
    """
    x_f = as_f32(x)
    x_norm = rms_norm(x_f, norm_weight, eps)                        # :42
    logits = (x_norm @ as_f32(router_weight).T).astype(np.float32)  # :43
    topk_logits, topk_idx = topk_desc(logits, top_k)                 # :44
    topk_w = softmax(topk_logits, axis=-1)                           # :45

    batch, hidden = x_f.shape
    out = np.zeros((batch, hidden), dtype=np.float32)                # :48
    for b in range(batch):                                           # :50-56
        for slot in range(top_k):
            e = int(topk_idx[b, slot])
            w = topk_w[b, slot]
            gate = silu(as_f32(expert_gate[e]) @ x_norm[b])
            up = as_f32(expert_up[e]) @ x_norm[b]
            out[b] += w * (as_f32(expert_down[e]) @ (gate * up))

    shared = silu(x_norm @ as_f32(shared_gate).T) * (x_norm @ as_f32(shared_up).T)  # :58
    shared_out = (shared @ as_f32(shared_down).T).astype(np.float32)                 # :59
    if shared_expert_gate is not None:
        wsg = as_f32(shared_expert_gate).reshape(-1)
        factor = sigmoid(x_norm @ wsg)                                # [B]
        shared_out = shared_out * factor[:, None]
    out += shared_out
    if add_residual:                                                  # :60-61
        out += x_f
    return out.astype(np.float32), topk_idx, topk_w


# ---------------------------------------------------------------------------
# Dense SwiGLU FFN  (reference.py:65-88)
# ---------------------------------------------------------------------------

def dense_ffn_decode(x, norm_weight, gate_weight, up_weight, down_weight, *, eps=1e-6, add_residual=True):
    """Restates ``dense_ffn_decode_reference`` (reference.py:65-88)."""
    x_f = as_f32(x)
    x_norm = rms_norm(x_f, norm_weight, eps)                                        # :83
    act = silu(x_norm @ as_f32(gate_weight).T) * (x_norm @ as_f32(up_weight).T)      # :84
    out = (act @ as_f32(down_weight).T).astype(np.float32)                          # :85
    if add_residual:
        out += x_f                                                                  # :86-87
    return out.astype(np.float32)


# ---------------------------------------------------------------------------
# Partial RoPE  (reference.py:91-114)
# ---------------------------------------------------------------------------

def apply_partial_rope(q, k, cos, sin, rotary_dim: int):
    """Rotate-half RoPE on the first ``rotary_dim`` dims (reference.py:91-114)."""
    if cos is None or sin is None or rotary_dim <= 0:
        return as_f32(q), as_f32(k)
    q = as_f32(q)
    k = as_f32(k)
    cos = as_f32(cos)
    sin = as_f32(sin)
    half = rotary_dim // 2

    def rot_half(t):
        return np.concatenate((-t[..., half:rotary_dim], t[..., :half]), axis=-1)

    q_rot, q_pass = q[..., :rotary_dim], q[..., rotary_dim:]
    k_rot, k_pass = k[..., :rotary_dim], k[..., rotary_dim:]
    while cos.ndim < q_rot.ndim:
        cos = cos[None]
        sin = sin[None]
    q_out = q_rot * cos + rot_half(q_rot) * sin
    kc, ks = cos, sin
    while kc.ndim < k_rot.ndim:
        kc = kc[None]
        ks = ks[None]
    k_out = k_rot * kc + rot_half(k_rot) * ks
    return (np.concatenate((q_out, q_pass), axis=-1).astype(np.float32),
            np.concatenate((k_out, k_pass), axis=-1).astype(np.float32))


# ---------------------------------------------------------------------------
# GQA attention decode  (reference.py:117-145)
# ---------------------------------------------------------------------------

def full_attention_decode(q, k_cache, v_cache, *, scale: Optional[float] = None) -> np.ndarray:
    """Restates ``full_attention_decode_reference`` (reference.py:117-145).

    q [B,Hq,D]; k_cache/v_cache [B,T,Hkv,D]; q-head ``qh`` reads kv head
    ``qh // (Hq // Hkv)``.  Returns [B,Hq,D] f32.
    """
    q = np.asarray(q)
    batch, query_heads, head_dim = q.shape
    kv_heads = k_cache.shape[2]
    if query_heads % kv_heads != 0:
        raise ValueError("query_heads must be divisible by kv_heads")   # :133-134
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    group = query_heads // kv_heads
    outs = []
    for qh in range(query_heads):                                         # :140-144
        kvh = qh // group
        qf = as_f32(q[:, qh])                                             # [B,D]
        kf = as_f32(k_cache[:, :, kvh])                                   # [B,T,D]
        vf = as_f32(v_cache[:, :, kvh])
        scores = np.einsum("bd,btd->bt", qf, kf).astype(np.float32) * np.float32(scale)
        probs = softmax(scores, axis=-1)
        outs.append(np.einsum("bt,btd->bd", probs, vf).astype(np.float32))
    return np.stack(outs, axis=1).astype(np.float32)


# ---------------------------------------------------------------------------
# Linear attention  (reference.py:148-166) and the gated delta rule
# ---------------------------------------------------------------------------

def linear_attention_decode(q, k, v, state, *, decay: float = 1.0):
    """Restates ``linear_attention_decode_reference`` (reference.py:148-166).

    ``S' = decay * S + k (x) v``;  ``o = q^T S'``.
    q/k [B,H,Dk]; v [B,H,Dv]; state [B,H,Dk,Dv].  Returns (o f32, S' f32).
    """
    new_state = as_f32(state) * np.float32(decay) + np.einsum("bhd,bhv->bhdv", as_f32(k), as_f32(v))
    new_state = new_state.astype(np.float32)
    out = np.einsum("bhd,bhdv->bhv", as_f32(q), new_state).astype(np.float32)
    return out, new_state


def gated_delta_decode(q, k, v, state, g, beta, qk_l2norm=False, q_scale=None):
    """Gated delta rule, one decode step (the task's config-5 formula).

    Per batch row b and v-head j (q/k head ``h = j // (Hv // Hk)``)::

        S  <- exp(g[b,j]) * S
        u  <- v[b,j] - S^T k[b,h]
        S  <- S + beta[b,j] * k[b,h] (x) u
        o  <- S^T q[b,h]

    No 1/sqrt(Dk) scale is applied to q (a caller folds it into q), unless
    ``qk_l2norm``: then q and k are first L2-normalised in FP32,
    x / sqrt(sum x^2 + 1e-6) over Dk, and q is multiplied by ``q_scale``
    (default 1/sqrt(Dk)) -- the ``use_qk_l2norm_in_kernel`` form of
    transformers' ``torch_recurrent_gated_delta_rule`` (modeling_qwen3_next.py
    l2norm and scale, transformers 5.15.0).
    q/k [B,Hk,Dk]; v [B,Hv,Dv]; state [B,Hv,Dk,Dv] f32; g/beta [B,Hv] f32.
    Returns (o [B,Hv,Dv] f32, new_state f32).
    """
    qf, kf, vf = as_f32(q), as_f32(k), as_f32(v)
    if qk_l2norm:
        dk = qf.shape[-1]
        scale = np.float32(1.0 / np.sqrt(dk) if q_scale is None else q_scale)
        qf = (qf / np.sqrt((qf * qf).sum(-1, keepdims=True) + np.float32(1e-6)) * scale).astype(np.float32)
        kf = (kf / np.sqrt((kf * kf).sum(-1, keepdims=True) + np.float32(1e-6))).astype(np.float32)
    s = as_f32(state).copy()
    g = as_f32(g)
    beta = as_f32(beta)
    batch, hk, dk = qf.shape
    hv = vf.shape[1]
    if hv % hk != 0:
        raise ValueError("value heads must be a multiple of key heads")
    rep = hv // hk
    out = np.empty((batch, hv, vf.shape[2]), dtype=np.float32)
    for b in range(batch):
        for j in range(hv):
            h = j // rep
            sj = s[b, j] * np.float32(np.exp(g[b, j]))                      # [Dk,Dv]
            u = vf[b, j] - kf[b, h] @ sj                                     # [Dv]
            sj = sj + np.float32(beta[b, j]) * np.outer(kf[b, h], u).astype(np.float32)
            s[b, j] = sj
            out[b, j] = qf[b, h] @ sj
    return out, s.astype(np.float32)


def causal_conv1d_update(x, conv_state, weight, bias=None, *, silu_activation=True, bf16=True):
    """One token through the depthwise causal convolution of the Qwen3.6
    linear-attention step (transformers 5.15.0 ``causal_conv1d_update``,
    modeling_qwen3_next.py: window = [state, x], conv over the window, SiLU,
    state <- window[1:]).  x [B, C]; conv_state [B, C, S]; weight [C, S+1];
    bias [C] or None.  With ``bf16`` the convolution and the SiLU are each
    rounded to bfloat16, as the model's bf16 ops round them.
    Returns (out [B, C] f32, new_state [B, C, S] f32)."""
    xf = as_f32(x)
    st = as_f32(conv_state)
    w = as_f32(weight)
    win = np.concatenate([st, xf[..., None]], axis=-1)                      # [B, C, S+1]
    acc = (win.astype(np.float64) * w.astype(np.float64)[None]).sum(-1).astype(np.float32)
    if bias is not None:
        acc = (acc + as_f32(bias)[None]).astype(np.float32)
    rnd = bf16_round if bf16 else (lambda a: a.astype(np.float32))
    y = rnd(acc)
    if silu_activation:
        y = rnd(silu(y))
    return y, win[..., 1:].astype(np.float32)


def gated_rms_norm(x, gate, weight, *, eps=1e-6, bf16=True):
    """Norm-before-gate RMSNorm of the Qwen3.6 linear-attention output
    (transformers 5.15.0 ``Qwen3NextRMSNormGated.forward``): n = x *
    rsqrt(mean(x^2) + eps) in FP32, rounded to the input dtype; t = weight * n
    rounded; out = t * silu(gate) in FP32, rounded."""
    rnd = bf16_round if bf16 else (lambda a: a.astype(np.float32))
    xf = as_f32(x)
    var = np.mean(xf * xf, axis=-1, keepdims=True, dtype=np.float32)
    n = rnd(xf * (np.float32(1.0) / np.sqrt(var + np.float32(eps))))
    t = rnd(as_f32(weight) * n)
    return rnd(t * silu(as_f32(gate)))


def attention_cache_view(fa: dict):
    """The contiguous [B, T, Hkv, D] float32 caches that one attention step
    reads, given the fields of ``FullAttentionInputs`` as a dict.

    The reference reads ``k_cache``/``v_cache`` as they are (ops.py:367-374).
    The two optional layouts of this build are restated as their definitions:

    * ``k_new``/``v_new`` (KV append): the new token's key and value
      [B, Hkv, D] are written to row ``cache_seqlen`` (default: the last row)
      of copies of the caches, and the first ``cache_seqlen + 1`` tokens are
      read;
    * ``block_table`` [B, max_blocks] (paged KV): the caches are block pools
      [num_blocks, block_size, Hkv, D]; token t of row b is row
      ``t % block_size`` of block ``block_table[b, t // block_size]``; a block
      id outside the pool reads as zeros and is never written.  ``seq_len``
      tokens are read (default max_blocks * block_size; with an append,
      ``cache_seqlen + 1`` when given).
    """
    kc, vc = as_f32(fa["k_cache"]), as_f32(fa["v_cache"])
    k_new, v_new = fa.get("k_new"), fa.get("v_new")
    if (k_new is None) != (v_new is None):
        raise ValueError("k_new and v_new must be given together")
    table = fa.get("block_table")
    if table is None:
        if k_new is None:
            return kc, vc
        b, cap, hkv, d = kc.shape
        pos = cap - 1 if fa.get("cache_seqlen") is None else int(fa["cache_seqlen"])
        if not 0 <= pos < cap:
            raise ValueError("cache_seqlen must leave room for the new token")
        kc, vc = kc.copy(), vc.copy()
        kc[:, pos] = as_f32(k_new).reshape(b, hkv, d)
        vc[:, pos] = as_f32(v_new).reshape(b, hkv, d)
        return kc[:, :pos + 1], vc[:, :pos + 1]
    table = np.asarray(table).astype(np.int64)
    nblocks, bs, hkv, d = kc.shape
    batch, max_blocks = table.shape
    seq = max_blocks * bs if fa.get("seq_len") is None else int(fa["seq_len"])
    if k_new is not None and fa.get("cache_seqlen") is not None:
        seq = int(fa["cache_seqlen"]) + 1
    if not 0 < seq <= max_blocks * bs:
        raise ValueError("seq_len must be in [1, max_blocks * block_size]")
    if k_new is not None:
        kc, vc = kc.copy(), vc.copy()
        kn, vn = as_f32(k_new).reshape(batch, hkv, d), as_f32(v_new).reshape(batch, hkv, d)
        for b in range(batch):
            blk = table[b, (seq - 1) // bs]
            if 0 <= blk < nblocks:
                kc[blk, (seq - 1) % bs] = kn[b]
                vc[blk, (seq - 1) % bs] = vn[b]
    k = np.zeros((batch, seq, hkv, d), np.float32)
    v = np.zeros((batch, seq, hkv, d), np.float32)
    for b in range(batch):
        for t in range(seq):
            blk = table[b, t // bs]
            if 0 <= blk < nblocks:
                k[b, t] = kc[blk, t % bs]
                v[b, t] = vc[blk, t % bs]
    return k, v


# ---------------------------------------------------------------------------
# decode_layer composition  (ops.py:701-748)
# ---------------------------------------------------------------------------

def decode_layer(
    hidden,
    *,
    kind: str,
    moe: Optional[dict] = None,
    dense_ffn: Optional[dict] = None,
    full_attention: Optional[dict] = None,
    linear_attention: Optional[dict] = None,
    eps: float = 1e-6,
    top_k: int = 8,
    round_to_bf16: bool = True,
):
    """Restates ``decode_layer`` (ops.py:701-748) over the oracle's ops.

    The dicts carry the same fields as the API's dataclasses.  An ``out_proj``
    entry ([H, heads*dim]) projects the attention output onto the hidden size
    before the residual add; without it the output is reshaped, as in the
    reference (ops.py:722,728).  With ``round_to_bf16`` each op's output is
    rounded to bfloat16 before it feeds the next op, as it is on the bf16
    device path.
    """
    h = as_f32(hidden)
    rnd = bf16_round if round_to_bf16 else (lambda a: a)
    res = {"attention_output": None, "linear_output": None, "linear_state": None,
           "router_indices": None, "router_weights": None}
    if kind == "full_attention":
        if full_attention is None:
            raise ValueError("full_attention inputs are required for full_attention layers")
        fa = dict(full_attention)
        if fa.get("qkv_proj") is not None:
            # q, then the new token's key and value, from the layer input
            kv_h, hd = np.shape(fa["k_cache"])[-2], np.shape(fa["k_cache"])[-1]
            qkv = rms_norm_linear(h.reshape(h.shape[0], -1), fa["input_norm"], fa["qkv_proj"], eps,
                                  round_to_bf16=round_to_bf16)
            qd = qkv.shape[1] - 2 * kv_h * hd
            if qd <= 0 or qd % hd:
                raise ValueError("qkv_proj must have (q_heads + 2 * kv_heads) * head_dim rows")
            b = qkv.shape[0]
            fa["q"] = qkv[:, :qd].reshape(b, qd // hd, hd)
            fa["k_new"] = qkv[:, qd:qd + kv_h * hd].reshape(b, kv_h, hd)
            fa["v_new"] = qkv[:, qd + kv_h * hd:].reshape(b, kv_h, hd)
        k_cache, v_cache = attention_cache_view(fa)
        q, kc = apply_partial_rope(fa["q"], k_cache, fa.get("cos"), fa.get("sin"), fa.get("rotary_dim", 64))
        a = rnd(full_attention_decode(q, kc, v_cache, scale=fa.get("scale")))
        if fa.get("out_proj") is not None:
            a = rnd(a.reshape(a.shape[0], -1) @ as_f32(fa["out_proj"]).T)
        a = a.reshape(h.shape)
        res["attention_output"] = a
        resid = rnd(h + a)
    elif kind == "linear_attention":
        if linear_attention is None:
            raise ValueError("linear_attention inputs are required for linear_attention layers")
        la = dict(linear_attention)
        if la.get("in_proj") is not None:
            # q, k and v from the layer input: rows [q | k | v] of in_proj
            _, hv, dk, dv = np.shape(la["state"])
            qkv = rms_norm_linear(h.reshape(h.shape[0], -1), la["input_norm"], la["in_proj"], eps,
                                  round_to_bf16=round_to_bf16)
            kd = qkv.shape[1] - hv * dv
            if kd <= 0 or kd % (2 * dk):
                raise ValueError("in_proj must have 2 * k_heads * key_dim + v_heads * value_dim rows")
            b, hk = qkv.shape[0], kd // (2 * dk)
            la["q"] = qkv[:, :hk * dk].reshape(b, hk, dk)
            la["k"] = qkv[:, hk * dk:kd].reshape(b, hk, dk)
            la["v"] = qkv[:, kd:].reshape(b, hv, dv)
        if la.get("g") is not None:
            o, s = gated_delta_decode(la["q"], la["k"], la["v"], la["state"], la["g"], la["beta"],
                                      qk_l2norm=bool(la.get("qk_l2norm", False)), q_scale=la.get("q_scale"))
        else:
            if la.get("qk_l2norm"):
                raise ValueError("qk_l2norm needs the gated delta rule (g and beta)")
            o, s = linear_attention_decode(la["q"], la["k"], la["v"], la["state"], decay=la.get("decay", 1.0))
        o = rnd(o)
        if la.get("out_proj") is not None:
            o = rnd(o.reshape(o.shape[0], -1) @ as_f32(la["out_proj"]).T)
        o = o.reshape(h.shape)
        res["linear_output"] = o
        res["linear_state"] = s
        resid = rnd(h + o)
    else:
        raise ValueError(f"unsupported layer_type: {kind}")
    if dense_ffn is not None:
        d = dense_ffn
        out = dense_ffn_decode(resid, d["norm_weight"], d["gate_weight"], d["up_weight"], d["down_weight"],
                               eps=eps, add_residual=True)
    else:
        if moe is None:
            raise ValueError("either moe or dense_ffn weights are required")
        m = moe
        out, idx, w = moe_decode(resid, m["norm_weight"], m["router_weight"], m["expert_gate"], m["expert_up"],
                                 m["expert_down"], m["shared_gate"], m["shared_up"], m["shared_down"],
                                 eps=eps, top_k=top_k, add_residual=True,
                                 shared_expert_gate=m.get("shared_expert_gate"))
        res["router_indices"] = idx
        res["router_weights"] = w
    res["residual"] = resid  # the FFN/MoE input: hidden plus the mixer output
    res["hidden"] = out
    return res


# Which independent check pins each function (see tests/test_oracle.py).
PINNING = {
    "rms_norm": "torch.nn.functional.rms_norm (library); golden vectors (float64 torch)",
    "topk_desc": "torch.topk on distinct values; tie rule (lower index first) by construction",
    "moe_decode": "E=1,k=1 reduces to dense FFN + shared; identical experts => routed part independent "
                  "of routing; w_sg=0 => shared factor 0.5; golden vectors (float64 torch composition)",
    "dense_ffn_decode": "zero gate => out = x; F.linear/F.silu float64 composition; golden vectors",
    "apply_partial_rope": "rotary_dim=0 / cos=1,sin=0 identity; norm preservation of rotated pairs",
    "full_attention_decode": "F.scaled_dot_product_attention(enable_gqa=True); T=1 => out=v; constant K => mean(V)",
    "linear_attention_decode": "decay=0 => S'=k v^T; closed-form o=(q.k) v + decay q^T S",
    "gated_delta_decode": "beta=0 => S'=e^g S; g=0,beta=0 => S'=S; |k|=1,beta=1 => S'^T k = v; "
                          "S=0,beta=1 => S'=k v^T; transformers' recurrent gated delta rule loop; "
                          "qk_l2norm: output invariant under positive scaling of q and k, beta=1 => "
                          "S'^T (k/|k|) = v for any k, S=0,beta=1 => o = scale cos(q,k) v, and the "
                          "transformers loop with use_qk_l2norm_in_kernel",
    "causal_conv1d_update": "transformers' causal_conv1d_update (torch conv1d) on float32 and bfloat16; last-tap weight 1 "
                            "and no activation => out = x and the state shifts by one",
    "gated_rms_norm": "transformers' Qwen3NextRMSNormGated on float32 and bfloat16; constant rows => "
                      "weight * sign(x) * silu(gate)",
    "attention_cache_view": "append: the written row reads back and every other row is untouched; paged: "
                            "a shuffled pool of blocks gathers back to the contiguous cache it was cut from, "
                            "out-of-pool ids read as zeros",
    "rms_norm_linear": "float64 torch F.linear(F.rms_norm(x).to(bf16)) composition; identity projection => "
                       "the rounded norm itself; a scaled input gives the same output (scale invariance of the norm)",
    "decode_layer": "float64 torch composition of ops.py:701-748 (library attention, transformers' gated "
                    "delta loop, float64 SwiGLU/MoE) with and without bf16 rounding between ops; zero out_proj "
                    "=> MoE of the input; zero-gate dense FFN => round(hidden + mixer output); the reshape "
                    "path; ValueError texts of ops.py:720-739",
}
