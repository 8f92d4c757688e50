"""Decode-path operator API for Qwen3.6 on MI355X (gfx950).

Drop-in for the reference's ``mega_kernel_qwen36/ops.py`` decode surface:
``moe_decode``, ``dense_ffn_decode``, ``full_attention_decode``,
``linear_attention_decode`` and ``decode_layer`` keep their signatures,
dataclasses and ``ValueError`` messages.  The default backends run the
hand-written HIP kernels of ``libmkq.so`` through the ``_C`` extension.

Differences from the reference, all deliberate:

* There is no silent fallback.  When ``_C`` is missing or a tensor is not on a
  GPU, the HIP backends raise ``RuntimeError``.  The reference instead drops to
  its CPU ``reference.py`` (ops.py:29-32,149-150,307).
* ``backend="reference"`` names the CPU oracle.  This build keeps the oracle
  outside the product (it is test infrastructure), so asking for it raises.
* ``backend="auto"`` goes to the HIP kernels for MoE and the dense FFN.  The
  reference sends ``auto`` to the grouped torch composite (ops.py:299-300,
  340-341).  ``"grouped"`` (MoE) and ``"torch"`` (dense) are still available
  as explicitly chosen torch composites, and ``"triton"`` maps to HIP.
* Optional extensions used by the Qwen3.6 shapes (reference has no code for
  them): ``GatedMoeWeights.shared_expert_gate`` (sigmoid-gated shared expert),
  ``LinearAttentionInputs.g/beta`` (gated delta rule) and ``out_proj`` on both
  attention input dataclasses (projection onto the hidden size inside
  ``decode_layer``).
"""

from __future__ import annotations

import dataclasses
import math
import os
import weakref
from dataclasses import dataclass
from typing import Optional, Tuple

import torch
import torch.nn.functional as F

from .config import qwen36_layer_type

try:
    from . import _C  # HIP kernels (libmkq.so) behind a thin torch binding
    _C_IMPORT_ERROR: Optional[BaseException] = None
except Exception as exc:  # pragma: no cover - exercised when the extension is not built
    _C = None
    _C_IMPORT_ERROR = exc


# ---------------------------------------------------------------------------
# dataclasses (reference ops.py:38-75,129-136)
# ---------------------------------------------------------------------------

@dataclass(frozen=True)
class MoeWeights:
    norm_weight: torch.Tensor
    router_weight: torch.Tensor
    expert_gate: torch.Tensor
    expert_up: torch.Tensor
    expert_down: torch.Tensor
    shared_gate: torch.Tensor
    shared_up: torch.Tensor
    shared_down: torch.Tensor


@dataclass(frozen=True)
class GatedMoeWeights(MoeWeights):
    """MoE weights whose shared expert is scaled by ``sigmoid(x_norm . shared_expert_gate)``.

    ``shared_expert_gate`` is ``[hidden]`` or ``[1, hidden]``; the gate reads the
    post-RMSNorm activation (as Qwen3-Next/Qwen3.6's sparse MoE block does).
    """

    shared_expert_gate: torch.Tensor = None  # type: ignore[assignment]


@dataclass(frozen=True)
class DenseFfnWeights:
    norm_weight: torch.Tensor
    gate_weight: torch.Tensor
    up_weight: torch.Tensor
    down_weight: torch.Tensor


@dataclass(frozen=True)
class FullAttentionInputs:
    q: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    cos: Optional[torch.Tensor] = None
    sin: Optional[torch.Tensor] = None
    rotary_dim: int = 64
    scale: Optional[float] = None
    out_proj: Optional[torch.Tensor] = None  # [hidden, q_heads*head_dim], used by decode_layer
    # KV append (no counterpart in the reference): the new token's key and
    # value [batch, kv_heads, head_dim], written in place into the caches'
    # row `cache_seqlen` (default: their last row) before attending over the
    # first cache_seqlen + 1 tokens.
    k_new: Optional[torch.Tensor] = None
    v_new: Optional[torch.Tensor] = None
    cache_seqlen: Optional[int] = None
    # Paged KV (no counterpart in the reference): with a block_table
    # [batch, max_blocks] (int32), k_cache/v_cache are block pools
    # [num_blocks, block_size, kv_heads, head_dim] and seq_len tokens are read
    # (default max_blocks * block_size).
    block_table: Optional[torch.Tensor] = None
    seq_len: Optional[int] = None
    # Input projection, used by decode_layer (the reference plans it as the
    # rmsnorm -> linear "qkv" tasks, mpk_graph.py:349-373): with qkv_proj
    # [(q_heads + 2*kv_heads)*head_dim, hidden] and input_norm [hidden], q,
    # k_new and v_new come from rms_norm(hidden) @ qkv_proj^T, in that order,
    # in one launch, and q may be None.
    qkv_proj: Optional[torch.Tensor] = None
    input_norm: Optional[torch.Tensor] = None


@dataclass(frozen=True)
class LinearAttentionInputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    state: torch.Tensor
    decay: float = 1.0
    g: Optional[torch.Tensor] = None      # [batch, v_heads] f32: selects the gated delta rule
    beta: Optional[torch.Tensor] = None   # [batch, v_heads] f32
    out_proj: Optional[torch.Tensor] = None  # [hidden, v_heads*value_dim], used by decode_layer
    # Gated rule only: L2-normalise q and k inside the kernel (FP32) and scale
    # q by q_scale (default 1/sqrt(key_dim)), as use_qk_l2norm_in_kernel does.
    qk_l2norm: bool = False
    q_scale: Optional[float] = None
    # Input projection, used by decode_layer: with in_proj
    # [2*k_heads*key_dim + v_heads*value_dim, hidden] and input_norm [hidden],
    # q, k and v come from rms_norm(hidden) @ in_proj^T (rows [q | k | v]) in
    # one launch, and q, k, v may be None.
    in_proj: Optional[torch.Tensor] = None
    input_norm: Optional[torch.Tensor] = None


@dataclass(frozen=True)
class DecodeLayerResult:
    hidden: torch.Tensor
    router_indices: Optional[torch.Tensor] = None
    router_weights: Optional[torch.Tensor] = None
    attention_output: Optional[torch.Tensor] = None
    linear_output: Optional[torch.Tensor] = None
    linear_state: Optional[torch.Tensor] = None


# ---------------------------------------------------------------------------
# dispatch predicates (reference ops.py:145-158)
# ---------------------------------------------------------------------------

def extension_available() -> bool:
    return _C is not None


def _use_extension(*tensors: torch.Tensor) -> bool:
    return _C is not None and all(t.is_cuda for t in tensors)


def _require_extension(op: str, *tensors: torch.Tensor) -> None:
    if _C is None:
        raise RuntimeError(
            f"{op}: the HIP extension mega_kernel_qwen36._C is not loaded "
            f"({_C_IMPORT_ERROR!r}); build it with mega-kernel-3.6_amd/build.py"
        )
    if not all(t.is_cuda for t in tensors):
        raise RuntimeError(f"{op}: the HIP kernels need every tensor on a GPU (got a CPU tensor)")


def _matmul_dtype(x: torch.Tensor) -> torch.dtype:
    return x.dtype if (x.is_cuda and x.dtype in (torch.float16, torch.bfloat16)) else torch.float32


def _no_reference(op: str) -> RuntimeError:
    return RuntimeError(
        f"{op}: backend='reference' is the CPU oracle, which this build keeps as test infrastructure "
        "(oracle/); use the HIP backend ('auto')"
    )


def _rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps) * weight.float()).to(x.dtype)


# ---------------------------------------------------------------------------
# torch composites (explicitly chosen backends only)
# ---------------------------------------------------------------------------

def _moe_decode_grouped_torch(x, w: MoeWeights, *, eps, top_k, add_residual):
    """Grouped-GEMM torch composite of the MoE (the reference's "grouped" backend, ops.py:161-199)."""
    x_norm = _rms_norm(x, w.norm_weight, eps).float()
    topk_logits, topk_idx = torch.topk(x_norm @ w.router_weight.float().t(), k=top_k, dim=-1)
    topk_w = torch.softmax(topk_logits, dim=-1)
    batch, hidden = x.shape
    mm = _matmul_dtype(x)
    sel = topk_idx.reshape(-1)
    xs = x_norm.to(mm).repeat_interleave(top_k, dim=0).unsqueeze(-1).contiguous()  # [B*k, H, 1]
    gate = torch.bmm(w.expert_gate.index_select(0, sel), xs).squeeze(-1).float()
    up = torch.bmm(w.expert_up.index_select(0, sel), xs).squeeze(-1).float()
    act = F.silu(gate) * up * topk_w.reshape(-1, 1)
    routed = torch.bmm(w.expert_down.index_select(0, sel), act.to(mm).unsqueeze(-1).contiguous())
    routed = routed.squeeze(-1).float().view(batch, top_k, hidden).sum(dim=1)
    xm = x_norm.to(mm)
    shared_act = F.silu(F.linear(xm, w.shared_gate).float()) * F.linear(xm, w.shared_up).float()
    shared = F.linear(shared_act.to(mm), w.shared_down).float()
    sg = getattr(w, "shared_expert_gate", None)
    if sg is not None:
        shared = shared * torch.sigmoid(x_norm @ sg.float().reshape(-1, 1))
    out = routed + shared
    if add_residual:
        out = out + x.float()
    return out.to(x.dtype), topk_idx, topk_w


def _dense_ffn_decode_torch(x, w: DenseFfnWeights, *, eps, add_residual):
    """torch composite of the dense FFN (the reference's "torch" backend, ops.py:202-218)."""
    mm = _matmul_dtype(x)
    xm = _rms_norm(x, w.norm_weight, eps).to(mm)
    act = F.silu(F.linear(xm, w.gate_weight).float()) * F.linear(xm, w.up_weight).float()
    out = F.linear(act.to(mm), w.down_weight).float()
    if add_residual:
        out = out + x.float()
    return out.to(x.dtype)


# ---------------------------------------------------------------------------
# public decode ops
# ---------------------------------------------------------------------------

def _moe_tensors(x, weights: MoeWeights):
    return (
        x,
        weights.norm_weight,
        weights.router_weight,
        weights.expert_gate,
        weights.expert_up,
        weights.expert_down,
        weights.shared_gate,
        weights.shared_up,
        weights.shared_down,
    )


def moe_decode(
    x: torch.Tensor,
    weights: MoeWeights,
    *,
    eps: float = 1e-6,
    top_k: int = 8,
    add_residual: bool = True,
    backend: str = "auto",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Fused MoE decode step.  Returns ``(out [B,H] x.dtype, indices [B,k] int64, weights [B,k] f32)``.

    ``auto``/``persistent``: one persistent HIP launch (RMSNorm, router, top-k
    softmax, routed SwiGLU experts, shared expert, down projection, residual).
    """
    if backend not in {"auto", "persistent", "grouped", "reference"}:
        raise ValueError("backend must be one of: auto, persistent, grouped, reference")
    tensors = _moe_tensors(x, weights)
    if backend == "grouped":
        return _moe_decode_grouped_torch(x, weights, eps=eps, top_k=top_k, add_residual=add_residual)
    if backend == "reference":
        raise _no_reference("moe_decode")
    _require_extension("moe_decode", *tensors)
    sg = getattr(weights, "shared_expert_gate", None)
    if sg is not None:
        return _check_moe(_C.moe_decode_persistent_gated(*tensors, sg, float(eps), int(top_k), bool(add_residual)))
    return _check_moe(_C.moe_decode_persistent(*tensors, float(eps), int(top_k), bool(add_residual)))


def moe_decode_status(*, reset: bool = False) -> int:
    """Error word of the persistent MoE on the current device and stream.

    0: no cross-workgroup wait has timed out since the last reset.  1: one
    has (for example because a kernel on another stream held CUs while the
    MoE's workgroups waited for each other); that call and every later one on
    the stream wrote NaN outputs, and they keep doing so until ``reset=True``
    clears the workspace.  Synchronises the stream, so it is not for use
    inside graph capture.  Set ``MKQ_MOE_CHECK=1`` to have every
    ``moe_decode`` call check it and raise (a debugging aid: it synchronises
    after each call).  No counterpart in the reference, whose cooperative
    launch either runs or fails at launch.
    """
    if _C is None:
        raise RuntimeError(f"moe_decode_status: the HIP extension is not loaded ({_C_IMPORT_ERROR!r})")
    return int(_C.moe_decode_status(bool(reset)))


def _check_moe(result):
    if os.environ.get("MKQ_MOE_CHECK", "0") not in ("", "0"):
        code = moe_decode_status(reset=True)
        if code:
            raise RuntimeError(f"moe_decode: a cross-workgroup wait timed out (error word {code}); "
                               "the outputs are NaN and the workspace has been reset")
    return result


def dense_ffn_decode(
    x: torch.Tensor,
    weights: DenseFfnWeights,
    *,
    eps: float = 1e-6,
    add_residual: bool = True,
    backend: str = "auto",
) -> torch.Tensor:
    """Fused RMSNorm + SwiGLU FFN decode step (HIP).  ``x [B,H]`` -> ``[B,H]``."""
    tensors = (x, weights.norm_weight, weights.gate_weight, weights.up_weight, weights.down_weight)
    if backend not in {"auto", "torch", "triton", "reference"}:
        raise ValueError("backend must be one of: auto, torch, triton, reference")
    if backend == "torch":
        return _dense_ffn_decode_torch(x, weights, eps=eps, add_residual=add_residual)
    if backend == "reference":
        raise _no_reference("dense_ffn_decode")
    _require_extension("dense_ffn_decode", *tensors)
    return _C.dense_ffn_decode(*tensors, float(eps), bool(add_residual))


def _rope_one(t, cos, sin, rotary_dim: int):
    """Rotate-half RoPE of one tensor; cos/sin FP32, broadcast over its leading dims."""
    half = rotary_dim // 2
    tr = t[..., :rotary_dim].float()
    rh = torch.cat((-tr[..., half:], tr[..., :half]), dim=-1)
    c, s = cos, sin
    while c.ndim < tr.ndim:
        c, s = c.unsqueeze(0), s.unsqueeze(0)
    return torch.cat(((tr * c + rh * s).to(t.dtype), t[..., rotary_dim:]), dim=-1)


def apply_partial_rope(q, k, cos, sin, rotary_dim: int):
    """Rotate-half RoPE on the first ``rotary_dim`` dims of q and k (reference.py:91-114)."""
    if cos is None or sin is None or rotary_dim <= 0:
        return q, k
    cos = cos.to(device=q.device, dtype=torch.float32)
    sin = sin.to(device=q.device, dtype=torch.float32)
    return _rope_one(q, cos, sin, rotary_dim), _rope_one(k, cos, sin, rotary_dim)


# Last (cos, sin) vector built for the kernel: weak references to the source
# tensors and their version counters, so a tensor that is modified in place,
# replaced or freed is never matched.
_ROPE_CS_CACHE: dict = {}


def _rope_in_kernel(inputs: FullAttentionInputs) -> Optional[torch.Tensor]:
    """The (cos, sin) pair as one device vector when the kernel can rotate the
    keys itself: one vector for every token and head (what the reference
    broadcasts), a power-of-two rotary_dim in [16, head_dim], bf16/f16 and a
    head_dim that is a multiple of 8.  None otherwise."""
    cos, sin, rot = inputs.cos, inputs.sin, inputs.rotary_dim
    k = inputs.k_cache
    d = k.shape[-1]
    if cos is None or sin is None or rot <= 0:
        return None
    if cos.numel() != rot or sin.numel() != rot or rot < 16 or rot > d or rot & (rot - 1) or d % 8:
        return None
    if k.dtype not in (torch.bfloat16, torch.float16) or not k.is_cuda:
        return None
    c = _ROPE_CS_CACHE
    versions = (cos._version, sin._version)
    if c and c["cos"]() is cos and c["sin"]() is sin and c["versions"] == versions and c["device"] == k.device:
        return c["cs"]
    cs = torch.cat((cos.reshape(-1), sin.reshape(-1))).to(device=k.device, dtype=torch.float32).contiguous()
    c.update(cos=weakref.ref(cos), sin=weakref.ref(sin), versions=versions, device=k.device, cs=cs)
    return cs


def _attention_append(inputs: FullAttentionInputs) -> torch.Tensor:
    """KV append fused into the attention step.  k_new/v_new go to row
    p = cache_seqlen (default: the last row) of k_cache/v_cache [batch,
    capacity, kv_heads, head_dim], in place, and the result is
    full_attention_decode over the first p + 1 tokens.  Where the kernel
    supports it (bf16/f16, head_dim % 8 == 0, 16-byte aligned tensors, RoPE in
    the kernel or none), the attention kernel writes the rows itself and
    uses the new key and value without reading them back; otherwise the rows
    are written first.  The reference's callers write the cache themselves
    before full_attention_decode (ops.py:367-374)."""
    if inputs.k_new is None or inputs.v_new is None:
        raise ValueError("k_new and v_new must be given together")
    k_cache, v_cache = inputs.k_cache, inputs.v_cache
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache must be [batch, capacity, kv_heads, head_dim]")
    b, cap, hkv, d = k_cache.shape
    pos = cap - 1 if inputs.cache_seqlen is None else int(inputs.cache_seqlen)
    if not 0 <= pos < cap:
        raise ValueError("cache_seqlen must leave room for the new token")
    q = inputs.q
    if q.shape[1] % hkv != 0:
        raise ValueError("query_heads must be divisible by kv_heads")
    k_new = inputs.k_new.reshape(b, hkv, d)
    v_new = inputs.v_new.reshape(b, hkv, d)
    _require_extension("full_attention_decode", q, k_cache, v_cache, k_new, v_new)
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache and v_cache must be contiguous: the new token is written in place")
    rope = inputs.cos is not None and inputs.sin is not None
    cs = _rope_in_kernel(inputs) if rope else None
    if (k_cache.dtype in (torch.bfloat16, torch.float16) and d % 8 == 0 and (cs is not None or not rope)
            and all(t.dtype == k_cache.dtype for t in (q, k_new, v_new, v_cache))):
        qc, kn, vn = q.contiguous(), k_new.contiguous(), v_new.contiguous()
        if all(t.data_ptr() % 16 == 0 for t in (qc, kn, vn, k_cache, v_cache)):
            scale = inputs.scale if inputs.scale is not None else 1.0 / math.sqrt(d)
            rot = int(inputs.rotary_dim) if cs is not None else 0
            return _C.full_attention_decode_append(qc, kn, vn, k_cache, v_cache, pos + 1, float(scale), cs, rot)
    k_cache[:, pos] = k_new
    v_cache[:, pos] = v_new
    return full_attention_decode(dataclasses.replace(inputs, k_cache=k_cache[:, :pos + 1],
                                                     v_cache=v_cache[:, :pos + 1], k_new=None, v_new=None,
                                                     cache_seqlen=None))


def _attention_paged(inputs: FullAttentionInputs) -> torch.Tensor:
    """Attention over a paged KV pool: token t of batch row b is row
    t % block_size of block block_table[b, t // block_size].  The kernel reads
    the blocks in place (bf16/f16, head_dim % 8 == 0, block_size % 16 == 0);
    other cases gather the rows into a contiguous cache first.  With
    k_new/v_new the new token is token seq_len - 1 (or cache_seqlen): the
    kernel writes it into its block and uses it directly; the fallback
    writes the row first.  With cos/sin, q and the keys are rotated in the
    kernel where it can (with or without the append); otherwise the rows are
    gathered and the contiguous path rotates them."""
    if (inputs.k_new is None) != (inputs.v_new is None):
        raise ValueError("k_new and v_new must be given together")
    kb, vb, table = inputs.k_cache, inputs.v_cache, inputs.block_table
    if kb.dim() != 4 or vb.shape != kb.shape:
        raise ValueError("k_cache and v_cache must be [num_blocks, block_size, kv_heads, head_dim] with a block_table")
    q = inputs.q
    nblocks, bs, hkv, d = kb.shape
    if table.dim() != 2 or table.shape[0] != q.shape[0]:
        raise ValueError("block_table must be [batch, max_blocks]")
    seq = int(inputs.seq_len) if inputs.seq_len is not None else table.shape[1] * bs
    append = inputs.k_new is not None
    if append and inputs.cache_seqlen is not None:
        seq = int(inputs.cache_seqlen) + 1
    if not 0 < seq <= table.shape[1] * bs:
        raise ValueError("seq_len must be in [1, max_blocks * block_size]")
    if q.shape[1] % hkv != 0:
        raise ValueError("query_heads must be divisible by kv_heads")
    _require_extension("full_attention_decode", q, kb, vb, table)
    scale = inputs.scale if inputs.scale is not None else 1.0 / math.sqrt(d)
    if append:
        if not (kb.is_contiguous() and vb.is_contiguous()):
            raise ValueError("k_cache and v_cache must be contiguous: the new token is written in place")
        k_new = inputs.k_new.reshape(q.shape[0], hkv, d)
        v_new = inputs.v_new.reshape(q.shape[0], hkv, d)
    rope = inputs.cos is not None and inputs.sin is not None
    cs = _rope_in_kernel(inputs) if rope else None
    if (kb.dtype in (torch.bfloat16, torch.float16) and d % 8 == 0 and bs % 16 == 0 and q.dtype == kb.dtype
            and not (rope and cs is None)):
        if rope and append:
            return _C.full_attention_decode_paged(q.contiguous(), kb, vb, table.to(torch.int32).contiguous(), seq,
                                                  float(scale), k_new.to(kb.dtype).contiguous(),
                                                  v_new.to(kb.dtype).contiguous(), cos_sin=cs,
                                                  rotary_dim=int(inputs.rotary_dim))
        if rope:
            return _C.full_attention_decode_paged(q.contiguous(), kb.contiguous(), vb.contiguous(),
                                                  table.to(torch.int32).contiguous(), seq, float(scale),
                                                  cos_sin=cs, rotary_dim=int(inputs.rotary_dim))
        if append:
            return _C.full_attention_decode_paged(q.contiguous(), kb, vb, table.to(torch.int32).contiguous(), seq,
                                                  float(scale), k_new.to(kb.dtype).contiguous(),
                                                  v_new.to(kb.dtype).contiguous())
        return _C.full_attention_decode_paged(q.contiguous(), kb.contiguous(), vb.contiguous(),
                                              table.to(torch.int32).contiguous(), seq, float(scale))
    if append:  # write the new row into its block first (ids outside the pool are skipped)
        blk = table[:, (seq - 1) // bs].long()
        ok = (blk >= 0) & (blk < nblocks)
        kb[blk[ok], (seq - 1) % bs] = k_new[ok].to(kb.dtype)
        vb[blk[ok], (seq - 1) % bs] = v_new[ok].to(vb.dtype)
    # Gather the blocks that hold the seq_len tokens; ids outside the pool
    # read as zeros, as in the kernel (never an out-of-range index).
    idx = table[:, : (seq + bs - 1) // bs].long()
    valid = ((idx >= 0) & (idx < nblocks))[..., None, None, None]
    safe = idx.clamp(0, nblocks - 1)
    k = torch.where(valid, kb[safe], torch.zeros((), dtype=kb.dtype, device=kb.device))
    v = torch.where(valid, vb[safe], torch.zeros((), dtype=vb.dtype, device=vb.device))
    k = k.reshape(q.shape[0], -1, hkv, d)[:, :seq]
    v = v.reshape(q.shape[0], -1, hkv, d)[:, :seq]
    return full_attention_decode(dataclasses.replace(inputs, k_cache=k, v_cache=v, block_table=None,
                                                     seq_len=None, scale=scale, k_new=None, v_new=None,
                                                     cache_seqlen=None))


def full_attention_decode(inputs: FullAttentionInputs) -> torch.Tensor:
    """One-token GQA attention over a contiguous KV cache (split-K flash-decode, HIP).

    With cos/sin, the reference rotates q and the whole k_cache before its
    kernel (ops.py:368).  Here, where the kernel supports it, q and the keys
    are rotated inside the kernel as the keys stream, with the same rounding;
    otherwise both are rotated first, as the reference does.  Device-resident
    cos/sin avoid a host-to-device copy per call.  With k_new/v_new the new
    token is appended to the caches first (see _attention_append)."""
    if inputs.block_table is not None:
        return _attention_paged(inputs)
    if inputs.k_new is not None or inputs.v_new is not None:
        return _attention_append(inputs)
    cs = _rope_in_kernel(inputs)
    if cs is not None:
        q, k_cache = inputs.q, inputs.k_cache  # both rotated inside the kernel
    else:
        q, k_cache = apply_partial_rope(inputs.q, inputs.k_cache, inputs.cos, inputs.sin, inputs.rotary_dim)
    scale = inputs.scale
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if q.shape[1] % k_cache.shape[2] != 0:
        raise ValueError("query_heads must be divisible by kv_heads")
    _require_extension("full_attention_decode", q, k_cache, inputs.v_cache)
    if cs is not None:
        return _C.full_attention_decode_rope(q.contiguous(), k_cache.contiguous(), inputs.v_cache.contiguous(),
                                             float(scale), cs, int(inputs.rotary_dim))
    return _C.full_attention_decode(q.contiguous(), k_cache.contiguous(), inputs.v_cache.contiguous(), float(scale))


def causal_conv1d_update(
    x: torch.Tensor,
    conv_state: torch.Tensor,
    weight: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    activation: Optional[str] = "silu",
) -> torch.Tensor:
    """One token through the depthwise causal convolution in front of the
    Qwen3.6 linear-attention recurrence (the model's causal_conv1d_update,
    kernel width 4): x [batch, channels] (or [batch, channels, 1]),
    conv_state [batch, channels, width - 1] updated in place, weight
    [channels, width] (or [channels, 1, width]).  Returns act(conv) shaped like
    x.  No counterpart in the reference."""
    if activation not in (None, "silu", "swish"):
        raise ValueError(f"unsupported activation: {activation}")
    _require_extension("causal_conv1d_update", x, conv_state, weight)
    if not conv_state.is_contiguous():
        raise ValueError("conv_state must be contiguous: it is updated in place")
    w = weight.reshape(weight.shape[0], weight.shape[-1]).contiguous()
    out = _C.causal_conv1d_update(x.reshape(x.shape[0], -1).contiguous(), conv_state, w,
                                  None if bias is None else bias.contiguous(), activation is not None)
    return out.reshape(x.shape)


def gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """weight * rms_norm(x) * silu(gate) over the last dimension, norm before
    gate, with the roundings of the model's RMSNormGated: the normalised x
    and the weighted value are rounded to x's dtype, the mean and rsqrt are
    FP32.  The output norm of the Qwen3.6 linear-attention step.  No
    counterpart in the reference."""
    _require_extension("gated_rms_norm", x, gate, weight)
    return _C.gated_rms_norm(x.contiguous(), gate.contiguous(), weight.contiguous(), float(eps))


def linear_attention_step(
    x_mixed: torch.Tensor,
    conv_state: torch.Tensor,
    conv_weight: torch.Tensor,
    state: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    z: torch.Tensor,
    norm_weight: torch.Tensor,
    *,
    k_heads: int,
    conv_bias: Optional[torch.Tensor] = None,
    q_scale: Optional[float] = None,
    eps: float = 1e-6,
) -> torch.Tensor:
    """One Qwen3.6 linear-attention decode step from the projected q/k/v row
    to the gated-norm output, in one launch: causal conv update of x_mixed
    [batch, 2*k_heads*Dk + Hv*Dv] (conv_state updated in place), the gated
    delta rule with q/k L2 norm on the conv output (state [batch, Hv, Dk, Dv]
    FP32 updated in place), and the gated RMS norm with z [batch, Hv, Dv].
    Bit-identical to causal_conv1d_update, linear_attention_decode and
    gated_rms_norm called in sequence.  Returns out [batch, Hv, Dv].  No
    counterpart in the reference."""
    _require_extension("linear_attention_step", x_mixed, conv_state, conv_weight, state, g, beta, z, norm_weight)
    for name, t in (("conv_state", conv_state), ("state", state)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous: it is updated in place")
    dk = state.shape[2]
    scale = q_scale if q_scale is not None else 1.0 / math.sqrt(dk)
    w = conv_weight.reshape(conv_weight.shape[0], conv_weight.shape[-1]).contiguous()
    return _C.linear_attention_step(x_mixed.contiguous(), conv_state, w,
                                    None if conv_bias is None else conv_bias.contiguous(), state,
                                    g.float().contiguous(), beta.float().contiguous(), z.contiguous(),
                                    norm_weight.contiguous(), int(k_heads), float(scale), float(eps))


def linear_attention_decode(inputs: LinearAttentionInputs) -> tuple[torch.Tensor, torch.Tensor]:
    """One recurrent step.  Returns ``(out, new_state)``; the input state is not modified.

    Without ``g``/``beta``: the reference rule ``S' = decay*S + k v^T``, ``o = q^T S'``.
    With them: the gated delta rule (v head j reads q/k head ``j // (Hv // Hk)``);
    ``qk_l2norm`` L2-normalises q and k inside the kernel and scales q.
    """
    if (inputs.g is None) != (inputs.beta is None):
        raise ValueError("g and beta must be given together")
    if inputs.qk_l2norm and inputs.g is None:
        raise ValueError("qk_l2norm needs the gated delta rule (g and beta)")
    tensors = (inputs.q, inputs.k, inputs.v, inputs.state)
    if inputs.g is not None:
        _require_extension("linear_attention_decode", *tensors, inputs.g, inputs.beta)
        q_scale = inputs.q_scale if inputs.q_scale is not None else 1.0 / math.sqrt(inputs.q.shape[-1])
        return _C.gated_delta_decode(
            inputs.q.contiguous(),
            inputs.k.contiguous(),
            inputs.v.contiguous(),
            inputs.state.contiguous(),
            inputs.g.float().contiguous(),
            inputs.beta.float().contiguous(),
            qk_l2norm=bool(inputs.qk_l2norm),
            q_scale=float(q_scale),
        )
    _require_extension("linear_attention_decode", *tensors)
    return _C.linear_attention_decode(
        inputs.q.contiguous(),
        inputs.k.contiguous(),
        inputs.v.contiguous(),
        inputs.state.contiguous(),
        float(inputs.decay),
    )


def _project_add(
    out: torch.Tensor, out_proj: Optional[torch.Tensor], hidden: torch.Tensor
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(y, hidden + y) for the mixer output y (reference ops.py:721-723,
    727-729).  Without out_proj, y is the output reshaped onto the hidden size
    as in the reference.  With it, y = out @ out_proj^T and the residual add
    runs in the GEMV's epilogue: y is rounded first, then added, the same two
    roundings as the separate add."""
    if out_proj is None:
        y = out.reshape_as(hidden)
        return y, hidden + y
    _require_extension("decode_layer out_proj", out, out_proj)
    x2 = out.reshape(out.shape[0], -1).contiguous()
    if hidden.dtype != out.dtype:
        y = _C.gemv(x2, out_proj.contiguous(), None)
        return y, hidden + y
    y, summed = _C.gemv_add(x2, out_proj.contiguous(), hidden.reshape(x2.shape[0], -1).contiguous())
    return y, summed.reshape_as(hidden)


def _project_inputs(hidden: torch.Tensor, norm: torch.Tensor, proj: torch.Tensor, eps: float) -> torch.Tensor:
    """rms_norm(hidden, norm) @ proj^T in one launch (mkq_rms_norm_gemv)."""
    _require_extension("decode_layer input projection", hidden, norm, proj)
    x2 = hidden.reshape(hidden.shape[0], -1).contiguous()
    return _C.rms_norm_gemv(x2, norm.contiguous(), proj.contiguous(), eps)


def _cut(t: torch.Tensor, lo: int, hi: int, *shape: int) -> torch.Tensor:
    return t[:, lo:hi].reshape(t.shape[0], *shape).contiguous()


def _with_projected_qkv(inp: FullAttentionInputs, hidden: torch.Tensor, eps: float) -> FullAttentionInputs:
    kv_heads, head_dim = inp.k_cache.shape[-2], inp.k_cache.shape[-1]
    qkv = _project_inputs(hidden, inp.input_norm, inp.qkv_proj, eps)
    qd = qkv.shape[1] - 2 * kv_heads * head_dim
    if qd <= 0 or qd % head_dim:
        raise ValueError("qkv_proj must have (q_heads + 2 * kv_heads) * head_dim rows")
    kd = kv_heads * head_dim
    return dataclasses.replace(inp, q=_cut(qkv, 0, qd, qd // head_dim, head_dim),
                               k_new=_cut(qkv, qd, qd + kd, kv_heads, head_dim),
                               v_new=_cut(qkv, qd + kd, qd + 2 * kd, kv_heads, head_dim))


def _with_projected_qkv_linear(inp: LinearAttentionInputs, hidden: torch.Tensor, eps: float) -> LinearAttentionInputs:
    _, v_heads, key_dim, value_dim = inp.state.shape
    qkv = _project_inputs(hidden, inp.input_norm, inp.in_proj, eps)
    kd = qkv.shape[1] - v_heads * value_dim
    if kd <= 0 or kd % (2 * key_dim):
        raise ValueError("in_proj must have 2 * k_heads * key_dim + v_heads * value_dim rows")
    k_heads = kd // (2 * key_dim)
    return dataclasses.replace(inp, q=_cut(qkv, 0, kd // 2, k_heads, key_dim),
                               k=_cut(qkv, kd // 2, kd, k_heads, key_dim),
                               v=_cut(qkv, kd, qkv.shape[1], v_heads, value_dim))


def decode_layer(
    layer_idx: int,
    hidden: torch.Tensor,
    moe: Optional[MoeWeights] = None,
    *,
    dense_ffn: Optional[DenseFfnWeights] = None,
    full_attention: Optional[FullAttentionInputs] = None,
    linear_attention: Optional[LinearAttentionInputs] = None,
    layer_type: Optional[str] = None,
    eps: float = 1e-6,
    top_k: int = 8,
) -> DecodeLayerResult:
    """One decoder layer step (reference ops.py:701-748): attention or linear
    attention plus residual, then dense FFN or MoE with the residual inside."""
    kind = layer_type or qwen36_layer_type(layer_idx)
    attention_output = None
    linear_output = None
    linear_state = None
    residual = hidden

    if kind == "full_attention":
        if full_attention is None:
            raise ValueError("full_attention inputs are required for full_attention layers")
        if full_attention.qkv_proj is not None:
            full_attention = _with_projected_qkv(full_attention, hidden, eps)
        attention_output, residual = _project_add(full_attention_decode(full_attention), full_attention.out_proj, hidden)
    elif kind == "linear_attention":
        if linear_attention is None:
            raise ValueError("linear_attention inputs are required for linear_attention layers")
        if linear_attention.in_proj is not None:
            linear_attention = _with_projected_qkv_linear(linear_attention, hidden, eps)
        linear_output, linear_state = linear_attention_decode(linear_attention)
        linear_output, residual = _project_add(linear_output, linear_attention.out_proj, hidden)
    else:
        raise ValueError(f"unsupported layer_type: {kind}")

    if dense_ffn is not None:
        out = dense_ffn_decode(residual, dense_ffn, eps=eps, add_residual=True)
        router_indices = None
        router_weights = None
    else:
        if moe is None:
            raise ValueError("either moe or dense_ffn weights are required")
        out, router_indices, router_weights = moe_decode(residual, moe, eps=eps, top_k=top_k, add_residual=True)
    return DecodeLayerResult(
        hidden=out,
        router_indices=router_indices,
        router_weights=router_weights,
        attention_output=attention_output,
        linear_output=linear_output,
        linear_state=linear_state,
    )
