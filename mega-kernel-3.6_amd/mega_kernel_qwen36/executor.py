"""Runs linearized decode plans (``mpk_graph.CompiledPlan``) on the HIP kernels.

The reference builds these plans but has no runtime that executes them
(mega_kernel_qwen36/mpk_graph.py:178-276 plans; nothing consumes the launch
steps).  Here a plan is compiled once into a list of launches, in launch-step
order, with each layer's task runs fused into the kernels that cover them:

    rmsnorm + linear(qkv)                  -> mkq_rms_norm_gemv (q, k_new, v_new)
    paged_attention                        -> attention with the KV append (contiguous or paged cache)
    linear_residual (attention output)     -> mkq_gemv_add (out_proj + residual)
    rmsnorm + linear_attention             -> mkq_rms_norm_gemv (q, k, v), gated delta rule, mkq_gemv_add
    rmsnorm + moe_router + moe_grouped_experts + linear_residual
                                           -> one persistent MoE launch (norm, routing, experts, shared
                                              expert, down projection and residual)
    rmsnorm + dense_gate_up + dense_down   -> the dense SwiGLU FFN (two launches)

``metadata`` and ``embed`` tasks are the caller's: hidden_0 and the cache
positions / block tables arrive with the inputs.  ``final_norm``,
``lm_head`` and ``argmax`` are not part of the decode hot path; they are
reported as not executed.  ``capture()`` records the whole plan into one
HIP graph, so a decode step replays with one launch.
"""

from __future__ import annotations

import dataclasses
import re
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import torch

from . import ops
from .mpk_graph import CompiledPlan

_LAYER_TASK = re.compile(r"^layer_(\d+)_(.+)$")
_CALLER_KINDS = ("metadata", "embed")
_NOT_RUN = ("final_norm", "lm_head", "argmax_or_sampler")

# The task runs of one layer, in launch order, and the launch group each
# belongs to (suffixes of the planner's task ids).
_GROUPS = {
    "full_attention": (("attn_norm", "qkv_proj"), ("paged_attention",), ("attn_out_proj_residual",)),
    "linear_attention": (("attn_norm", "linear_attention_recurrent"),),
    "moe": (("ffn_norm", "moe_router_topk", "moe_grouped_experts", "moe_down_residual"),),
    "dense": (("ffn_norm", "dense_gate_up", "dense_down_residual"),),
}


@dataclass
class DecodeLayerWeights:
    """One layer's weights and mixer state for a plan.  ``input_norm`` is the
    layer's attention RMSNorm; the mixer inputs carry the projections
    (``qkv_proj`` / ``in_proj``, ``out_proj``) and the cache or recurrent
    state; ``moe.norm_weight`` / ``dense_ffn.norm_weight`` is the FFN norm."""

    input_norm: torch.Tensor
    full_attention: Optional[ops.FullAttentionInputs] = None
    linear_attention: Optional[ops.LinearAttentionInputs] = None
    moe: Optional[ops.MoeWeights] = None
    dense_ffn: Optional[ops.DenseFfnWeights] = None


@dataclass
class DecodeStepResult:
    hidden: torch.Tensor                      # hidden_L, the input of final_norm
    router_indices: List[Optional[torch.Tensor]]
    router_weights: List[Optional[torch.Tensor]]
    linear_states: List[Optional[torch.Tensor]]
    not_executed: Tuple[str, ...]


class DecodePlanExecutor:
    def __init__(self, plan: CompiledPlan, layers: Sequence[DecodeLayerWeights], *, eps: float = 1e-6,
                 top_k: int = 8):
        self.plan = plan
        self.layers = list(layers)
        self.eps = eps
        self.top_k = top_k
        tasks = {t.id: t for t in plan.graph.tasks}
        order = [s.task_id for s in plan.launch_steps]
        seen = set()
        for tid in order:  # launch order must respect every dependency
            missing = [d for d in tasks[tid].depends_on if d not in seen]
            if missing:
                raise ValueError(f"plan launches {tid} before its dependencies {missing}")
            seen.add(tid)
        self.not_executed = tuple(t for t in order if t in _NOT_RUN)
        self._steps: List[Tuple[int, str]] = []  # (layer, group name) in launch order
        pos = 0
        layer_ids = []
        while pos < len(order):
            tid = order[pos]
            kind = tasks[tid].kind
            if kind in _CALLER_KINDS or tid in _NOT_RUN:
                pos += 1
                continue
            m = _LAYER_TASK.match(tid)
            if m is None:
                raise ValueError(f"task {tid} ({kind}) has no HIP launch in this executor")
            layer = int(m.group(1))
            if layer >= len(self.layers):
                raise ValueError(f"plan has layer {layer}, weights for {len(self.layers)} layers were given")
            w = self.layers[layer]
            family = None
            for fam, groups in _GROUPS.items():
                for grp in groups:
                    if order[pos:pos + len(grp)] == [f"layer_{layer}_{s}" for s in grp]:
                        family, group = fam, grp
                        break
                if family:
                    break
            if family is None:
                raise ValueError(f"unexpected task run at {tid} ({kind})")
            need = {"full_attention": w.full_attention, "linear_attention": w.linear_attention,
                    "moe": w.moe, "dense": w.dense_ffn}[family]
            if need is None:
                raise ValueError(f"layer {layer}: the plan has a {family} part but its weights were not given")
            if family == "full_attention" and w.full_attention.qkv_proj is None:
                raise ValueError(f"layer {layer}: full_attention needs qkv_proj for the plan's qkv_proj task")
            if family == "linear_attention" and w.linear_attention.in_proj is None:
                raise ValueError(f"layer {layer}: linear_attention needs in_proj for the plan's input projection")
            self._steps.append((layer, group[0] if family in ("full_attention",) else family))
            if layer not in layer_ids:
                layer_ids.append(layer)
            pos += len(group)
        self.layer_ids = tuple(layer_ids)
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._static_in: Optional[torch.Tensor] = None
        self._static_out: Optional[DecodeStepResult] = None

    # -- one decode step -------------------------------------------------
    def run(self, hidden: torch.Tensor) -> DecodeStepResult:
        n = len(self.layers)
        idx: List[Optional[torch.Tensor]] = [None] * n
        wts: List[Optional[torch.Tensor]] = [None] * n
        states: List[Optional[torch.Tensor]] = [None] * n
        h = hidden
        attn: Optional[ops.FullAttentionInputs] = None
        attn_out: Optional[torch.Tensor] = None
        resid = h
        for layer, group in self._steps:
            w = self.layers[layer]
            if group == "attn_norm":  # rmsnorm + qkv projection: q, k_new, v_new
                fa = dataclasses.replace(w.full_attention, input_norm=w.input_norm)
                attn = ops._with_projected_qkv(fa, h, self.eps)
            elif group == "paged_attention":
                attn_out = ops.full_attention_decode(attn)
            elif group == "attn_out_proj_residual":
                _, resid = ops._project_add(attn_out, attn.out_proj, h)
            elif group == "linear_attention":
                la = dataclasses.replace(w.linear_attention, input_norm=w.input_norm)
                la = ops._with_projected_qkv_linear(la, h, self.eps)
                out, states[layer] = ops.linear_attention_decode(la)
                _, resid = ops._project_add(out, la.out_proj, h)
            elif group == "moe":
                h, idx[layer], wts[layer] = ops.moe_decode(resid, w.moe, eps=self.eps, top_k=self.top_k,
                                                           add_residual=True)
            else:  # dense
                h = ops.dense_ffn_decode(resid, w.dense_ffn, eps=self.eps, add_residual=True)
        return DecodeStepResult(hidden=h, router_indices=idx, router_weights=wts, linear_states=states,
                                not_executed=self.not_executed)

    # -- the whole plan as one HIP graph ---------------------------------
    def capture(self, hidden: torch.Tensor) -> None:
        """Records run() into a HIP graph whose input is a copy of `hidden`'s
        storage; replay(h) copies h in and replays.  The graph keeps its own
        output tensors (returned by replay)."""
        self._static_in = hidden.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.run(self._static_in)  # creates the per-stream workspaces before capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self._graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph, stream=s):
            self._static_out = self.run(self._static_in)
        torch.cuda.synchronize()

    def replay(self, hidden: Optional[torch.Tensor] = None) -> DecodeStepResult:
        if self._graph is None:
            raise RuntimeError("capture() first")
        if hidden is not None:
            self._static_in.copy_(hidden)
        self._graph.replay()
        return self._static_out

    def launch_groups(self) -> Tuple[Tuple[int, str], ...]:
        """(layer, launch group) in the order run() issues them."""
        return tuple(self._steps)
